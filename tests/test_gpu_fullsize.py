"""Full-size parity of the persistent GEMM on the north-star shapes.

At these sizes every workgroup walks several tiles, so the cross-tile LDS
pipeline is exercised; the small-shape tests do not reach it. Checks:
bit-exact against the oracle at ~10^6 random output positions plus every
column of selected rows, and bitwise run-to-run determinism of the whole
output (a race shows up as a few differing elements between two runs)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (M, K, N, epilogue): DiT FFN up-projection with bias (the bench workload)
# and FFN down-projection with the gated residual (ovi_dit.cpp:217-221).
CASES = [(27280, 3072, 14336, "none"), (27280, 14336, 3072, "gated")]


def _positions(M, N, K, seed):
    rng = np.random.default_rng(seed)
    count = int(min(1 << 20, 3e9 // K))
    ms = rng.integers(0, M, count)
    ns = rng.integers(0, N, count)
    rows = np.array([0, 100, 255, 256 + 13, M // 2, M - 1], np.int64)
    ms = np.concatenate([ms, np.repeat(rows, N)])
    ns = np.concatenate([ns, np.tile(np.arange(N), rows.size)])
    return ms.astype(np.int64), ns.astype(np.int64)


@pytest.mark.parametrize("M,K,N,epi", CASES)
def test_fullsize_spot_checks_and_determinism(sdq_dev, oracle, M, K, N, epi):
    import torch

    import sdq

    print(f"[fullsize] M={M} K={K} N={N} epilogue={epi}", flush=True)
    A = oracle.randn(M * K, 900 + K).reshape(M, K)
    W = oracle.randn(N * K, 901 + K).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    del W
    bias = oracle.randn(N, 902) * np.float32(0.01)
    gate = oracle.randn(N, 903) if epi == "gated" else None
    resid = oracle.randn(M * N, 904).reshape(M, N) if epi == "gated" else None

    w = sdq.Weight.from_host(q, s)
    A_d = torch.from_numpy(A).to(sdq_dev)
    b_d = torch.from_numpy(bias).to(sdq_dev)
    g_d = None if gate is None else torch.from_numpy(gate).to(sdq_dev)
    r_d = None if resid is None else torch.from_numpy(resid).to(sdq_dev)
    outs = []
    for _ in range(2):
        Y = torch.full((M, N), -7.0, dtype=torch.float32, device=sdq_dev)
        sdq.qlinear(w, A_d, Y, kind=epi, bias=b_d, gate=g_d, resid=r_d)
        outs.append(Y)
    torch.cuda.synchronize()
    diff = (outs[0].view(torch.int32) != outs[1].view(torch.int32)).sum().item()
    assert diff == 0, f"{diff} outputs differ between two identical runs"

    ms, ns = _positions(M, N, K, 905)
    flat = torch.from_numpy(ms * N + ns).to(sdq_dev)
    got = outs[0].view(-1)[flat].cpu().numpy()
    aq, asc = oracle.act_quant(A)
    want = oracle.linear_at(aq, asc, q, s, ms, ns, bias, epi, gate, resid)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, (
        f"{bad.size} of {ms.size} spot checks differ, first at m={ms[bad[0]]} n={ns[bad[0]]}: "
        f"got {got[bad[0]]!r} want {want[bad[0]]!r}")


def _golden_hashes():
    import json
    import os

    from conftest import GOLDEN

    with open(os.path.join(GOLDEN, "fullsize_sha256.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["ns_27280x3072x14336", "ffn_down_27280x14336x3072",
                                  "cross_q_27280x3072x3072"])
def test_fullsize_whole_output_hash(sdq_dev, oracle, name):
    """Every one of the 391M outputs at the headline shapes, bit for bit: the
    SHA-256 of the GPU's qgemm output equals that of the reference's own
    sd::qgemm (src/core/qgemm.cpp, compiled in oracle/_ref) on the same seeded
    inputs, recorded by tests/golden/make_fullsize_hashes.py."""
    import hashlib

    import torch

    import sdq

    g = _golden_hashes()[name]
    M, K, N = g["M"], g["K"], g["N"]
    print(f"[fullsize-hash] {name}", flush=True)
    A = oracle.randn(M * K, g["seed_a"]).reshape(M, K)
    W = oracle.randn(N * K, g["seed_w"]).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    del W

    def sha(*arrays):
        h = hashlib.sha256()
        for a in arrays:
            h.update(np.ascontiguousarray(a).view(np.uint8).data)
        return h.hexdigest()

    assert sha(A) == g["sha256_A"], "regenerated activations differ from the recorded ones"
    assert sha(q, s) == g["sha256_W"], "regenerated weights differ from the recorded ones"
    w = sdq.Weight.from_host(q, s)
    A_d = torch.from_numpy(A).to(sdq_dev)
    del A
    Y = torch.full((M, N), -7.0, dtype=torch.float32, device=sdq_dev)
    sdq.qgemm(w, A_d, Y)
    torch.cuda.synchronize()
    got = sha(Y.cpu().numpy())
    w.free()
    assert got == g["sha256_out"], f"{name}: whole-output SHA-256 differs from the reference's"
