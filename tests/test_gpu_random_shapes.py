"""Seeded random shapes through the C ABI against the CPU oracle.

Hand-picked shapes sit on or beside tile edges by intent; these do not. Each
case draws M, K and N at random (fixed seeds) in a range that sends the
library down one of its own dispatch choices: the skinny kernel that
quantizes its few rows itself, the 128x128 persistent kernel, split-K for
long K on a small grid, and the 256x256 kernel with its 128x128 tail on a
large grid. The epilogue form cycles through bias-free, bias, gated residual
(fma and separate multiply-add), plain residual, GELU and raw int32
accumulators, and every third case places A, Y and the residual 4 bytes off
16-byte alignment (the scalar load/store paths). Bit-exact against the
oracle (qgemm.cpp:73-142 plus the consumers), GELU within 1e-6 (1 + |y|).
"""
import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu

KINDS = ["none", "bias", "gated", "gated_sep", "resid", "gelu", "acc"]


def _cases():
    out = []
    for i in range(16):  # general: 1-800 rows, K up to 4700, N up to 1300
        r = np.random.default_rng(7100 + i)
        M = int(r.integers(1, 65)) if i % 4 == 0 else int(r.integers(65, 801))
        out.append(("general", i, M, int(r.integers(1, 4701)), int(r.integers(1, 1301))))
    for i in range(4):  # long K on a small grid: split-K (which needs N % 4 == 0)
        r = np.random.default_rng(7200 + i)
        out.append(("splitk", 16 + i, int(r.integers(65, 401)), int(r.integers(6144, 9001)),
                    4 * int(r.integers(16, 376))))
    for i in range(2):  # a grid of >= 2 rounds of 256x256 tiles: 256x256 plus its tail
        r = np.random.default_rng(7300 + i)
        out.append(("large", 20 + i, int(r.integers(2600, 2900)), int(r.integers(128, 401)),
                    int(r.integers(12800, 13300))))
    for i in range(2):  # at most 4 rows: the skinny kernel quantizes them itself
        r = np.random.default_rng(7400 + i)
        out.append(("tiny", 22 + i, int(r.integers(1, 5)), int(r.integers(1, 3073)),
                    int(r.integers(1, 4097))))
    return out


def _device_view(torch, dev, host, misalign):
    """host array on the device; with misalign, 4 bytes past a 16-byte boundary."""
    flat = torch.from_numpy(np.ascontiguousarray(host).ravel()).to(dev)
    if not misalign:
        return flat.view(host.shape)
    buf = torch.zeros(flat.numel() + 1, dtype=flat.dtype, device=dev)
    buf[1:] = flat
    return buf[1:].view(host.shape)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}{c[1]}-{c[2]}x{c[3]}x{c[4]}")
def test_random_shape_bitexact(sdq_dev, oracle, case):
    import torch

    import sdq

    what, i, M, K, N = case
    kind = KINDS[i % len(KINDS)]
    misalign = i % 3 == 2
    A = oracle.randn(M * K, 8000 + i).reshape(M, K)
    W = oracle.randn(N * K, 8100 + i).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    bias = oracle.randn(N, 8200 + i) * np.float32(0.01)
    gate = oracle.randn(N, 8300 + i)
    x = oracle.randn(M * N, 8400 + i).reshape(M, N)
    w = sdq.Weight.from_host(q, s)
    epi = {"gated_sep": "gated", "bias": "none"}.get(kind, kind)
    plan = [p[0] for p in sdq.qlinear_plan(w, M, epi)]
    print(f"[random] {what}{i} M={M} K={K} N={N} kind={kind} misalign={misalign} plan={plan}",
          flush=True)
    A_d = _device_view(torch, sdq_dev, A, misalign)
    out_dtype = np.int32 if kind == "acc" else np.float32
    Y_d = _device_view(torch, sdq_dev, np.full((M, N), -7, out_dtype), misalign)
    b_d = None if kind in ("none", "acc") else torch.from_numpy(bias).to(sdq_dev)
    g_d = torch.from_numpy(gate).to(sdq_dev) if kind.startswith("gated") else None
    r_d = _device_view(torch, sdq_dev, x, misalign) if kind in ("gated", "gated_sep", "resid") \
        else None
    sdq.qlinear(w, A_d, Y_d, kind=epi, bias=b_d, gate=g_d, resid=r_d,
                gate_fma=(kind != "gated_sep"))
    torch.cuda.synchronize()
    got = Y_d.cpu().numpy()
    if kind == "acc":
        aq, _ = oracle.act_quant(A)
        assert_bitexact(got, oracle.qgemm_acc(aq, q), f"{what}{i} acc")
        return
    want = oracle.linear(A, q, s, bias=None if kind == "none" else bias,
                         epilogue={"bias": "none", "gated_sep": "gated"}.get(kind, kind),
                         gate=gate, resid=x, use_fma=(kind != "gated_sep"))
    if kind == "gelu":
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        assert np.all(err <= 1e-6 * (1.0 + np.abs(want))), float(err.max())
    else:
        assert_bitexact(got, want, f"{what}{i} {kind}")
