"""GPU parity of the HIP path (through the C ABI) against the CPU oracle:
bit-exact quantized activations, int32 accumulators and fp32 outputs."""
import os

import ctypes

import numpy as np
import pytest

from conftest import GOLDEN, assert_bitexact

pytestmark = pytest.mark.gpu


def _inputs(M, K, N, seed):
    import pyoracle

    A = pyoracle.randn(M * K, seed).reshape(M, K)
    W = pyoracle.randn(N * K, seed + 1).reshape(N, K) * np.float32(0.02)
    q, s = pyoracle.quant_rows(W)
    bias = pyoracle.randn(N, seed + 2) * np.float32(0.01)
    return A, q, s, bias


def _run(sdq_dev, w, A, kind="none", bias=None, gate=None, resid=None, gate_fma=True):
    import torch

    import sdq

    M = A.shape[0]
    dt = torch.int32 if kind == "acc" else torch.float32
    A_d = torch.from_numpy(np.ascontiguousarray(A)).to(sdq_dev)
    Y = torch.full((M, w.N), -7, dtype=dt, device=sdq_dev)
    b_d = None if bias is None else torch.from_numpy(bias).to(sdq_dev)
    g_d = None if gate is None else torch.from_numpy(gate).to(sdq_dev)
    r_d = None if resid is None else torch.from_numpy(np.ascontiguousarray(resid)).to(sdq_dev)
    sdq.qlinear(w, A_d, Y, kind=kind, bias=b_d, gate=g_d, resid=r_d, gate_fma=gate_fma)
    torch.cuda.synchronize()
    return Y.cpu().numpy()


# --------------------------------------------------------------- quantizer
@pytest.mark.parametrize("M,K", [(1, 31), (17, 64), (37, 320), (256, 3072), (5, 14336),
                                 (33, 4160), (3, 1), (20, 100)])
def test_act_quant_bitexact(sdq_dev, oracle, M, K):
    import torch

    import sdq

    rng = np.random.default_rng(M * 1000 + K)
    A = (rng.standard_normal((M, K)) * rng.uniform(1e-3, 1e3, (M, 1))).astype(np.float32)
    A_d = torch.from_numpy(A).to(sdq_dev)
    aq = torch.zeros((M, K), dtype=torch.int8, device=sdq_dev)
    asc = torch.zeros((M,), dtype=torch.float32, device=sdq_dev)
    sdq.act_quant(A_d, aq, asc)
    torch.cuda.synchronize()
    want_q, want_s = oracle.act_quant(A)
    assert_bitexact(asc.cpu().numpy(), want_s, "as")
    assert_bitexact(aq.cpu().numpy(), want_q, "aq")


def test_act_quant_special_rows(sdq_dev, oracle):
    import torch

    import sdq

    g = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    A = g["special_a"]
    M, K = A.shape
    A_d = torch.from_numpy(A).to(sdq_dev)
    aq = torch.zeros((M, K), dtype=torch.int8, device=sdq_dev)
    asc = torch.zeros((M,), dtype=torch.float32, device=sdq_dev)
    sdq.act_quant(A_d, aq, asc)
    torch.cuda.synchronize()
    want_q, want_s = oracle.act_quant(A)
    assert_bitexact(asc.cpu().numpy(), want_s, "as")
    assert_bitexact(aq.cpu().numpy(), want_q, "aq")


# ------------------------------------------------------------ weight repack
@pytest.mark.parametrize("N,K", [(13, 31), (256, 3072), (300, 257), (18432, 64)])
def test_weight_repack_roundtrip(sdq_dev, N, K):
    import sdq

    rng = np.random.default_rng(N + K)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    # scales at an odd byte offset, as in a .sdcpp blob with no padding
    raw = bytearray(b"\x00" + s.tobytes())
    w = sdq.Weight.from_host(q, memoryview(raw)[1:])
    q2, s2 = w.export()
    assert_bitexact(q2, q, "q")
    assert_bitexact(s2, s, "scale")


# ------------------------------------------------------------------- qgemm
SHAPES = [
    (1, 3072, 18432),    # AdaLN time_projection (skinny, M=1)
    (1, 256, 3072),      # time_embedding.0
    (3, 31, 13),         # tiny, K and N not multiples of anything
    (17, 31, 13),        # tests/test_core.cpp shape
    (20, 3072, 3072),    # skinny16..32
    (64, 1024, 512),     # tests/test_core.cpp shape, skinny64
    (65, 4096, 3072),    # text_embedding.0 K, first tiled size
    (157, 3072, 3072),   # audio branch tokens
    (192, 3072, 14336),  # video tokens at 256x256/9 frames, FFN up
    (256, 3072, 3072),   # BASELINE cfg1
    (300, 257, 129),     # ragged everything
    (512, 3072, 3072),   # cross-attn K/V on ctx[512]
    (512, 4096, 3072),   # cfg4 text_embedding.0 on the whole [512, 4096] UMT5 context
    (768, 14336, 3072),  # cfg2 FFN down
    (70, 4200, 300),     # long rows, last 32-fragment group of the quantizer partial
    (33, 16384, 64),     # the longest row the single-pass quantizer keeps in registers
    (40, 20000, 96),     # longer rows: the quantizer's re-read loop
]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_qgemm_bitexact(sdq_dev, oracle, M, K, N):
    import sdq

    A, q, s, bias = _inputs(M, K, N, seed=M + 3 * K + 7 * N)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A)
    assert_bitexact(got, oracle.qgemm(A, q, s), f"qgemm {M}x{K}x{N}")
    got_b = _run(sdq_dev, w, A, bias=bias)
    assert_bitexact(got_b, oracle.linear(A, q, s, bias=bias), f"mlin {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(9, 200, 77), (130, 3072, 1000), (700, 512, 4096)])
def test_accumulators_bitexact(sdq_dev, oracle, M, K, N):
    import sdq

    A, q, s, _ = _inputs(M, K, N, seed=5 * M + K)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A, kind="acc")
    aq, _ = oracle.act_quant(A)
    assert_bitexact(got, oracle.qgemm_acc(aq, q), "int32 acc")


def test_golden_vectors_on_gpu(sdq_dev, oracle):
    """The reference's golden qgemm inputs (gen_basic.py) and its compiled
    outputs on the test_core shapes and special rows."""
    import sdq

    g = np.load(os.path.join(GOLDEN, "basic_golden.npz"))
    w = sdq.Weight.from_host(g["qg_bq"], g["qg_bs"])
    got = _run(sdq_dev, w, g["qg_a"])
    assert_bitexact(got, oracle.qgemm(g["qg_a"], g["qg_bq"], g["qg_bs"]), "golden qg")
    a = got.astype(np.float64).ravel()
    b = g["qg_out"].astype(np.float64).ravel()
    assert a @ b / np.sqrt((a @ a) * (b @ b)) > 0.999
    r = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    for (M, K, N) in [(17, 31, 13), (64, 1024, 512)]:
        A = oracle.randu(M * K, 7 + M).reshape(M, K)
        W = oracle.randu(N * K, 13 + N).reshape(N, K)
        q, s = oracle.quantize_rowwise(W)
        w = sdq.Weight.from_host(q, s)
        assert_bitexact(_run(sdq_dev, w, A), r[f"core_{M}x{K}x{N}_out"], f"ref core {M}x{K}x{N}")
    w = sdq.Weight.from_host(r["special_bq"], r["special_bs"])
    assert_bitexact(_run(sdq_dev, w, r["special_a"]), r["special_out"], "ref special rows")


def test_cfg1_matches_reference_hash(sdq_dev, oracle):
    import hashlib

    import sdq

    r = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    M, K, N = 256, 3072, 3072
    A = oracle.randn(M * K, 1001).reshape(M, K)
    W = oracle.randn(N * K, 1002).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A)
    assert hashlib.sha256(got.tobytes()).digest() == r["cfg1_sha256"].tobytes()


def test_core_3072x5120x5120_matches_reference_hash(sdq_dev, oracle):
    """The reference's --bench shape (tests/test_core.cpp:165-174)."""
    import hashlib

    import sdq

    r = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    M, K, N = 3072, 5120, 5120
    A = oracle.randu(M * K, 7 + M).reshape(M, K)
    W = oracle.randu(N * K, 13 + N).reshape(N, K)
    q, s = oracle.quantize_rowwise(W)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A)
    assert hashlib.sha256(got.tobytes()).digest() == r["core_3072x5120x5120_sha256"].tobytes()


@pytest.mark.parametrize("M,K,N", [(300, 257, 129), (700, 3072, 1000), (513, 1024, 520)])
def test_256_tiles_forced_bitexact(sdq_dev, oracle, monkeypatch, M, K, N):
    """The 256x256 persistent kernel (chosen by itself only for large grids)
    forced onto ragged shapes, with every epilogue form: partial tiles in
    both dimensions, K not a multiple of the 64-byte k-step."""
    import sdq

    monkeypatch.setenv("SDQ_FORCE_CFG", "2")  # kCfg256x256
    monkeypatch.setenv("SDQ_NO_TAIL", "1")
    print(f"[256-forced] M={M} K={K} N={N}", flush=True)
    A, q, s, bias = _inputs(M, K, N, seed=11 * M + K + N)
    w = sdq.Weight.from_host(q, s)
    aq, _ = oracle.act_quant(A)
    assert_bitexact(_run(sdq_dev, w, A, kind="acc"), oracle.qgemm_acc(aq, q), "256 acc")
    assert_bitexact(_run(sdq_dev, w, A), oracle.qgemm(A, q, s), "256 qgemm")
    assert_bitexact(_run(sdq_dev, w, A, bias=bias), oracle.linear(A, q, s, bias=bias), "256 mlin")
    gate = oracle.randn(N, 96)
    x = oracle.randn(M * N, 95).reshape(M, N)
    got = _run(sdq_dev, w, A, kind="gated", bias=bias, gate=gate, resid=x)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x)
    assert_bitexact(got, want, "256 gated")
    got = _run(sdq_dev, w, A, kind="resid", bias=bias, resid=x)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias, epilogue="resid", resid=x), "256 resid")
    got = _run(sdq_dev, w, A, kind="gelu", bias=bias)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gelu")
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want))), float(err.max())


# ---------------------------------------------------------------- epilogues
@pytest.mark.parametrize("M,K,N", [(40, 3072, 3072), (300, 1024, 3072), (5, 14336, 3072)])
@pytest.mark.parametrize("fma", [True, False])
def test_gated_residual_bitexact(sdq_dev, oracle, M, K, N, fma):
    import sdq

    A, q, s, bias = _inputs(M, K, N, seed=M + K + N)
    gate = oracle.randn(N, 99)
    x = oracle.randn(M * N, 98).reshape(M, N)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A, kind="gated", bias=bias, gate=gate, resid=x, gate_fma=fma)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x, use_fma=fma)
    assert_bitexact(got, want, "gated")


@pytest.mark.parametrize("M,K,N", [(40, 3072, 3072), (300, 1024, 3072)])
def test_plain_residual_bitexact(sdq_dev, oracle, M, K, N):
    import sdq

    A, q, s, bias = _inputs(M, K, N, seed=2 * M + K)
    x = oracle.randn(M * N, 97).reshape(M, N)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A, kind="resid", bias=bias, resid=x)
    want = oracle.linear(A, q, s, bias=bias, epilogue="resid", resid=x)
    assert_bitexact(got, want, "resid")


def test_gated_residual_in_place(sdq_dev, oracle):
    """Y aliases resid: x <- fma(y, g, x) in place, as gated_add_inplace."""
    import torch

    import sdq

    M, K, N = 300, 3072, 3072
    A, q, s, bias = _inputs(M, K, N, seed=4242)
    gate = oracle.randn(N, 1)
    x = oracle.randn(M * N, 2).reshape(M, N)
    w = sdq.Weight.from_host(q, s)
    X = torch.from_numpy(x.copy()).to(sdq_dev)
    sdq.qlinear(w, torch.from_numpy(A).to(sdq_dev), X, kind="gated",
                bias=torch.from_numpy(bias).to(sdq_dev), gate=torch.from_numpy(gate).to(sdq_dev),
                resid=X)
    torch.cuda.synchronize()
    want = oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x)
    assert_bitexact(X.cpu().numpy(), want, "in-place gated")


@pytest.mark.parametrize("M,K,N", [(30, 3072, 14336), (200, 3072, 1000)])
def test_gelu_epilogue_tolerance(sdq_dev, oracle, M, K, N):
    """GELU runs as x / (1 + e^(-2u)) on the GPU's exp2 and reciprocal; the
    reference uses libm tanh, so this one is a tolerance check:
    max abs err <= 1e-6 * (1 + |y|)."""
    import sdq

    A, q, s, bias = _inputs(M, K, N, seed=M * 3 + N)
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A, kind="gelu", bias=bias)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gelu")
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want))), float(err.max())
    # the pre-activation is bit-exact, so the GELU input matches the oracle's
    pre = _run(sdq_dev, w, A, kind="none", bias=bias)
    assert_bitexact(pre, oracle.linear(A, q, s, bias=bias), "pre-gelu")


@pytest.mark.parametrize("M,K,N", [(40, 3072, 1024), (300, 1024, 1024)])
def test_gelu_epilogue_saturation(sdq_dev, oracle, M, K, N):
    """GELU inputs driven into both saturations by large biases (|b| up to
    1e6): within the tolerance of the reference's 0.5 x (1 + tanh(u)), with
    the same sign of zero where that underflows (x < 0: -0.0), and y = x for
    large x."""
    import sdq

    A, q, s, _ = _inputs(M, K, N, seed=4 * M + N)
    levels = np.array([-1e6, -30.0, -8.0, -3.0, -1.0, 0.0, 1.0, 3.0, 8.0, 30.0, 1e6], np.float32)
    bias = levels[np.arange(N) % levels.size]
    w = sdq.Weight.from_host(q, s)
    got = _run(sdq_dev, w, A, kind="gelu", bias=bias)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gelu")
    assert np.isfinite(got).all()
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want))), float(err.max())
    zero = want == 0
    assert np.array_equal(np.signbit(got[zero]), np.signbit(want[zero])), "sign of zero"
    big = bias >= 30.0
    pre = oracle.linear(A, q, s, bias=bias)
    assert_bitexact(got[:, big], pre[:, big], "GELU(x) = x for large x")


def test_k_zero_and_m_zero(sdq_dev, oracle):
    """K == 0 gives the reference's zero-filled out (+bias); M == 0 is a no-op."""
    import torch

    import sdq

    N = 40
    q = np.zeros((N, 0), np.int8)
    s = np.ones(N, np.float32)
    w = sdq.Weight.from_host(q, s)
    A = np.zeros((5, 0), np.float32)
    got = _run(sdq_dev, w, A)
    assert_bitexact(got, np.zeros((5, N), np.float32), "K=0")
    bias = oracle.randn(N, 3)
    got = _run(sdq_dev, w, A, bias=bias)
    assert_bitexact(got, np.broadcast_to(bias, (5, N)).astype(np.float32), "K=0 + bias")
    w2 = sdq.Weight.from_host(np.ones((8, 16), np.int8), np.ones(8, np.float32))
    Y = torch.full((0, 8), 1.0, device=sdq_dev)
    sdq.qlinear(w2, torch.zeros((0, 16), device=sdq_dev), Y)


def test_errors_are_reported(sdq_dev):
    import torch

    import sdq

    w = sdq.Weight.from_host(np.ones((8, 16), np.int8), np.ones(8, np.float32))
    A = torch.zeros((4, 15), device=sdq_dev)
    Y = torch.zeros((4, 8), device=sdq_dev)
    with pytest.raises(sdq.SdqError, match=r"A: shape \(4, 15\)"):
        sdq.qlinear(w, A, Y)
    # the C ABI's own check, without the binding in front of it
    e = sdq.make_epilogue()
    rc = sdq._lib.sdq_qlinear(w.h, ctypes.c_void_p(A.data_ptr()), 4, 15, ctypes.byref(e),
                              ctypes.c_void_p(Y.data_ptr()), None)
    assert rc == sdq.ERR_INVALID and b"K mismatch" in sdq._lib.sdq_last_error()
    with pytest.raises(sdq.SdqError, match="GATED"):
        sdq.qlinear(w, torch.zeros((4, 16), device=sdq_dev), Y, kind="gated")


def test_size_limits_are_refused(sdq_dev):
    """Shapes past the GEMM kernels' 32-bit offsets and tile counters are
    refused through the C ABI before anything is read, allocated or launched
    (the small buffers passed here are never touched)."""
    import torch

    import sdq

    lib = sdq._lib
    q, s = np.ones(64, np.int8), np.ones(16, np.float32)
    for N, K in ((2**20 + 1, 16), (4, 2**22 + 1)):
        out = ctypes.c_void_p()
        rc = lib.sdq_weight_upload(q.ctypes.data, s.ctypes.data, N, K, None, ctypes.byref(out))
        assert rc == sdq.ERR_INVALID and b"weight too large" in lib.sdq_last_error(), (N, K)
        assert not out.value
    w = sdq.Weight.from_host(np.ones((8, 16), np.int8), np.ones(8, np.float32))
    A = torch.zeros((4, 16), device=sdq_dev)
    Y = torch.zeros((4, 8), device=sdq_dev)
    e = sdq.make_epilogue()
    pa, py = ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(Y.data_ptr())
    rc = lib.sdq_qlinear(w.h, pa, 2**30 + 1, 16, ctypes.byref(e), py, None)
    assert rc == sdq.ERR_INVALID and b"M too large" in lib.sdq_last_error()
    item = sdq.GroupItem(w.h, pa, 2**30 + 1, e, py)
    rc = lib.sdq_qlinear_group(ctypes.byref(item), 1, None)
    assert rc == sdq.ERR_INVALID and b"group item 0: M too large" in lib.sdq_last_error()
    rc = lib.sdq_act_quant(pa, 4, 2**22 + 1, py, py, None)
    assert rc == sdq.ERR_INVALID and b"2^22" in lib.sdq_last_error()
    torch.cuda.synchronize()
    assert float(Y.abs().sum()) == 0.0  # nothing ran


def test_host_pointer_entry_point(sdq_dev, oracle):
    import sdq

    M, K, N = 123, 3072, 640
    A, q, s, bias = _inputs(M, K, N, seed=77)
    w = sdq.Weight.from_host(q, s)
    got = sdq.qlinear_host(w, A, bias=bias)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias), "host entry")
    gate = oracle.randn(N, 5)
    x = oracle.randn(M * N, 6).reshape(M, N)
    got = sdq.qlinear_host(w, A, kind="gated", bias=bias, gate=gate, resid=x)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x),
                    "host gated")


def test_host_entry_multi_chunk(sdq_dev, oracle):
    """Host arrays larger than one 16 MiB pinned bounce buffer: A (2 chunks),
    the residual and Y (3 chunks each) cross chunk edges in the middle of a
    row (K*4 and N*4 do not divide 16 MiB). Two calls in a row, the second
    smaller, reuse the same staging. Each result equals the device entry's
    bit for bit; the device entry is pinned against the oracle elsewhere."""
    import sdq

    rng = np.random.default_rng(5)
    K, N = 1540, 2620
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = (rng.random(N, dtype=np.float32) * 0.01 + 1e-3).astype(np.float32)
    w = sdq.Weight.from_host(q, s)
    bias = rng.standard_normal(N).astype(np.float32)
    gate = rng.standard_normal(N).astype(np.float32)
    for M in (4100, 1703):
        A = rng.standard_normal((M, K)).astype(np.float32)
        x = rng.standard_normal((M, N)).astype(np.float32)
        got = sdq.qlinear_host(w, A, kind="gated", bias=bias, gate=gate, resid=x)
        want = _run(sdq_dev, w, A, kind="gated", bias=bias, gate=gate, resid=x)
        assert_bitexact(got, want, f"host multi-chunk M={M}")


def test_unaligned_and_strided_buffers(sdq_dev, oracle):
    """A and Y at 4-byte (not 16-byte) aligned device addresses take the
    scalar load/store paths and still match bit for bit."""
    import torch

    import sdq

    M, K, N = 50, 1028, 516
    A, q, s, bias = _inputs(M, K, N, seed=31)
    w = sdq.Weight.from_host(q, s)
    Abuf = torch.zeros(M * K + 1, device=sdq_dev)
    Abuf[1:] = torch.from_numpy(A.ravel()).to(sdq_dev)
    Ybuf = torch.zeros(M * N + 1, device=sdq_dev)
    A_v = Abuf[1:].view(M, K)
    Y_v = Ybuf[1:].view(M, N)
    sdq.qlinear(w, A_v, Y_v, bias=torch.from_numpy(bias).to(sdq_dev))
    torch.cuda.synchronize()
    assert_bitexact(Y_v.cpu().numpy(), oracle.linear(A, q, s, bias=bias), "unaligned")


def test_repeated_calls_and_streams(sdq_dev, oracle):
    """Same result on a second stream and on repeated calls (workspace reuse)."""
    import torch

    import sdq

    M, K, N = 400, 3072, 2048
    A, q, s, _ = _inputs(M, K, N, seed=555)
    w = sdq.Weight.from_host(q, s)
    A_d = torch.from_numpy(A).to(sdq_dev)
    want = oracle.qgemm(A, q, s)
    st = torch.cuda.Stream()
    outs = []
    for i in range(3):
        Y = torch.empty((M, N), device=sdq_dev)
        with torch.cuda.stream(st if i == 1 else torch.cuda.current_stream()):
            sdq.qgemm(w, A_d, Y)
        torch.cuda.synchronize()
        outs.append(Y.cpu().numpy())
    for o in outs:
        assert_bitexact(o, want, "repeat")


# ----------------------------------------------------------------- split-K
# Few output tiles over a long K: the 128x128 kernel splits K across
# workgroups (int32 partial slices, exact) and a reduction applies the
# epilogue. M is not a multiple of 128, so the last row tile of every slice
# is masked.
SPLITK_SHAPES = [(157, 14336, 3072),  # FFN down at the audio branch's token count
                 (200, 6144, 1000),   # ragged N, eight splits
                 (90, 8192, 512)]     # fewest tiles


@pytest.mark.parametrize("M,K,N", SPLITK_SHAPES)
def test_splitk_epilogues_bitexact(sdq_dev, oracle, M, K, N):
    import sdq

    print(f"[splitk] M={M} K={K} N={N}", flush=True)
    A, q, s, bias = _inputs(M, K, N, seed=11 * M + K + N)
    gate = oracle.randn(N, 91)
    x = oracle.randn(M * N, 92).reshape(M, N)
    w = sdq.Weight.from_host(q, s)
    aq, _ = oracle.act_quant(A)
    assert_bitexact(_run(sdq_dev, w, A, kind="acc"), oracle.qgemm_acc(aq, q), "int32 acc")
    assert_bitexact(_run(sdq_dev, w, A), oracle.qgemm(A, q, s), "qgemm")
    assert_bitexact(_run(sdq_dev, w, A, bias=bias), oracle.linear(A, q, s, bias=bias), "mlin")
    for fma in (True, False):
        got = _run(sdq_dev, w, A, kind="gated", bias=bias, gate=gate, resid=x, gate_fma=fma)
        want = oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x,
                             use_fma=fma)
        assert_bitexact(got, want, f"gated fma={fma}")
    got = _run(sdq_dev, w, A, kind="resid", bias=bias, resid=x)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias, epilogue="resid", resid=x), "resid")
    got = _run(sdq_dev, w, A, kind="gelu", bias=bias)
    want = oracle.linear(A, q, s, bias=bias, epilogue="gelu")
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want))), float(err.max())


# ------------------------------------------------- tiny M, quantized in-kernel
# M <= 4 rows: the skinny GEMM quantizes A itself (every workgroup, into LDS).
@pytest.mark.parametrize("M,K,N", [(1, 3072, 18432), (2, 3072, 3072), (3, 31, 13), (4, 14336, 3072),
                                   (4, 257, 516), (1, 1, 64)])
def test_tiny_m_in_kernel_quant_bitexact(sdq_dev, oracle, M, K, N):
    import sdq

    print(f"[qin] M={M} K={K} N={N}", flush=True)
    A, q, s, bias = _inputs(M, K, N, seed=7 * M + K + N)
    A[0, 0] = np.float32(-A[0].__abs__().max() * 2)  # the row max is a negative value
    w = sdq.Weight.from_host(q, s)
    gate = oracle.randn(N, 77)
    x = oracle.randn(M * N, 78).reshape(M, N)
    assert_bitexact(_run(sdq_dev, w, A), oracle.qgemm(A, q, s), "qgemm")
    assert_bitexact(_run(sdq_dev, w, A, bias=bias), oracle.linear(A, q, s, bias=bias), "mlin")
    got = _run(sdq_dev, w, A, kind="gated", bias=bias, gate=gate, resid=x)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias, epilogue="gated", gate=gate, resid=x),
                    "gated")
    got = _run(sdq_dev, w, A, kind="resid", bias=bias, resid=x)
    assert_bitexact(got, oracle.linear(A, q, s, bias=bias, epilogue="resid", resid=x), "resid")
    aq, _ = oracle.act_quant(A)
    assert_bitexact(_run(sdq_dev, w, A, kind="acc"), oracle.qgemm_acc(aq, q), "acc")


def test_tiny_m_special_rows_and_unaligned(sdq_dev, oracle):
    """The reference's special rows (zero, NaN, +-Inf, denormal, huge, ties)
    in groups of 1..4 rows, through the in-kernel quantizer; then A and Y at
    4-byte aligned addresses (scalar loads)."""
    import torch

    import sdq

    r = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    A_all, bq, bs, want = r["special_a"], r["special_bq"], r["special_bs"], r["special_out"]
    w = sdq.Weight.from_host(bq, bs)
    for M in (1, 2, 3, 4):
        for i0 in range(0, A_all.shape[0] - M + 1, M):
            got = _run(sdq_dev, w, A_all[i0:i0 + M])
            assert_bitexact(got, want[i0:i0 + M], f"special rows {i0}..{i0 + M - 1}")
    M, K, N = 3, 1028, 516
    A, q, s, bias = _inputs(M, K, N, seed=33)
    w = sdq.Weight.from_host(q, s)
    Abuf = torch.zeros(M * K + 1, device=sdq_dev)
    Abuf[1:] = torch.from_numpy(A.ravel()).to(sdq_dev)
    Ybuf = torch.zeros(M * N + 1, device=sdq_dev)
    sdq.qlinear(w, Abuf[1:].view(M, K), Ybuf[1:].view(M, N), bias=torch.from_numpy(bias).to(sdq_dev))
    torch.cuda.synchronize()
    assert_bitexact(Ybuf[1:].view(M, N).cpu().numpy(), oracle.linear(A, q, s, bias=bias),
                    "unaligned tiny M")


# ------------------------------------------------------ streamed batch upload
def test_weight_upload_batch_equals_single_uploads(sdq_dev):
    """sdq_weight_upload_batch (pinned ring, async copies, repack overlap) gives
    the same device weights as sdq_weight_upload of the concatenated parts:
    multi-part sources (q|k|v style), odd shapes, unaligned scale bytes, and
    more sources than staging slots."""
    import sdq

    rng = np.random.default_rng(77)
    shapes = [[(64, 96)], [(13, 31)], [(100, 257), (28, 257), (1, 257)], [(300, 1024)],
              [(256, 3072), (256, 3072)], [(5, 8)], [(1000, 64)]]
    sources, whole = [], []
    for parts in shapes:
        src, qs, ss = [], [], []
        for (n, k) in parts:
            q = rng.integers(-127, 128, (n, k)).astype(np.int8)
            s = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
            src.append((q, memoryview(b"\x00" + s.tobytes())[1:]))  # unaligned scale bytes
            qs.append(q)
            ss.append(s)
        sources.append(src)
        whole.append((np.concatenate(qs), np.concatenate(ss)))
    ws = sdq.upload_batch(sources)
    for w, (q, s) in zip(ws, whole):
        q2, s2 = w.export()
        assert_bitexact(q2, q, "batch q")
        assert_bitexact(s2, s, "batch scale")
        single = sdq.Weight.from_host(q, s)
        q3, s3 = single.export()
        assert_bitexact(q3, q2, "single vs batch")
