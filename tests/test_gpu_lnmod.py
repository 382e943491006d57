"""The DiT's norm + modulation folded into the activation quantizer
(sdq_qlinear_lnmod, sdq_ffn_lnmod): Y = epilogue(qgemm(mod_rows(layernorm(x),
shift, scale), W)) against the oracle's layernorm (blocks.cpp:18-43) and
mod_rows (ovi_dit.cpp:161-172), both pinned bit-exactly to the reference
build, then its linear. Bit-exact, including zero, constant, tiny, huge
and NaN rows."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _x(oracle, M, K, seed):
    rng = np.random.default_rng(seed)
    x = (oracle.randn(M * K, seed).reshape(M, K) * rng.uniform(0.05, 20, (M, 1))).astype(np.float32)
    if M > 6:
        x[1] = 0.0
        x[2] = np.float32(-1.5)
        x[3] *= np.float32(1e-30)
        x[4] *= np.float32(1e15)
        x[5, 3] = np.nan
    return x


def _mod(oracle, K, seed):
    return oracle.randn(K, seed), oracle.randn(K, seed + 1) * np.float32(0.2)


def _w(oracle, N, K, seed):
    W = oracle.randn(N * K, seed).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    return q, s, oracle.randn(N, seed + 2) * np.float32(0.01)


@pytest.mark.parametrize("M,K,N", [(1, 3072, 512), (40, 3072, 3072), (300, 998, 516),
                                   (768, 3072, 9216), (4500, 512, 2048)])
def test_qlinear_lnmod_bitexact(sdq_dev, oracle, M, K, N):
    import torch

    import sdq

    print(f"[lnmod] M={M} K={K} N={N}", flush=True)
    x = _x(oracle, M, K, 100 + M)
    shift, scale = _mod(oracle, K, 200 + K)
    q, s, bias = _w(oracle, N, K, 300 + N)
    h = oracle.mod_rows(oracle.layernorm(x, 1e-6), shift, scale)
    w = sdq.Weight.from_host(q, s)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    Y = torch.full((M, N), -7.0, device=sdq_dev)
    sdq.qlinear_lnmod(w, t(x), Y, t(shift), t(scale), 1e-6, kind="none", bias=t(bias))
    torch.cuda.synchronize()
    assert_bitexact(Y.cpu().numpy(), oracle.linear(h, q, s, bias=bias), "lnmod linear")
    gate = oracle.randn(N, 7)
    r = oracle.randn(M * N, 8).reshape(M, N)
    R = t(r)
    sdq.qlinear_lnmod(w, t(x), R, t(shift), t(scale), 1e-6, kind="gated", bias=t(bias),
                      gate=t(gate), resid=R)
    torch.cuda.synchronize()
    assert_bitexact(R.cpu().numpy(),
                    oracle.linear(h, q, s, bias=bias, epilogue="gated", gate=gate, resid=r),
                    "lnmod gated, in place")


@pytest.mark.parametrize("M,D,F", [(157, 3072, 14336), (300, 512, 1408), (40, 512, 1408)])
def test_ffn_lnmod_equals_ffn_on_reference_h(sdq_dev, oracle, M, D, F):
    import torch

    import sdq

    print(f"[ffn-lnmod] M={M} D={D} F={F}", flush=True)
    x = _x(oracle, M, D, 400 + M)
    shift, scale = _mod(oracle, D, 500 + D)
    q1, s1, b1 = _w(oracle, F, D, 600)
    q2, s2, b2 = _w(oracle, D, F, 700)
    gate = oracle.randn(D, 9)
    h = oracle.mod_rows(oracle.layernorm(x, 1e-6), shift, scale)
    w1, w2 = sdq.Weight.from_host(q1, s1), sdq.Weight.from_host(q2, s2)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    xa, hid_a = t(x), torch.empty((M, F), device=sdq_dev)
    sdq.ffn_lnmod(w1, t(b1), w2, t(b2), xa, t(shift), t(scale), t(gate), hid_a)
    xb, hid_b = t(x), torch.empty((M, F), device=sdq_dev)
    sdq.ffn(w1, t(b1), w2, t(b2), t(h), t(gate), hid_b, xb)
    torch.cuda.synchronize()
    assert_bitexact(hid_a.cpu().numpy(), hid_b.cpu().numpy(), "hid")
    assert_bitexact(xa.cpu().numpy(), xb.cpu().numpy(), "x")
    rows = np.arange(0, M, max(1, M // 16))
    want = oracle.linear(hid_b.cpu().numpy()[rows], q2, s2, bias=b2, epilogue="gated", gate=gate,
                         resid=x[rows])
    assert_bitexact(xa.cpu().numpy()[rows], want, "x vs oracle")


def test_qlinear_lnmod_fullsize_sampled(sdq_dev, oracle):
    """q|k|v at 720p/121 frames: M=27280, K=3072, N=9216, sampled rows."""
    import torch

    import sdq

    M, K, N = 27280, 3072, 9216
    print(f"[lnmod-full] M={M} K={K} N={N}", flush=True)
    x = _x(oracle, M, K, 800)
    shift, scale = _mod(oracle, K, 801)
    q, s, bias = _w(oracle, N, K, 802)
    w = sdq.Weight.from_host(q, s)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    Y = torch.empty((M, N), device=sdq_dev)
    sdq.qlinear_lnmod(w, t(x), Y, t(shift), t(scale), 1e-6, kind="none", bias=t(bias))
    torch.cuda.synchronize()
    rows = np.array([0, 1, 2, 3, 4, 5, 255, 256, 4097, M // 2, M - 257, M - 1])
    h = oracle.mod_rows(oracle.layernorm(x[rows], 1e-6), shift, scale)
    got = Y[torch.from_numpy(rows).to(sdq_dev)].cpu().numpy()
    assert_bitexact(got, oracle.linear(h, q, s, bias=bias), "sampled rows")


def test_lnmod_errors(sdq_dev, oracle):
    import torch

    import sdq

    q, s, _ = _w(oracle, 64, 128, 1)
    w = sdq.Weight.from_host(q, s)
    x = torch.zeros((4, 128), device=sdq_dev)
    Y = torch.empty((4, 64), device=sdq_dev)
    sc = torch.zeros(128, device=sdq_dev)
    with pytest.raises(sdq.SdqError, match="shift: required"):
        sdq.qlinear_lnmod(w, x, Y, None, sc)
    e = sdq.make_epilogue()
    rc = sdq._lib.sdq_qlinear_lnmod(w.h, ctypes.c_void_p(x.data_ptr()), 4, 128, None,
                                    ctypes.c_void_p(sc.data_ptr()), 1e-6, ctypes.byref(e),
                                    ctypes.c_void_p(Y.data_ptr()), None)
    assert rc == sdq.ERR_INVALID and b"shift or scale" in sdq._lib.sdq_last_error()
