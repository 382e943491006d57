"""sdq_qlinear_noalloc: the qlinear entry point that allocates nothing (its
scratch is a static per-GPU device array), against sdq_qlinear, bit for bit,
through the C ABI: two calls in a row on one weight (the second with fewer
rows), a long-K shape that takes the split-K path (its partial sums live in
the scratch too), a few-row shape (quantized inside the GEMM), a call too
large for the scratch, which must fail before anything is launched, and calls
on a stream that sdq_qlinear never used, which must leave the device's free
memory unchanged (sdq_qlinear's workspace is per stream and grows on first
use)."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _noalloc(sdq, w, A, Y, kind="none", bias=None, gate=None, resid=None):
    e = sdq.make_epilogue(kind, bias, gate, resid, True)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return sdq._lib.sdq_qlinear_noalloc(w.h, P(A), A.shape[0], A.shape[1], ctypes.byref(e), P(Y),
                                        None)


def _case(sdq_dev, oracle, w, q, s, M, K, kind, seed):
    import torch

    import sdq

    print(f"[noalloc] M={M} K={K} N={w.N} {kind}", flush=True)
    A = torch.from_numpy(oracle.randn(M * K, seed).reshape(M, K)).to(sdq_dev)
    b = torch.from_numpy(oracle.randn(w.N, seed + 1) * np.float32(0.01)).to(sdq_dev)
    g = torch.from_numpy(oracle.randn(w.N, seed + 2)).to(sdq_dev) if kind == "gated" else None
    r0 = torch.from_numpy(oracle.randn(M * w.N, seed + 3).reshape(M, w.N)).to(sdq_dev)
    want = r0.clone() if kind == "gated" else torch.full((M, w.N), -7.0, device=sdq_dev)
    got = r0.clone() if kind == "gated" else torch.full((M, w.N), -9.0, device=sdq_dev)
    sdq.qlinear(w, A, want, kind=kind, bias=b, gate=g, resid=want if kind == "gated" else None)
    rc = _noalloc(sdq, w, A, got, kind, b, g, got if kind == "gated" else None)
    assert rc == sdq.OK, sdq._lib.sdq_last_error()
    torch.cuda.synchronize()
    assert_bitexact(got.cpu().numpy(), want.cpu().numpy(), f"noalloc M={M} K={K} {kind}")


def test_noalloc_matches_qlinear(sdq_dev, oracle):
    import sdq

    K, N = 3072, 2048
    W = oracle.randn(N * K, 1).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    w = sdq.Weight.from_host(q, s)
    _case(sdq_dev, oracle, w, q, s, 1000, K, "none", 10)   # 128x128 tiles
    _case(sdq_dev, oracle, w, q, s, 300, K, "gated", 20)   # a second, smaller call
    _case(sdq_dev, oracle, w, q, s, 3, K, "none", 30)      # few rows: quantized in the GEMM
    _case(sdq_dev, oracle, w, q, s, 1000, K, "none", 40)   # larger again after smaller
    w.free()
    # long K, few tiles: split-K, with its partial sums in the scratch
    K2, N2 = 14336, 3072
    W2 = oracle.randn(N2 * K2, 2).reshape(N2, K2) * np.float32(0.02)
    q2, s2 = oracle.quant_rows(W2)
    w2 = sdq.Weight.from_host(q2, s2)
    _case(sdq_dev, oracle, w2, q2, s2, 157, K2, "gated", 50)
    _case(sdq_dev, oracle, w2, q2, s2, 100, K2, "none", 60)
    w2.free()


def test_noalloc_rejects_calls_beyond_its_scratch(sdq_dev, oracle):
    import torch

    import sdq

    K, N = 3072, 256
    q, s = oracle.quant_rows(oracle.randn(N * K, 3).reshape(N, K))
    w = sdq.Weight.from_host(q, s)
    M = 30000  # 30000 x 3072 bytes of quantized activations > 64 MiB
    A = torch.zeros((M, K), device=sdq_dev)
    Y = torch.full((M, N), -3.0, device=sdq_dev)
    rc = _noalloc(sdq, w, A, Y)
    assert rc == sdq.ERR_INVALID
    assert b"bytes of scratch" in sdq._lib.sdq_last_error()
    torch.cuda.synchronize()
    assert bool((Y == -3.0).all()), "a rejected call must not write its output"
    w.free()


def test_noalloc_allocates_nothing(sdq_dev, oracle):
    import torch

    import sdq

    K, N = 3072, 1024
    K2, N2 = 14336, 3072
    q, s = oracle.quant_rows(oracle.randn(N * K, 4).reshape(N, K) * np.float32(0.02))
    q2, s2 = oracle.quant_rows(oracle.randn(N2 * K2, 5).reshape(N2, K2) * np.float32(0.02))
    w, w2 = sdq.Weight.from_host(q, s), sdq.Weight.from_host(q2, s2)
    A = torch.from_numpy(oracle.randn(900 * K, 6).reshape(900, K)).to(sdq_dev)
    A2 = torch.from_numpy(oracle.randn(157 * K2, 7).reshape(157, K2)).to(sdq_dev)
    Y, Y2 = torch.empty((900, N), device=sdq_dev), torch.empty((157, N2), device=sdq_dev)
    want, want2 = torch.empty_like(Y), torch.empty_like(Y2)
    # load every kernel these calls use (on the default stream) before measuring
    sdq.qlinear(w, A, want)
    sdq.qlinear(w2, A2, want2)
    assert _noalloc(sdq, w, A, Y) == sdq.OK
    torch.cuda.synchronize()
    fresh = torch.cuda.Stream()
    # the stream's first launches (its queue) come from an in-place torch op,
    # so that only the calls below are measured
    with torch.cuda.stream(fresh):
        Y.mul_(1.0)
        Y2.mul_(1.0)
    fresh.synchronize()
    print("[noalloc] free memory around calls on a fresh stream", flush=True)
    free0 = torch.cuda.mem_get_info()[0]
    e = sdq.make_epilogue("none", None, None, None, True)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for a, wt, y in ((A, w, Y), (A2, w2, Y2), (A, w, Y)):  # 128x128 tiles, split-K, again
        rc = sdq._lib.sdq_qlinear_noalloc(wt.h, P(a), a.shape[0], a.shape[1], ctypes.byref(e), P(y),
                                          ctypes.c_void_p(fresh.cuda_stream))
        assert rc == sdq.OK, sdq._lib.sdq_last_error()
    fresh.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
    assert_bitexact(Y.cpu().numpy(), want.cpu().numpy(), "noalloc on a fresh stream")
    assert_bitexact(Y2.cpu().numpy(), want2.cpu().numpy(), "noalloc split-K on a fresh stream")
    w.free()
    w2.free()
