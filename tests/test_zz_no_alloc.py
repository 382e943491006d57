"""sdq_qlinear_noalloc: the qlinear entry point that allocates nothing (its
scratch is a static per-GPU device array), against sdq_qlinear, bit for bit,
through the C ABI: two calls in a row on one weight (the second with fewer
rows), a long-K shape that takes the split-K path (its partial sums live in
the scratch too), a few-row shape (quantized inside the GEMM), and a call too
large for the scratch, which must fail before anything is launched."""
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
