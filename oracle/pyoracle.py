"""CPU ORACLE — test infrastructure only.

numpy/ctypes front end over oracle/liboracle.so (our plain-C restatement of
the reference's int8 qGEMM path) and oracle/_ref/libsdref.so (the reference's
own qgemm/tensor/sdcpp sources compiled in place). Imported only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, and only as the
checker: the shipped library never calls into this module.

Also holds a numpy writer for the .sdcpp v1 format, restating
tools/quantize/pack_sdcpp.py:4-13 (layout), 45-51 (quant_rows) and 90-124
(write order), used to build fixtures for the product's loader.
"""
from __future__ import annotations

import ctypes
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(HERE, "liboracle.so")
_REF = os.path.join(HERE, "_ref", "libsdref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def _load():
    if not os.path.exists(_LIB):
        raise RuntimeError(f"oracle library missing: {_LIB} (run __graft_entry__.build())")
    lib = ctypes.CDLL(_LIB)
    lib.orc_act_quant.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
    lib.orc_qgemm_acc.argtypes = [_i8p, _i8p, _i64, _i64, _i64, _i32p, ctypes.c_int]
    lib.orc_rescale.argtypes = [_i32p, _f32p, _f32p, _i64, _i64, _f32p]
    lib.orc_linear_at.argtypes = [_i8p, _f32p, _i8p, _f32p, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, _i64, _i64,
                                  ctypes.c_void_p, ctypes.c_void_p, _i64, _f32p]
    lib.orc_qgemm.argtypes = [_f32p, _i8p, _f32p, _i64, _i64, _i64, _f32p, ctypes.c_int]
    lib.orc_qgemm.restype = ctypes.c_int
    lib.orc_bias_add.argtypes = [_f32p, _f32p, _i64, _i64]
    lib.orc_gated_add.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_int]
    lib.orc_add.argtypes = [_f32p, _f32p, _i64]
    lib.orc_linear_f32.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_void_p, _f32p]
    lib.orc_gelu_tanh.argtypes = [_f32p, _i64]
    lib.orc_layernorm.argtypes = [_f32p, _i64, _i64, ctypes.c_float, _f32p]
    lib.orc_layernorm_affine.argtypes = [_f32p, _i64, _i64, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_float, _f32p]
    lib.orc_mod_rows.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _f32p]
    lib.orc_rmsnorm.argtypes = [_f32p, _i64, _i64, _i64, _f32p, ctypes.c_float]
    lib.orc_sdpa.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64, _f32p, _i64, _i64, _i64,
                             ctypes.c_int, ctypes.c_int, _f32p]
    lib.orc_rope_cs.argtypes = [_f32p, _i64, _f32p]
    lib.orc_rope.argtypes = [_f32p, _i64, _i64, _i64, ctypes.c_int, _f32p, ctypes.c_int]
    lib.orc_rope_freqs_3d.argtypes = [ctypes.c_int] * 4 + [ctypes.c_float, _f32p]
    lib.orc_rope_freqs_1d.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                      _f32p]
    lib.orc_quantize_rowwise.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
    lib.orc_quant_rows.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
    lib.orc_randu.argtypes = [_f32p, _i64, ctypes.c_uint64]
    lib.orc_randn.argtypes = [_f32p, _i64, ctypes.c_uint64]
    lib.orc_round_to_i8.argtypes = [ctypes.c_float]
    lib.orc_round_to_i8.restype = ctypes.c_int
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def nthreads_default() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    if cap > 0:
        n = min(n, cap)
    return max(1, min(n, 64))


# ---------------------------------------------------------------- restatement
def act_quant(A: np.ndarray):
    A = np.ascontiguousarray(A, np.float32)
    M, K = A.shape
    aq = np.empty((M, K), np.int8)
    asc = np.empty((M,), np.float32)
    lib().orc_act_quant(A, M, K, aq, asc)
    return aq, asc


def qgemm_acc(aq: np.ndarray, bq: np.ndarray, nthreads: int | None = None):
    aq = np.ascontiguousarray(aq, np.int8)
    bq = np.ascontiguousarray(bq, np.int8)
    M, K = aq.shape
    N = bq.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().orc_qgemm_acc(aq, bq, M, N, K, acc, nthreads or nthreads_default())
    return acc


def rescale(acc, asc, bs):
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.float32)
    lib().orc_rescale(acc, np.ascontiguousarray(asc, np.float32),
                      np.ascontiguousarray(bs, np.float32), M, N, out)
    return out


def qgemm(A, Bq, bs, nthreads: int | None = None):
    """sd::qgemm restated (src/core/qgemm.cpp:73-142)."""
    A = np.ascontiguousarray(A, np.float32)
    Bq = np.ascontiguousarray(Bq, np.int8)
    bs = np.ascontiguousarray(bs, np.float32)
    M, K = A.shape
    N = Bq.shape[0]
    out = np.empty((M, N), np.float32)
    if M * N == 0:
        return out
    if K == 0:
        out[:] = 0
        return out
    rc = lib().orc_qgemm(A, Bq, bs, M, K, N, out, nthreads or nthreads_default())
    if rc != 0:
        raise MemoryError("orc_qgemm allocation failed")
    return out


def linear_at(aq, asc, bq, bs, ms, ns, bias=None, epilogue="none", gate=None, resid=None,
              use_fma=True):
    """Outputs of qgemm (+ bias, + the gated / plain residual epilogue) at
    positions (ms[i], ns[i]) only, from the quantized activations (act_quant)
    and the packed weights; resid is the full [M, N] residual."""
    aq = np.ascontiguousarray(aq, np.int8)
    bq = np.ascontiguousarray(bq, np.int8)
    asc = np.ascontiguousarray(asc, np.float32)
    bs = np.ascontiguousarray(bs, np.float32)
    ms = np.ascontiguousarray(ms, np.int64)
    ns = np.ascontiguousarray(ns, np.int64)
    K, N = aq.shape[1], bq.shape[0]
    assert bq.shape[1] == K and ms.shape == ns.shape
    assert ms.size == 0 or (0 <= ms.min() and ms.max() < aq.shape[0])
    assert ns.size == 0 or (0 <= ns.min() and ns.max() < N)
    epi = {"none": 0, "gated": 2, "resid": 3}[epilogue]
    keep = []

    def ptr(x, shape):
        if x is None:
            return None
        x = np.ascontiguousarray(x, np.float32)
        assert x.shape == shape
        keep.append(x)
        return x.ctypes.data

    b = ptr(bias, (N,))
    g = ptr(gate, (N,)) if epi == 2 else None
    r = ptr(resid, (aq.shape[0], N)) if epi in (2, 3) else None
    out = np.empty(ms.shape, np.float32)
    lib().orc_linear_at(aq, asc, bq, bs, b, epi, 1 if use_fma else 0, g, r, K, N, ms.ctypes.data,
                        ns.ctypes.data, ms.size, out)
    return out


def bias_add(y, b):
    y = np.array(y, np.float32, copy=True, order="C")
    M, N = y.shape
    lib().orc_bias_add(y, np.ascontiguousarray(b, np.float32), M, N)
    return y


def gated_add(x, y, g, use_fma=True):
    x = np.array(x, np.float32, copy=True, order="C")
    M, N = x.shape
    lib().orc_gated_add(x, np.ascontiguousarray(y, np.float32),
                        np.ascontiguousarray(g, np.float32), M, N, 1 if use_fma else 0)
    return x


def add(x, y):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().orc_add(x.reshape(-1), np.ascontiguousarray(y, np.float32).reshape(-1), x.size)
    return x


def linear_f32(x, w, bias=None):
    """The F32 Linear (blk::linear -> sd::matmul): x [M,K] . w [K,N] (+ bias)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    M, K = x.shape
    K2, N = w.shape
    assert K == K2, (x.shape, w.shape)
    y = np.empty((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_linear_f32(x, M, K, w, N, None if b is None else b.ctypes.data, y)
    return y


def gelu_tanh(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().orc_gelu_tanh(x.reshape(-1), x.size)
    return x


def layernorm(x, eps=1e-6, w=None, b=None):
    """blocks.cpp:18-43 (no affine unless w / b: norm3, the fusion pre-norm)."""
    x = np.ascontiguousarray(x, np.float32)
    M, N = x.shape
    y = np.empty_like(x)
    if w is None and b is None:
        lib().orc_layernorm(x, M, N, eps, y)
    else:
        w = None if w is None else np.ascontiguousarray(w, np.float32)
        b = None if b is None else np.ascontiguousarray(b, np.float32)
        lib().orc_layernorm_affine(x, M, N, None if w is None else w.ctypes.data,
                                   None if b is None else b.ctypes.data, eps, y)
    return y


def mod_rows(x, shift, scale):
    """ovi_dit.cpp:161-172: x*(1+scale)+shift (fused multiply-add)."""
    x = np.ascontiguousarray(x, np.float32)
    L, C = x.shape
    y = np.empty_like(x)
    lib().orc_mod_rows(x, np.ascontiguousarray(shift, np.float32),
                       np.ascontiguousarray(scale, np.float32), L, C, y)
    return y


def rmsnorm(x, w, eps=1e-6):
    """tensor.cpp:112-123 over the last dim (returns a new array)."""
    y = np.array(x, np.float32, copy=True, order="C")
    M, N = y.shape
    lib().orc_rmsnorm(y, M, N, N, np.ascontiguousarray(w, np.float32), eps)
    return y


def sdpa(q, k, v, heads):
    """blocks.cpp:112-199 (non-causal) on contiguous q [Lq, C], k, v [Lk, C]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    Lq, C = q.shape
    Lk = k.shape[0]
    out = np.empty((Lq, C), np.float32)
    p = np.empty((max(Lk, 1),), np.float32)
    lib().orc_sdpa(q, C, k, C, v, C, out, C, Lq, Lk, heads, C // heads, p)
    return out


def rope_cs(ang):
    """(cosf, sinf) of a [L, nr] angle table -> [L, nr, 2]."""
    ang = np.ascontiguousarray(ang, np.float32)
    cs = np.empty(ang.shape + (2,), np.float32)
    lib().orc_rope_cs(ang, ang.size, cs)
    return cs


def rope(x, cs, heads):
    """blocks.cpp:86-100 with the (cos, sin) table cs [L, nr, 2]."""
    y = np.array(x, np.float32, copy=True, order="C")
    L, C = y.shape
    lib().orc_rope(y, L, C, C, heads, np.ascontiguousarray(cs, np.float32), cs.shape[1])
    return y


def rope_freqs_3d(T, H, W, head_dim, theta=10000.0):
    d = head_dim
    nr = (d - 4 * (d // 6)) // 2 + (2 * (d // 6)) // 2 * 2
    ang = np.empty((T * H * W, nr), np.float32)
    assert lib().orc_rope_freqs_3d(T, H, W, d, theta, ang) == nr
    return ang


def rope_freqs_1d(L, head_dim, theta=10000.0, scaling=1.0):
    nr = (head_dim - 4 * (head_dim // 6)) // 2
    ang = np.empty((L, nr), np.float32)
    assert lib().orc_rope_freqs_1d(L, head_dim, theta, scaling, ang) == nr
    return ang


def quantize_rowwise(W):
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    lib().orc_quantize_rowwise(W, N, K, q, s)
    return q, s


def quant_rows(W):
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    lib().orc_quant_rows(W, N, K, q, s)
    return q, s


def randu(n, seed):
    x = np.empty((n,), np.float32)
    lib().orc_randu(x, n, seed)
    return x


def randn(n, seed):
    x = np.empty((n,), np.float32)
    lib().orc_randn(x, n, seed)
    return x


def round_to_i8(v: float) -> int:
    return lib().orc_round_to_i8(ctypes.c_float(v))


def linear(A, Bq, bs, bias=None, epilogue="none", gate=None, resid=None, use_fma=True,
           nthreads=None):
    """mlin (src/model/ovi_dit.cpp:66-84) plus the consumer that follows it in
    the reference blocks: 'none' (qgemm+bias), 'gelu' (fc1 then
    gelu_tanh_inplace, 214-222), 'gated' (fc2/self-o then gated_add_inplace,
    152-159, 187, 221), 'resid' (cross-o then add_inplace, 144-149, 251)."""
    y = qgemm(A, Bq, bs, nthreads)
    if bias is not None:
        y = bias_add(y, bias)
    if epilogue == "none":
        return y
    if epilogue == "gelu":
        return gelu_tanh(y)
    if epilogue == "gated":
        return gated_add(resid, y, gate, use_fma)
    if epilogue == "resid":
        return add(resid, y)
    raise ValueError(epilogue)


# ----------------------------------------------------------- reference build
class Ref:
    """The reference's own sources compiled in place (oracle/_ref)."""

    def __init__(self, nthreads: int | None = None):
        if not os.path.exists(_REF):
            raise FileNotFoundError(_REF)
        L = ctypes.CDLL(_REF)
        L.sdref_qgemm.argtypes = [_f32p, _i8p, _f32p, _i64, _i64, _i64, _f32p]
        L.sdref_qgemm.restype = ctypes.c_int
        L.sdref_quantize_rowwise.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
        L.sdref_randu.argtypes = [_f32p, _i64, ctypes.c_uint64]
        L.sdref_set_nthreads.argtypes = [ctypes.c_int]
        L.sdref_nthreads.restype = ctypes.c_int
        L.sdref_sdcpp_lookup.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int),
            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int),
            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, ctypes.c_int]
        L.sdref_sdcpp_lookup.restype = ctypes.c_int
        L.sdref_layernorm.argtypes = [_f32p, _i64, _i64, ctypes.c_float, ctypes.c_void_p,
                                      ctypes.c_void_p, _f32p]
        L.sdref_layernorm.restype = ctypes.c_int
        L.sdref_mod_rows.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _f32p]
        L.sdref_mod_rows.restype = ctypes.c_int
        L.sdref_rmsnorm.argtypes = [_f32p, _i64, _i64, _f32p, ctypes.c_float]
        L.sdref_rmsnorm.restype = ctypes.c_int
        L.sdref_apply_rope.argtypes = [_f32p, _i64, _i64, _f32p, ctypes.c_int, ctypes.c_int]
        L.sdref_apply_rope.restype = ctypes.c_int
        L.sdref_rope_freqs_3d.argtypes = [ctypes.c_int] * 4 + [ctypes.c_float, _f32p]
        L.sdref_rope_freqs_3d.restype = ctypes.c_int
        L.sdref_rope_freqs_1d.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                          ctypes.c_float, _f32p]
        L.sdref_rope_freqs_1d.restype = ctypes.c_int
        L.sdref_sdpa.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int, _f32p]
        L.sdref_sdpa.restype = ctypes.c_int
        L.sdref_matmul.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_void_p, _f32p]
        L.sdref_matmul.restype = ctypes.c_int
        self.L = L
        self.set_nthreads(nthreads or nthreads_default())

    @staticmethod
    def available() -> bool:
        return os.path.exists(_REF)

    def set_nthreads(self, n: int):
        self.L.sdref_set_nthreads(int(n))
        self.nthreads = int(self.L.sdref_nthreads())

    def qgemm(self, A, Bq, bs):
        A = np.ascontiguousarray(A, np.float32)
        Bq = np.ascontiguousarray(Bq, np.int8)
        bs = np.ascontiguousarray(bs, np.float32)
        M, K = A.shape
        N = Bq.shape[0]
        out = np.empty((M, N), np.float32)
        if self.L.sdref_qgemm(A, Bq, bs, M, K, N, out) != 0:
            raise RuntimeError("reference qgemm threw")
        return out

    def matmul(self, x, w, bias=None):
        """sd::matmul (gemm.cpp:115): x [M,K] . w [K,N] (+ bias)."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        M, K = x.shape
        N = w.shape[1]
        out = np.empty((M, N), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        if self.L.sdref_matmul(x, M, K, w, N, None if b is None else b.ctypes.data, out) != 0:
            raise RuntimeError("reference matmul threw")
        return out

    def quantize_rowwise(self, W):
        W = np.ascontiguousarray(W, np.float32)
        N, K = W.shape
        q = np.empty((N, K), np.int8)
        s = np.empty((N,), np.float32)
        self.L.sdref_quantize_rowwise(W, N, K, q, s)
        return q, s

    def layernorm(self, x, eps=1e-6, w=None, b=None):
        x = np.ascontiguousarray(x, np.float32)
        M, N = x.shape
        y = np.empty_like(x)
        w = None if w is None else np.ascontiguousarray(w, np.float32)
        b = None if b is None else np.ascontiguousarray(b, np.float32)
        if self.L.sdref_layernorm(x, M, N, eps, None if w is None else w.ctypes.data,
                                  None if b is None else b.ctypes.data, y) != 0:
            raise RuntimeError("reference layernorm threw")
        return y

    def mod_rows(self, x, shift, scale):
        x = np.ascontiguousarray(x, np.float32)
        L, C = x.shape
        y = np.empty_like(x)
        if self.L.sdref_mod_rows(x, np.ascontiguousarray(shift, np.float32),
                                 np.ascontiguousarray(scale, np.float32), L, C, y) != 0:
            raise RuntimeError("reference mod_rows threw")
        return y

    def rmsnorm(self, x, w, eps=1e-6):
        y = np.array(x, np.float32, copy=True, order="C")
        M, N = y.shape
        if self.L.sdref_rmsnorm(y, M, N, np.ascontiguousarray(w, np.float32), eps) != 0:
            raise RuntimeError("reference rmsnorm threw")
        return y

    def apply_rope(self, x, ang, heads):
        y = np.array(x, np.float32, copy=True, order="C")
        L, C = y.shape
        ang = np.ascontiguousarray(ang, np.float32)
        if self.L.sdref_apply_rope(y, L, C, ang, ang.shape[1], heads) != 0:
            raise RuntimeError("reference apply_rope threw")
        return y

    def rope_freqs_3d(self, T, H, W, head_dim, theta=10000.0):
        ang = np.empty((T * H * W, head_dim), np.float32)
        nr = self.L.sdref_rope_freqs_3d(T, H, W, head_dim, theta, ang)
        return np.ascontiguousarray(ang.ravel()[:T * H * W * nr].reshape(T * H * W, nr))

    def rope_freqs_1d(self, L, head_dim, theta=10000.0, scaling=1.0):
        ang = np.empty((L, head_dim), np.float32)
        nr = self.L.sdref_rope_freqs_1d(L, head_dim, theta, scaling, ang)
        return np.ascontiguousarray(ang.ravel()[:L * nr].reshape(L, nr))

    def sdpa(self, q, k, v, heads):
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        out = np.empty(q.shape, np.float32)
        if self.L.sdref_sdpa(q, k, v, q.shape[0], k.shape[0], q.shape[1], heads, out) != 0:
            raise RuntimeError("reference sdpa threw")
        return out

    def randu(self, n, seed):
        x = np.empty((n,), np.float32)
        self.L.sdref_randu(x, n, seed)
        return x

    def sdcpp_lookup(self, path: str, name: str):
        dt = ctypes.c_int()
        dims = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int()
        doff = ctypes.c_int64()
        soff = ctypes.c_int64()
        cnt = ctypes.c_int()
        err = ctypes.create_string_buffer(256)
        rc = self.L.sdref_sdcpp_lookup(path.encode(), name.encode(), ctypes.byref(dt), dims,
                                       ctypes.byref(nd), ctypes.byref(doff), ctypes.byref(soff),
                                       ctypes.byref(cnt), err, 256)
        if rc < 0:
            raise RuntimeError(err.value.decode())
        if rc == 1:
            return None
        return dict(dtype=dt.value, dims=list(dims[: nd.value]), data_off=doff.value,
                    scale_off=soff.value, count=cnt.value)


# -------------------------------------------------------------- .sdcpp writer
SDCP_MAGIC = b"SDCP"
SDCP_VERSION = 1
MIN_QUANT_NUMEL = 65536  # tools/quantize/pack_sdcpp.py:22


def write_sdcpp(path: str, tensors, min_quant_numel: int = MIN_QUANT_NUMEL,
                force_quant=None):
    """Write a .sdcpp v1 file from {name: float32 array} in insertion order,
    following tools/quantize/pack_sdcpp.py:75-124: float tensors with
    numel >= min_quant_numel are quantized row-wise along the last dim with
    quant_rows, the rest stored raw f32. Blobs are packed back to back with
    no alignment padding (pack_sdcpp.py:86-88). Returns {name: (code, q, s)}."""
    force_quant = set(force_quant or ())
    plan, off = [], 0
    items = list(tensors.items())
    for name, x in items:
        x = np.ascontiguousarray(x, np.float32)
        dims = list(x.shape)
        numel = int(x.size)
        quant = (numel >= min_quant_numel or name in force_quant) and len(dims) > 0 and dims[-1] > 0
        rows = numel // dims[-1] if quant else 0
        blob = numel + rows * 4 if quant else numel * 4
        plan.append((name, 0 if quant else 1, dims, off, numel, rows, x))
        off += blob
    out = {}
    with open(path, "wb") as f:
        f.write(SDCP_MAGIC + struct.pack("<II", SDCP_VERSION, len(plan)))
        for name, code, dims, o, numel, rows, x in plan:
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<B", code))
            f.write(struct.pack("<I", len(dims)))
            f.write(struct.pack("<%dq" % len(dims), *dims))
            f.write(struct.pack("<Q", o))
        for name, code, dims, o, numel, rows, x in plan:
            if code == 0:
                q, s = quant_rows(x.reshape(rows, dims[-1]))
                f.write(q.tobytes())
                f.write(s.tobytes())
                out[name] = (0, q, s)
            else:
                f.write(x.tobytes())
                out[name] = (1, x, None)
    return out
