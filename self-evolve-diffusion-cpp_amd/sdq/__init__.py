"""Python binding of the sdq C ABI (include/sdq.h) via ctypes.

The library does the work; this module only marshals pointers. Device
buffers come from torch (ROCm) tensors and the stream from
torch.cuda.current_stream(); nothing here computes results itself, and a
missing libsdq.so raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libsdq.so")
HOST_TEST_BIN = os.path.join(LIB_DIR, "test_host")

OK = 0
ERR_INVALID, ERR_HIP, ERR_NOMEM, ERR_FORMAT, ERR_NODEV, ERR_NOTFOUND = 1, 2, 3, 4, 5, 6
EPI_NONE, EPI_GELU, EPI_GATED, EPI_RESID, EPI_ACC = 0, 1, 2, 3, 4
EPI_NAMES = {"none": EPI_NONE, "gelu": EPI_GELU, "gated": EPI_GATED, "resid": EPI_RESID,
             "acc": EPI_ACC}


class SdqError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"sdq error {code}: {msg}")
        self.code = code


class Epilogue(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("gate_fma", ctypes.c_int),
                ("bias", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("resid", ctypes.c_void_p)]


class GroupItem(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("A", ctypes.c_void_p), ("M", ctypes.c_int64),
                ("epi", Epilogue), ("Y", ctypes.c_void_p)]


class FfnItem(ctypes.Structure):
    _fields_ = [("fc1", ctypes.c_void_p), ("b1", ctypes.c_void_p), ("fc2", ctypes.c_void_p),
                ("b2", ctypes.c_void_p), ("h", ctypes.c_void_p), ("M", ctypes.c_int64),
                ("gate", ctypes.c_void_p), ("gate_fma", ctypes.c_int), ("hid", ctypes.c_void_p),
                ("x", ctypes.c_void_p)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int), ("cu_count", ctypes.c_int),
                ("max_clock_khz", ctypes.c_int), ("mem_clock_khz", ctypes.c_int),
                ("total_mem", ctypes.c_int64), ("arch", ctypes.c_char * 64)]


class GemmPlan(ctypes.Structure):
    _fields_ = [("nlaunch", ctypes.c_int), ("splitk", ctypes.c_int),
                ("name", (ctypes.c_char * 48) * 2), ("row0", ctypes.c_int64 * 2),
                ("rows", ctypes.c_int64 * 2)]


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int),
                ("total_ms", ctypes.c_double)]


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64

# name -> (restype, argtypes); mirrors include/sdq.h
SIGNATURES = {
    "sdq_last_error": (ctypes.c_char_p, []),
    "sdq_version": (ctypes.c_char_p, []),
    "sdq_init": (ctypes.c_int, [ctypes.c_int]),
    "sdq_device_info_get": (ctypes.c_int, [ctypes.POINTER(DeviceInfo)]),
    "sdq_weight_upload": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, ctypes.POINTER(_vp)]),
    "sdq_weight_upload_device": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, ctypes.POINTER(_vp)]),
    "sdq_weight_free": (ctypes.c_int, [_vp]),
    "sdq_weight_upload_batch": (ctypes.c_int, [_vp, ctypes.c_int, _vp, ctypes.POINTER(_vp)]),
    "sdq_weight_upload_file": (ctypes.c_int, [ctypes.c_char_p, _vp, ctypes.c_int, _vp,
                                              ctypes.POINTER(_vp)]),
    "sdq_weight_dims": (ctypes.c_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "sdq_weight_export_host": (ctypes.c_int, [_vp, _vp, _vp]),
    "sdq_qlinear": (ctypes.c_int, [_vp, _vp, _i64, _i64, ctypes.POINTER(Epilogue), _vp, _vp]),
    "sdq_qgemm": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "sdq_qlinear_noalloc": (ctypes.c_int, [_vp, _vp, _i64, _i64, ctypes.POINTER(Epilogue), _vp,
                                           _vp]),
    "sdq_qlinear_group": (ctypes.c_int, [ctypes.POINTER(GroupItem), ctypes.c_int, _vp]),
    "sdq_qlinear_stack": (ctypes.c_int, [ctypes.POINTER(GroupItem), ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(FfnItem), _vp]),
    "sdq_rmsnorm_rope_batch": (ctypes.c_int, [_vp, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_float,
                                              _vp]),
    "sdq_layernorm": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, ctypes.c_float, _vp, _vp]),
    "sdq_add": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "sdq_linear_f32": (ctypes.c_int, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "sdq_sdpa": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64,
                                ctypes.c_int, ctypes.c_int, _vp]),
    "sdq_sdpa_batched": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]),
    "sdq_rmsnorm_rope": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, ctypes.c_float, ctypes.c_int,
                                        _vp, ctypes.c_int, _vp]),
    "sdq_ffn": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _vp, ctypes.c_int, _vp, _vp, _vp]),
    "sdq_qlinear_lnmod": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _vp, ctypes.c_float,
                                         ctypes.POINTER(Epilogue), _vp, _vp]),
    "sdq_ffn_lnmod": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, ctypes.c_float, _vp,
                                     ctypes.c_int, _vp, _vp]),
    "sdq_qlinear_host": (ctypes.c_int, [_vp, _vp, _i64, _i64, ctypes.POINTER(Epilogue), _vp]),
    "sdq_act_quant": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "sdq_device_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "sdq_device_free": (ctypes.c_int, [_vp]),
    "sdq_memcpy": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, ctypes.c_int, _vp]),
    "sdq_stream_sync": (ctypes.c_int, [_vp]),
    "sdq_stream_wait": (ctypes.c_int, [_vp, _vp]),
    "sdq_profile_begin": (ctypes.c_int, []),
    "sdq_profile_end": (ctypes.c_int, [ctypes.POINTER(KernelTime), ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_int)]),
    "sdq_sync": (ctypes.c_int, []),
    "sdq_qlinear_plan": (ctypes.c_int, [_vp, _i64, ctypes.c_int, ctypes.POINTER(GemmPlan)]),
}

_lib = None


def load_library(path: str = LIB_PATH):
    """Load libsdq.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libsdq.so not built: {path} (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc):
    if rc != OK:
        msg = _lib.sdq_last_error().decode(errors="replace")
        raise SdqError(rc, msg)


def init(device: int = 0):
    _check(load_library().sdq_init(device))


def device_info() -> dict:
    info = DeviceInfo()
    _check(load_library().sdq_device_info_get(ctypes.byref(info)))
    return dict(device=info.device, cu_count=info.cu_count, max_clock_khz=info.max_clock_khz,
                mem_clock_khz=info.mem_clock_khz, total_mem=info.total_mem,
                arch=info.arch.decode())


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    return ctypes.c_void_p(stream.cuda_stream)


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        return t.ctypes.data_as(ctypes.c_void_p)
    return ctypes.c_void_p(t.data_ptr())


def _bad(msg):
    return SdqError(ERR_INVALID, msg)


_DT = {"f32": "float32", "i32": "int32", "i8": "int8", "u8": "uint8"}


class _Args:
    """Checks the device-tensor arguments of one call before anything is
    launched. The C ABI receives bare pointers and cannot see a host buffer,
    a wrong element type, a strided view or a short buffer; any of those
    would reach a kernel as an out-of-bounds address, so each raises
    SdqError (ERR_INVALID) here. Calling the object checks one argument's
    type, element type, shape and layout and returns its address; done()
    then checks that every argument lives on the current GPU."""

    def __init__(self):
        self._seen = []

    def __call__(self, t, name, dt="f32", shape=None, contig=True, optional=False):
        """shape: the exact shape (None entries are free); contig=False accepts
        2-D views whose rows are contiguous but strided (the caller passes
        stride(0) as the row stride)."""
        if t is None:
            if optional:
                return None
            raise _bad(f"{name}: required")
        import torch

        if not isinstance(t, torch.Tensor):
            raise _bad(f"{name}: expected a torch device tensor, got {type(t).__name__}")
        want = getattr(torch, _DT[dt])
        if t.dtype != want:
            raise _bad(f"{name}: dtype {t.dtype}, expected {want}")
        if shape is not None:
            if t.dim() != len(shape) or any(w is not None and int(d) != int(w)
                                            for d, w in zip(t.shape, shape)):
                want_s = tuple("*" if w is None else int(w) for w in shape)
                raise _bad(f"{name}: shape {tuple(t.shape)}, expected {want_s}")
        if contig:
            if not t.is_contiguous():
                raise _bad(f"{name}: must be contiguous")
        elif t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
            raise _bad(f"{name}: must be 2-D with contiguous rows")
        self._seen.append((name, t))
        return ctypes.c_void_p(t.data_ptr())

    def done(self):
        import torch

        for name, t in self._seen:
            if not t.is_cuda:
                raise _bad(f"{name}: must be on the GPU (got device {t.device})")
            cur = torch.cuda.current_device()
            if t.device.index is not None and t.device.index != cur:
                raise _bad(f"{name}: on {t.device}, current device is cuda:{cur}")


def _ld(t):
    """Row stride (elements) of a 2-D tensor with contiguous rows."""
    return int(t.stride(0)) if t.shape[0] > 1 else int(t.shape[1])


class Weight:
    """Device copy of an int8 [N,K] weight + f32 [N] scales (one-time upload
    and repack into the MFMA fragment layout)."""

    def __init__(self, handle, N, K):
        self.h = handle
        self.N, self.K = int(N), int(K)

    @classmethod
    def from_host(cls, q: np.ndarray, scale, stream=None):
        """q: int8 [N,K]; scale: float32 [N], or raw bytes / uint8 array of
        4N bytes (e.g. an unaligned slice of a .sdcpp blob)."""
        lib = load_library()
        q = np.ascontiguousarray(q, np.int8)
        N, K = q.shape
        if isinstance(scale, (bytes, bytearray, memoryview)):
            sbuf = np.frombuffer(scale, np.uint8)
        else:
            sbuf = np.ascontiguousarray(scale)
        if sbuf.nbytes != 4 * N:
            raise ValueError("scale must hold N float32 values")
        h = ctypes.c_void_p()
        _check(lib.sdq_weight_upload(_ptr(q), _ptr(sbuf), N, K,
                                     _stream(stream) if stream is not None else None,
                                     ctypes.byref(h)))
        return cls(h, N, K)

    @classmethod
    def from_device(cls, q_dev, scale_dev, stream=None):
        c = _Args()
        lib = load_library()
        pq = c(q_dev, "q", "i8", (None, None))
        N, K = q_dev.shape
        ps = c(scale_dev, "scale", "f32", (N,))
        c.done()
        h = ctypes.c_void_p()
        _check(lib.sdq_weight_upload_device(pq, ps, N, K, _stream(stream), ctypes.byref(h)))
        return cls(h, N, K)

    def export(self):
        q = np.empty((self.N, self.K), np.int8)
        s = np.empty((self.N,), np.float32)
        _check(_lib.sdq_weight_export_host(self.h, _ptr(q), _ptr(s)))
        return q, s

    def free(self):
        if self.h is not None and self.h.value:
            _lib.sdq_weight_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # pragma: no cover - interpreter shutdown
            pass


def make_epilogue(kind="none", bias=None, gate=None, resid=None, gate_fma=True):
    e = Epilogue()
    e.kind = EPI_NAMES[kind] if isinstance(kind, str) else int(kind)
    e.gate_fma = 1 if gate_fma else 0
    e.bias = _ptr(bias)
    e.gate = _ptr(gate)
    e.resid = _ptr(resid)
    return e


def _epilogue_args(c, kind, M, N, out, bias, gate, resid, gate_fma, prefix=""):
    """make_epilogue for device tensors, every operand checked against
    [M, N] (out: int32 for the raw-accumulator kind, else float32); prefix
    names the operands in errors (e.g. "items[2].")."""
    k = EPI_NAMES[kind] if isinstance(kind, str) else int(kind)
    c(out, prefix + "out", "i32" if k == EPI_ACC else "f32", (M, N))
    e = Epilogue()
    e.kind = k
    e.gate_fma = 1 if gate_fma else 0
    e.bias = c(bias, prefix + "bias", "f32", (N,), optional=True)
    e.gate = c(gate, prefix + "gate", "f32", (N,), optional=True)
    e.resid = c(resid, prefix + "resid", "f32", (M, N), optional=True)
    return e


class WeightSrc(ctypes.Structure):
    _fields_ = [("nparts", ctypes.c_int), ("q", ctypes.c_void_p * 4), ("scale", ctypes.c_void_p * 4),
                ("rows", ctypes.c_int64 * 4), ("K", ctypes.c_int64)]


def upload_batch(sources, stream=None):
    """sources: list of lists of (q int8 [rows,K], scale f32 [rows] or raw bytes)
    host parts; returns one Weight per source (sdq_weight_upload_batch)."""
    load_library()
    n = len(sources)
    arr = (WeightSrc * max(n, 1))()
    keep = []
    for i, parts in enumerate(sources):
        arr[i].nparts = len(parts)
        arr[i].K = parts[0][0].shape[1]
        for p, (q, sc) in enumerate(parts):
            q = np.ascontiguousarray(q, np.int8)
            keep.append(q)
            arr[i].q[p] = q.ctypes.data
            if isinstance(sc, (bytes, bytearray, memoryview)):
                buf = (ctypes.c_char * len(sc)).from_buffer_copy(bytes(sc))
                keep.append(buf)
                arr[i].scale[p] = ctypes.addressof(buf)
            else:
                sc = np.ascontiguousarray(sc, np.float32)
                keep.append(sc)
                arr[i].scale[p] = sc.ctypes.data
            arr[i].rows[p] = q.shape[0]
    handles = (ctypes.c_void_p * max(n, 1))()
    _check(_lib.sdq_weight_upload_batch(arr, n, _stream(stream), handles))
    return [Weight(ctypes.c_void_p(handles[i]), sum(arr[i].rows[p] for p in range(arr[i].nparts)),
                   arr[i].K) for i in range(n)]


def _weight(w, name="w"):
    if not isinstance(w, Weight) or w.h is None or not w.h.value:
        raise _bad(f"{name}: not a live Weight")
    return w.h


class WeightFileSrc(ctypes.Structure):
    _fields_ = [("nparts", ctypes.c_int), ("q_off", ctypes.c_uint64 * 4),
                ("scale_off", ctypes.c_uint64 * 4), ("rows", ctypes.c_int64 * 4),
                ("K", ctypes.c_int64)]


def upload_file(path, sources, stream=None):
    """sources: list of lists of (q_offset, scale_offset, rows, K) parts inside the
    .sdcpp file `path` (absolute file offsets); one Weight per source, read with
    sequential file reads (sdq_weight_upload_file)."""
    load_library()
    n = len(sources)
    arr = (WeightFileSrc * max(n, 1))()
    for i, parts in enumerate(sources):
        arr[i].nparts = len(parts)
        arr[i].K = parts[0][3]
        for p, (qo, so, rows, _k) in enumerate(parts):
            arr[i].q_off[p], arr[i].scale_off[p], arr[i].rows[p] = qo, so, rows
    handles = (ctypes.c_void_p * max(n, 1))()
    _check(_lib.sdq_weight_upload_file(os.fsencode(path), arr, n, _stream(stream), handles))
    return [Weight(ctypes.c_void_p(handles[i]), sum(arr[i].rows[p] for p in range(arr[i].nparts)),
                   arr[i].K) for i in range(n)]


def qlinear(w: Weight, A, out, kind="none", bias=None, gate=None, resid=None, gate_fma=True,
            stream=None):
    """out = epilogue(qgemm(A, W) + bias) on device tensors (stream-ordered).
    A [M, K] and out [M, N] (int32 for kind "acc"), bias / gate [N], resid
    [M, N]; all checked before the launch (SdqError on a mismatch)."""
    c = _Args()
    h = _weight(w)
    pa = c(A, "A", "f32", (None, w.K))
    M = A.shape[0]
    e = _epilogue_args(c, kind, M, w.N, out, bias, gate, resid, gate_fma)
    c.done()
    _check(_lib.sdq_qlinear(h, pa, M, w.K, ctypes.byref(e), _ptr(out), _stream(stream)))
    return out


MAX_GROUP = 16  # SDQ_MAX_GROUP


def qlinear_group(items, stream=None):
    """Several independent Linears in one call (sdq_qlinear_group): the same
    results as qlinear on each item. items: dicts with keys w, A, out and
    optionally kind, bias, gate, resid, gate_fma (as qlinear's arguments)."""
    if len(items) > MAX_GROUP:
        raise _bad(f"at most {MAX_GROUP} items")
    c = _Args()
    arr = _group_items(c, items)
    c.done()
    _check(_lib.sdq_qlinear_group(arr, len(items), _stream(stream)))


def _group_items(c, items):
    """The GroupItem array of qlinear_group / qlinear_stack, every tensor
    checked by c."""
    arr = (GroupItem * max(1, len(items)))()
    for i, it in enumerate(items):
        w = it["w"]
        arr[i].w = _weight(w, f"items[{i}].w")
        arr[i].A = c(it["A"], f"items[{i}].A", "f32", (None, w.K))
        M = it["A"].shape[0]
        arr[i].M = M
        arr[i].epi = _epilogue_args(c, it.get("kind", "none"), M, w.N, it["out"], it.get("bias"),
                                    it.get("gate"), it.get("resid"), it.get("gate_fma", True),
                                    prefix=f"items[{i}].")
        arr[i].Y = c(it["out"], f"items[{i}].out", "i32" if arr[i].epi.kind == EPI_ACC else "f32",
                     (M, w.N))
    return arr


def qlinear_stack(items, ngroup, ffn=None, stream=None):
    """A block's linear stack from given inputs (sdq_qlinear_stack): the same
    results as qlinear_group(items[:ngroup]), then qlinear on each later item
    in order, then ffn(**ffn); every input quantized by one launch first.
    items: as for qlinear_group; ffn: dict with fc1, b1, fc2, b2, h, gate,
    hid, x and optionally gate_fma (as ffn's arguments), or None."""
    if len(items) > MAX_GROUP:
        raise _bad(f"at most {MAX_GROUP} items")
    c = _Args()
    arr = _group_items(c, items)
    f = None
    if ffn is not None:
        fc1, fc2 = ffn["fc1"], ffn["fc2"]
        M = ffn["h"].shape[0]
        f = FfnItem()
        f.fc1, f.fc2 = _weight(fc1, "fc1"), _weight(fc2, "fc2")
        f.b1 = c(ffn.get("b1"), "b1", "f32", (fc1.N,), optional=True)
        f.b2 = c(ffn.get("b2"), "b2", "f32", (fc2.N,), optional=True)
        f.h = c(ffn["h"], "h", "f32", (M, fc1.K))
        f.M = M
        f.gate = c(ffn["gate"], "gate", "f32", (fc2.N,))
        f.gate_fma = 1 if ffn.get("gate_fma", True) else 0
        f.hid = c(ffn["hid"], "hid", "f32", (M, fc1.N))
        f.x = c(ffn["x"], "x", "f32", (M, fc2.N))
    c.done()
    _check(_lib.sdq_qlinear_stack(arr, len(items), ngroup,
                                  ctypes.byref(f) if f is not None else None, _stream(stream)))


NOALLOC_SCRATCH_BYTES = 64 << 20  # SDQ_NOALLOC_SCRATCH_BYTES


def qlinear_noalloc(w: Weight, A, out, kind="none", bias=None, gate=None, resid=None,
                    gate_fma=True, stream=None):
    """qlinear without any device allocation (sdq_qlinear_noalloc: scratch in a
    static per-GPU array; calls that overlap on one GPU race)."""
    c = _Args()
    h = _weight(w)
    pa = c(A, "A", "f32", (None, w.K))
    M = A.shape[0]
    e = _epilogue_args(c, kind, M, w.N, out, bias, gate, resid, gate_fma)
    c.done()
    _check(_lib.sdq_qlinear_noalloc(h, pa, M, w.K, ctypes.byref(e), _ptr(out), _stream(stream)))
    return out


def qgemm(w: Weight, A, out, stream=None):
    c = _Args()
    h = _weight(w)
    pa = c(A, "A", "f32", (None, w.K))
    M = A.shape[0]
    po = c(out, "out", "f32", (M, w.N))
    c.done()
    _check(_lib.sdq_qgemm(h, pa, M, w.K, po, _stream(stream)))
    return out


def _ffn_args(c, fc1, b1, fc2, b2, M, gate, hid):
    if fc2.K != fc1.N or fc2.N != fc1.K:
        raise _bad(f"ffn: fc1 [{fc1.N},{fc1.K}] and fc2 [{fc2.N},{fc2.K}] do not chain")
    D, F = fc1.K, fc1.N
    return (c(b1, "b1", "f32", (F,), optional=True), c(b2, "b2", "f32", (D,), optional=True),
            c(gate, "gate", "f32", (D,)), c(hid, "hid", "f32", (M, F)))


def ffn(fc1: Weight, b1, fc2: Weight, b2, h, gate, hid, x, gate_fma=True, stream=None):
    """hid = gelu_tanh(mlin(h, fc1)); x = fma(mlin(hid, fc2), gate, x), in place
    (ovi_dit.cpp:218-221), device tensors, stream-ordered."""
    c = _Args()
    h1, h2 = _weight(fc1, "fc1"), _weight(fc2, "fc2")
    ph = c(h, "h", "f32", (None, fc1.K))
    M = h.shape[0]
    pb1, pb2, pg, phid = _ffn_args(c, fc1, b1, fc2, b2, M, gate, hid)
    px = c(x, "x", "f32", (M, fc1.K))
    c.done()
    _check(_lib.sdq_ffn(h1, pb1, h2, pb2, ph, M, pg, 1 if gate_fma else 0, phid, px,
                        _stream(stream)))
    return x


def qlinear_lnmod(w: Weight, x, out, shift, scale, eps=1e-6, kind="none", bias=None, gate=None,
                  resid=None, gate_fma=True, stream=None):
    """out = epilogue(qgemm(mod_rows(layernorm(x), shift, scale), W) + bias)."""
    c = _Args()
    hw = _weight(w)
    px = c(x, "x", "f32", (None, w.K))
    M, K = x.shape
    psh, psc = c(shift, "shift", "f32", (K,)), c(scale, "scale", "f32", (K,))
    e = _epilogue_args(c, kind, M, w.N, out, bias, gate, resid, gate_fma)
    c.done()
    _check(_lib.sdq_qlinear_lnmod(hw, px, M, K, psh, psc, eps, ctypes.byref(e), _ptr(out),
                                  _stream(stream)))
    return out


def ffn_lnmod(fc1: Weight, b1, fc2: Weight, b2, x, shift, scale, gate, hid, eps=1e-6,
              gate_fma=True, stream=None):
    """ffn_fwd (ovi_dit.cpp:214-222) with x the norm input and the residual."""
    c = _Args()
    h1, h2 = _weight(fc1, "fc1"), _weight(fc2, "fc2")
    px = c(x, "x", "f32", (None, fc1.K))
    M, D = x.shape
    pb1, pb2, pg, phid = _ffn_args(c, fc1, b1, fc2, b2, M, gate, hid)
    psh, psc = c(shift, "shift", "f32", (D,)), c(scale, "scale", "f32", (D,))
    c.done()
    _check(_lib.sdq_ffn_lnmod(h1, pb1, h2, pb2, px, M, psh, psc, eps, pg, 1 if gate_fma else 0,
                              phid, _stream(stream)))
    return x


def layernorm(x, y, w=None, b=None, eps=1e-6, stream=None):
    c = _Args()
    px = c(x, "x", "f32", (None, None))
    M, K = x.shape
    py = c(y, "y", "f32", (M, K))
    pw, pb = c(w, "w", "f32", (K,), optional=True), c(b, "b", "f32", (K,), optional=True)
    load_library()
    c.done()
    _check(_lib.sdq_layernorm(px, M, K, pw, pb, eps, py, _stream(stream)))
    return y


def linear_f32(x, w, out, bias=None, stream=None):
    """out = x . w (+ bias): the F32 branch of mlin (blk::linear -> sd::matmul,
    src/core/gemm.cpp:115-160), bit-exact. x [M,K], w [K,N] (the [in, out]
    layout lin() gives F32 weights), bias [N] or None, out [M,N]."""
    c = _Args()
    px = c(x, "x", "f32", (None, None))
    M, K = x.shape
    pw = c(w, "w", "f32", (K, None))
    N = w.shape[1]
    py = c(out, "out", "f32", (M, N))
    pb = c(bias, "bias", "f32", (N,), optional=True)
    load_library()
    c.done()
    _check(_lib.sdq_linear_f32(px, M, K, pw, N, pb, py, _stream(stream)))
    return out


def add_(x, y, stream=None):
    c = _Args()
    px = c(x, "x", "f32")
    py = c(y, "y", "f32", tuple(x.shape))
    load_library()
    c.done()
    _check(_lib.sdq_add(px, py, x.numel(), _stream(stream)))
    return x


def _cols(c, t, name, col, C):
    """Address of column `col` of a 2-D row-strided device tensor whose rows
    hold at least col + C floats."""
    c(t, name, "f32", contig=False)
    if col < 0 or col + C > t.shape[1]:
        raise _bad(f"{name}: columns [{col}, {col + C}) outside its {t.shape[1]} columns")
    return ctypes.c_void_p(t.data_ptr() + 4 * col)


def sdpa(q, k, v, out, heads, qcol=0, kcol=0, vcol=0, batch=1, stream=None):
    """out = attention(q, k, v) over `heads` heads of 128 columns, taken from
    column offsets qcol / kcol / vcol of the device tensors q, k, v (e.g. one
    q|k|v tensor passed three times); rows may be strided (stride(0)).
    batch > 1: that many sequences stacked along the rows, each attending to
    its own keys only (sdq_sdpa_batched)."""
    c = _Args()
    C = heads * 128
    pq, pk, pv = _cols(c, q, "q", qcol, C), _cols(c, k, "k", kcol, C), _cols(c, v, "v", vcol, C)
    po = _cols(c, out, "out", 0, C)
    if batch < 1 or q.shape[0] % batch or k.shape[0] % batch:
        raise _bad(f"sdpa: {q.shape[0]} query and {k.shape[0]} key rows do not split into "
                   f"{batch} sequences")
    Lq, Lk = q.shape[0] // batch, k.shape[0] // batch
    if v.shape[0] != k.shape[0] or out.shape[0] != q.shape[0]:
        raise _bad(f"sdpa: {q.shape[0]} queries, {k.shape[0]} keys, {v.shape[0]} values, "
                   f"{out.shape[0]} out rows")
    load_library()
    c.done()
    _check(_lib.sdq_sdpa_batched(pq, _ld(q), pk, _ld(k), pv, _ld(v), po, _ld(out), Lq, Lk, heads,
                                 128, batch, _stream(stream)))
    return out


def _rope_table(c, cs, L, name="cs"):
    if cs is None:
        return None, 0
    p = c(cs, name, "f32", (None, None, 2))
    if cs.shape[0] < L:
        raise _bad(f"{name}: {cs.shape[0]} rows of (cos, sin) pairs for {L} tokens")
    return p, int(cs.shape[1])


def rmsnorm_rope(x, C, w, heads, cs=None, eps=1e-6, col0=0, stream=None):
    """In place: columns [col0, col0+C) of every row of the device tensor x
    (rows may be strided) get rmsnorm(w, eps) then RoPE with the (cos, sin)
    table cs [>= L, nr, 2] (None: no rotation)."""
    c = _Args()
    p = _cols(c, x, "x", col0, C)
    L = x.shape[0]
    pw = c(w, "w", "f32", (C,), optional=True)
    pcs, nr = _rope_table(c, cs, L)
    load_library()
    c.done()
    _check(_lib.sdq_rmsnorm_rope(p, L, C, _ld(x), pw, eps, heads, pcs, nr, _stream(stream)))
    return x


class RmsSeg(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("L", ctypes.c_int64), ("ld", ctypes.c_int64),
                ("w", ctypes.c_void_p), ("cs", ctypes.c_void_p), ("nr", ctypes.c_int)]


def rmsnorm_rope_batch(segs, C, heads, eps=1e-6, stream=None):
    """sdq_rmsnorm_rope_batch: segs = [(x, col0, w, cs)], each as in
    rmsnorm_rope (x a device tensor whose rows hold the block at col0)."""
    c = _Args()
    arr = (RmsSeg * max(len(segs), 1))()
    for i, (x, col0, w, cs) in enumerate(segs):
        arr[i].x = _cols(c, x, f"segs[{i}].x", col0, C).value
        arr[i].L, arr[i].ld = x.shape[0], _ld(x)
        arr[i].w = c(w, f"segs[{i}].w", "f32", (C,), optional=True)
        arr[i].cs, arr[i].nr = _rope_table(c, cs, x.shape[0], f"segs[{i}].cs")
    load_library()
    c.done()
    _check(_lib.sdq_rmsnorm_rope_batch(arr, len(segs), C, heads, eps, _stream(stream)))


def qlinear_host(w: Weight, A: np.ndarray, kind="none", bias=None, gate=None, resid=None,
                 gate_fma=True):
    """Synchronous host-array variant (copies in and out)."""
    A = np.ascontiguousarray(A, np.float32)
    M, K = A.shape
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    gate = None if gate is None else np.ascontiguousarray(gate, np.float32)
    resid = None if resid is None else np.ascontiguousarray(resid, np.float32)
    out = np.empty((M, w.N), np.int32 if kind == "acc" else np.float32)
    e = make_epilogue(kind, bias, gate, resid, gate_fma)
    _check(_lib.sdq_qlinear_host(w.h, _ptr(A), M, K, ctypes.byref(e), _ptr(out)))
    return out


def act_quant(A, aq, asc, stream=None):
    c = _Args()
    pa = c(A, "A", "f32", (None, None))
    M, K = A.shape
    pq, ps = c(aq, "aq", "i8", (M, K)), c(asc, "as", "f32", (M,))
    load_library()
    c.done()
    _check(_lib.sdq_act_quant(pa, M, K, pq, ps, _stream(stream)))


def qlinear_plan(w: Weight, M: int, kind="none") -> list:
    """[(record name, first row, rows)] of the GEMM launches sdq_qlinear makes
    for M rows (sdq_qlinear_plan)."""
    p = GemmPlan()
    k = EPI_NAMES[kind] if isinstance(kind, str) else int(kind)
    _check(load_library().sdq_qlinear_plan(_weight(w), M, k, ctypes.byref(p)))
    return [(p.name[i].value.decode(), int(p.row0[i]), int(p.rows[i])) for i in range(p.nlaunch)]


def version() -> str:
    return load_library().sdq_version().decode()


def profile_begin():
    _check(load_library().sdq_profile_begin())


def profile_end() -> dict:
    """{kernel name: (launches, total device ms)} since profile_begin()."""
    recs = (KernelTime * 32)()
    n = ctypes.c_int()
    _check(_lib.sdq_profile_end(recs, 32, ctypes.byref(n)))
    return {recs[i].name.decode(): (recs[i].launches, recs[i].total_ms)
            for i in range(min(n.value, 32))}


def sync():
    _check(_lib.sdq_sync())


def stream_wait(waiter=None, signaler=None):
    """sdq_stream_wait: work enqueued on `waiter` from now on starts after the
    work already enqueued on `signaler` (torch streams, raw handles or None)."""
    _check(load_library().sdq_stream_wait(_stream(waiter), _stream(signaler)))


# ---- the DiT block linear stack (C++ host mirror, lib/libsd_host.so) ----
HOST_LIB_PATH = os.path.join(LIB_DIR, "libsd_host.so")
_host = None

# order of sd_dit_block_create's Linear array (include: host/sd/dit_block.h)
BLOCK_LINEARS = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "kf", "vf", "fc1", "fc2")


class Linear(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("out", ctypes.c_int64), ("in_", ctypes.c_int64)]


_BLOCK_PTRS = ("h_sa", "att", "gate_sa", "xq", "ctx", "tn", "xt", "h_ffn", "gate_ffn", "qkv", "cq",
               "ckv", "kvt", "hid", "x", "shift_sa", "scale_sa", "shift_ffn", "scale_ffn")


class BlockIO(ctypes.Structure):
    _fields_ = ([("M", ctypes.c_int64), ("Mc", ctypes.c_int64), ("Mt", ctypes.c_int64)] +
                [(n, ctypes.c_void_p) for n in _BLOCK_PTRS] + [("eps", ctypes.c_float)])


# fields of sd_dit_norms (host/sd/dit_block.h), in order
NORM_NAMES = ("sa_nq", "sa_nk", "ca_nq", "ca_nk", "ln3_w", "ln3_b", "nk_fusion", "pnf_w", "pnf_b")


class DitNorms(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in NORM_NAMES]


class BlockStep(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int64), ("Mc", ctypes.c_int64), ("Mt", ctypes.c_int64),
                ("heads", ctypes.c_int), ("eps", ctypes.c_float), ("x", ctypes.c_void_p),
                ("ctx", ctypes.c_void_p), ("target", ctypes.c_void_p), ("e", ctypes.c_void_p),
                ("cs", ctypes.c_void_p), ("nr", ctypes.c_int), ("cs_tgt", ctypes.c_void_p),
                ("nr_tgt", ctypes.c_int), ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t)]


SELF, CROSS_FFN, ALL = 1, 2, 3


def rope_table_3d(T, H, W, head_dim=128, theta=10000.0):
    """(cos, sin) table [T*H*W, n_rot, 2] of the reference's rope_freqs_3d
    (host library, sd_rope_table_3d)."""
    h = load_host_library()
    nr = h.sd_rope_table_3d(T, H, W, head_dim, theta, None)
    if nr < 0:
        raise ValueError("rope_table_3d: bad arguments")
    cs = np.empty((T * H * W, nr, 2), np.float32)
    if h.sd_rope_table_3d(T, H, W, head_dim, theta, _ptr(cs)) != nr:
        raise ValueError("rope_table_3d failed")
    return cs


def rope_table_1d(L, head_dim=128, theta=10000.0, scaling=1.0):
    """(cos, sin) table [L, n_rot, 2] of the reference's rope_freqs_1d."""
    h = load_host_library()
    nr = h.sd_rope_table_1d(L, head_dim, theta, scaling, None)
    if nr < 0:
        raise ValueError("rope_table_1d: bad arguments")
    cs = np.empty((L, nr, 2), np.float32)
    if h.sd_rope_table_1d(L, head_dim, theta, scaling, _ptr(cs)) != nr:
        raise ValueError("rope_table_1d failed")
    return cs


def load_host_library(path: str = HOST_LIB_PATH):
    """Load libsd_host.so (raises if it has not been built)."""
    global _host
    if _host is not None:
        return _host
    load_library()  # libsdq first (libsd_host links it)
    if not os.path.exists(path):
        raise RuntimeError(f"libsd_host.so not built: {path} (run __graft_entry__.build())")
    h = ctypes.CDLL(path)
    h.sd_dit_last_error.restype = ctypes.c_char_p
    h.sd_dit_last_error.argtypes = []
    h.sd_dit_block_create.restype = ctypes.c_int
    h.sd_dit_block_create.argtypes = [ctypes.POINTER(Linear), ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_void_p)]
    h.sd_dit_block_create_many.restype = ctypes.c_int
    h.sd_dit_block_create_many.argtypes = [ctypes.POINTER(Linear), ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_void_p)]
    h.sd_dit_block_forward.restype = ctypes.c_int
    h.sd_dit_block_forward.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockIO), ctypes.c_void_p]
    h.sd_dit_block_forward_pair.restype = ctypes.c_int
    h.sd_dit_block_forward_pair.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockIO),
                                            ctypes.c_void_p, ctypes.POINTER(BlockIO),
                                            ctypes.c_void_p]
    h.sd_dit_block_forward_pair2.restype = ctypes.c_int
    h.sd_dit_block_forward_pair2.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockIO),
                                             ctypes.c_void_p, ctypes.POINTER(BlockIO),
                                             ctypes.c_void_p, ctypes.c_void_p]
    h.sd_dit_block_set_norms.restype = ctypes.c_int
    h.sd_dit_block_set_norms.argtypes = [ctypes.c_void_p, ctypes.POINTER(DitNorms)]
    h.sd_dit_block_workspace_bytes.restype = ctypes.c_size_t
    h.sd_dit_block_workspace_bytes.argtypes = [ctypes.c_void_p, _i64, _i64, _i64]
    h.sd_dit_block_step_forward.restype = ctypes.c_int
    h.sd_dit_block_step_forward.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockStep),
                                            ctypes.c_int, ctypes.c_void_p]
    h.sd_dit_block_step_forward_batched.restype = ctypes.c_int
    h.sd_dit_block_step_forward_batched.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockStep),
                                                    ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    h.sd_dit_block_step_ops.restype = ctypes.c_double
    h.sd_dit_block_step_ops.argtypes = [ctypes.c_void_p, _i64, _i64, _i64]
    for f in (h.sd_rope_table_3d, h.sd_rope_table_1d):
        f.restype = ctypes.c_int
    h.sd_rope_table_3d.argtypes = [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_void_p]
    h.sd_rope_table_1d.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_void_p]
    h.sd_dit_block_set_modulation.restype = ctypes.c_int
    h.sd_dit_block_set_modulation.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    h.sd_dit_block_modulation.restype = ctypes.c_int
    h.sd_dit_block_modulation.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_void_p]
    h.sd_dit_blocks_from_pack.restype = ctypes.c_int
    h.sd_dit_blocks_from_pack.argtypes = [ctypes.c_char_p, ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_int), ctypes.c_int, _i64, _i64,
                                          ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_void_p)]
    h.sd_dit_block_free.restype = ctypes.c_int
    h.sd_dit_block_free.argtypes = [ctypes.c_void_p]
    h.sd_dit_block_ops.restype = ctypes.c_double
    h.sd_dit_block_ops.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_int64]
    _host = h
    return h


def _hcheck(rc):
    if rc != OK:
        raise SdqError(rc, _host.sd_dit_last_error().decode(errors="replace"))


class DitBlock:
    """One DiT block's int8 Linears on the GPU (sd::gpu::DitBlock).

    lin: {name: (q int8 [out,in], scale f32 [out], bias f32 [out])} for the
    names in BLOCK_LINEARS (kf/vf only with fusion); numpy arrays (host) or
    torch device tensors (device)."""

    def __init__(self, lin: dict, fusion: bool):
        h = load_host_library()
        arr = (Linear * len(BLOCK_LINEARS))()
        on_device = None
        keep = []
        for i, name in enumerate(BLOCK_LINEARS):
            if name not in lin:
                if name in ("kf", "vf") and not fusion:
                    continue
                raise ValueError(f"DitBlock: missing Linear {name}")
            q, s, b = lin[name]
            dev = not isinstance(q, np.ndarray)
            if on_device is None:
                on_device = dev
            elif on_device != dev:
                raise ValueError("DitBlock: mix of host and device arrays")
            if not dev:
                q = np.ascontiguousarray(q, np.int8)
                s = np.ascontiguousarray(s, np.float32)
                b = None if b is None else np.ascontiguousarray(b, np.float32)
            keep += [q, s, b]
            arr[i].w, arr[i].scale, arr[i].bias = _ptr(q), _ptr(s), _ptr(b)
            arr[i].out, arr[i].in_ = q.shape
        self.h = ctypes.c_void_p()
        _hcheck(h.sd_dit_block_create(arr, 1 if fusion else 0, 1 if on_device else 0,
                                      ctypes.byref(self.h)))
        self.fusion = fusion
        self.dim, self.ffn_dim = int(arr[0].in_), int(arr[10].out)

    @classmethod
    def create_many(cls, lins, fusion: bool):
        """Blocks from host arrays in one streamed weight upload
        (sd_dit_block_create_many); lins: list of the dicts __init__ takes."""
        h = load_host_library()
        n = len(lins)
        arr = (Linear * (len(BLOCK_LINEARS) * max(n, 1)))()
        keep = []
        for b, lin in enumerate(lins):
            for i, name in enumerate(BLOCK_LINEARS):
                if name not in lin:
                    if name in ("kf", "vf") and not fusion:
                        continue
                    raise ValueError(f"DitBlock: missing Linear {name}")
                q, s, bias = (None if a is None else np.ascontiguousarray(a) for a in lin[name])
                keep += [q, s, bias]
                j = b * len(BLOCK_LINEARS) + i
                arr[j].w, arr[j].scale, arr[j].bias = _ptr(q), _ptr(s), _ptr(bias)
                arr[j].out, arr[j].in_ = q.shape
        handles = (ctypes.c_void_p * max(n, 1))()
        _hcheck(h.sd_dit_block_create_many(arr, n, 1 if fusion else 0, handles))
        out = []
        for b in range(n):
            blk = cls.__new__(cls)
            blk.h = ctypes.c_void_p(handles[b])
            blk.fusion = fusion
            blk.dim, blk.ffn_dim = int(arr[0].in_), int(arr[10].out)
            out.append(blk)
        return out

    def _io_shapes(self, M, Mc, Mt):
        d, f = self.dim, self.ffn_dim
        return {"h_sa": (M, d), "att": (M, d), "gate_sa": (d,), "xq": (M, d), "ctx": (Mc, d),
                "tn": (Mt, d), "xt": (M, d), "h_ffn": (M, d), "gate_ffn": (d,),
                "qkv": (M, 3 * d), "cq": (M, d), "ckv": (Mc, 2 * d), "kvt": (Mt, 2 * d),
                "hid": (M, f), "x": (M, d), "shift_sa": (d,), "scale_sa": (d,),
                "shift_ffn": (d,), "scale_ffn": (d,)}

    @classmethod
    def from_pack(cls, path, prefix, layers, dim, ffn_dim, fusion, file_reads=True):
        """Blocks `layers` of backbone `prefix` ("video_model." / "audio_model.")
        of a .sdcpp file, whole: Linears, norms and modulation bias, with
        OviDit::load_impl's names and checks (sd_dit_blocks_from_pack);
        file_reads: sequential file reads (else load_sdcpp's mapping)."""
        h = load_host_library()
        n = len(layers)
        arr = (ctypes.c_int * max(n, 1))(*layers)
        handles = (ctypes.c_void_p * max(n, 1))()
        _hcheck(h.sd_dit_blocks_from_pack(os.fsencode(path), prefix.encode(), arr, n, dim,
                                          ffn_dim, 1 if fusion else 0, 1 if file_reads else 0,
                                          handles))
        out = []
        for b in range(n):
            blk = cls.__new__(cls)
            blk.h = ctypes.c_void_p(handles[b])
            blk.fusion, blk.dim, blk.ffn_dim = fusion, int(dim), int(ffn_dim)
            out.append(blk)
        return out

    def set_modulation(self, mod):
        """mod: host float32 [6, dim] (or [1, 6, dim]), modulation.modulation."""
        m = np.ascontiguousarray(mod, np.float32).reshape(6, self.dim)
        _hcheck(_host.sd_dit_block_set_modulation(self.h, _ptr(m)))

    def modulation(self, t6, e, stream=None):
        """e = t6 + the block's modulation bias (device [6, dim] tensors)."""
        c = _Args()
        pt = c(t6, "t6", "f32", (6, self.dim))
        pe = c(e, "e", "f32", (6, self.dim))
        c.done()
        _hcheck(_host.sd_dit_block_modulation(self.h, pt, pe, _stream(stream)))
        return e

    def _block_io(self, c, io):
        b = BlockIO()
        b.M, b.Mc, b.Mt = int(io.get("M", 0)), int(io.get("Mc", 0)), int(io.get("Mt", 0))
        shapes = self._io_shapes(b.M, b.Mc, b.Mt)
        for name in _BLOCK_PTRS:
            t = io.get(name)
            if t is not None and shapes[name][0] == 0:
                t = None  # a fusion input of a call without target rows is not read
            setattr(b, name, c(t, name, "f32", shapes[name], optional=True))
        b.eps = float(io.get("eps", 1e-6))
        return b

    def forward(self, stream=None, **io):
        """io: M, Mc, Mt and the device tensors named in BlockIO; each tensor
        given is checked against its [rows, cols] before the launch."""
        c = _Args()
        b = self._block_io(c, io)
        c.done()
        _hcheck(_host.sd_dit_block_forward(self.h, ctypes.byref(b), _stream(stream)))

    def forward_pair(self, other, io, io_other, stream=None, stream2=None):
        """forward(**io) on this block and forward(**io_other) on `other` (two
        blocks with independent inputs, e.g. the video and audio blocks of a
        twin layer), their attention Linears grouped (sd_dit_block_forward_pair);
        with stream2, `other`'s Linears and this block's text / fusion k|v run
        there beside this block's own (sd_dit_block_forward_pair2, forked from
        and joined into stream)."""
        c = _Args()
        a, b = self._block_io(c, io), other._block_io(c, io_other)
        c.done()
        if stream2 is None:
            _hcheck(_host.sd_dit_block_forward_pair(self.h, ctypes.byref(a), other.h,
                                                    ctypes.byref(b), _stream(stream)))
        else:
            _hcheck(_host.sd_dit_block_forward_pair2(self.h, ctypes.byref(a), other.h,
                                                     ctypes.byref(b), _stream(stream),
                                                     _stream(stream2)))

    def ops(self, M, Mc=0, Mt=0) -> float:
        return _host.sd_dit_block_ops(self.h, M, Mc, Mt)

    def set_norms(self, norms: dict):
        """norms: {NORM_NAMES entry: host float32 [dim]} (sd_dit_block_set_norms)."""
        n = DitNorms()
        keep = []
        for name in NORM_NAMES:
            a = norms.get(name)
            if a is not None:
                a = np.ascontiguousarray(a, np.float32)
                keep.append(a)
            setattr(n, name, _ptr(a))
        _hcheck(_host.sd_dit_block_set_norms(self.h, ctypes.byref(n)))

    def workspace_bytes(self, M, Mc, Mt=0) -> int:
        return _host.sd_dit_block_workspace_bytes(self.h, M, Mc, Mt)

    def step_ops(self, M, Mc, Mt=0) -> float:
        return _host.sd_dit_block_step_ops(self.h, M, Mc, Mt)

    def step(self, x, ctx, e, heads, cs=None, target=None, cs_tgt=None, ws=None, phases=ALL,
             eps=1e-6, stream=None, batch=1):
        """The whole block on device tensors (sd_dit_block_step_forward): x
        [M,dim] in place, ctx [Mc,dim], e [6,dim], cs [M,nr,2] (RoPE table on
        the device), target [Mt,dim] and cs_tgt for fusion blocks; ws a device
        byte tensor of workspace_bytes (allocated here when None). batch > 1:
        that many sequences stacked along the rows of x, ctx, target, cs and
        cs_tgt (sd_dit_block_step_forward_batched)."""
        c = _Args()
        import torch

        d = self.dim
        st = BlockStep()
        st.x = c(x, "x", "f32", (None, d))
        st.ctx = c(ctx, "ctx", "f32", (None, d))
        st.target = c(target, "target", "f32", (None, d), optional=True)
        rows = (x.shape[0], ctx.shape[0], 0 if target is None else target.shape[0])
        if batch < 1 or any(r % batch for r in rows):
            raise _bad(f"step: rows {rows} of x, ctx, target do not split into {batch} sequences")
        st.M, st.Mc, st.Mt = (r // batch for r in rows)
        st.heads, st.eps = heads, eps
        st.e = c(e, "e", "f32", (6, d))
        st.cs, st.nr = _rope_table(c, cs, batch * st.M)
        st.cs_tgt, st.nr_tgt = _rope_table(c, cs_tgt, batch * st.Mt, "cs_tgt")
        need = self.workspace_bytes(batch * st.M, batch * st.Mc, batch * st.Mt)
        if ws is None:
            if stream is not None:
                # a workspace allocated here would be freed on return while
                # the side stream still uses it
                raise ValueError("DitBlock.step: pass ws when running on a given stream")
            ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        st.ws = c(ws, "ws", "u8")
        st.ws_bytes = ws.numel()
        if st.ws_bytes < need:
            raise _bad(f"ws: workspace too small ({st.ws_bytes} bytes, the block needs {need})")
        c.done()
        _hcheck(_host.sd_dit_block_step_forward_batched(self.h, ctypes.byref(st), batch, phases,
                                                        _stream(stream)))
        return x

    def free(self):
        if self.h is not None and self.h.value:
            _host.sd_dit_block_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # pragma: no cover - interpreter shutdown
            pass
