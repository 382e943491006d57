"""Argument checks of the Python binding (CPU: nothing is launched).

The C ABI takes bare device pointers and cannot see a host buffer, a wrong
element type, a strided view or a short output; the binding must turn each of
those into SdqError(ERR_INVALID) before any call reaches the library, because
on the GPU they would become out-of-bounds addresses. These tests drive every
device-pointer wrapper with such arguments on the CPU: the check fires before
the library is called (a live weight handle is faked; the library is never
entered), so no GPU is needed.
"""
import ctypes

import pytest

torch = pytest.importorskip("torch")

import sdq  # noqa: E402


class _FakeWeight(sdq.Weight):
    """A Weight with a non-null handle value that is never dereferenced: the
    checks run before the handle is used, and it is never freed."""

    def free(self):
        self.h = None


class _FakeBlock(sdq.DitBlock):
    def free(self):
        self.h = None


def _fake_weight(N, K):
    return _FakeWeight(ctypes.c_void_p(0x1000), N, K)


@pytest.fixture(autouse=True)
def _no_library_calls(monkeypatch):
    """Fail the test if a wrapper reaches the library despite a bad argument."""
    class Trap:
        def __getattr__(self, name):
            raise AssertionError(f"library entered ({name}) with a bad argument")
    monkeypatch.setattr(sdq, "_lib", Trap())
    monkeypatch.setattr(sdq, "load_library", lambda *a, **k: None)
    yield


def _raises(match, fn, *a, **k):
    with pytest.raises(sdq.SdqError, match=match) as ei:
        fn(*a, **k)
    assert ei.value.code == sdq.ERR_INVALID


def test_qlinear_rejects_host_tensors():
    w = _fake_weight(16, 32)
    A = torch.zeros((4, 32))
    Y = torch.zeros((4, 16))
    _raises("A: must be on the GPU", sdq.qlinear, w, A, Y)


def test_qlinear_rejects_short_output():
    w = _fake_weight(16, 32)
    _raises(r"out: shape \(4, 15\)", sdq.qlinear, w, torch.zeros((4, 32)), torch.zeros((4, 15)))
    _raises(r"out: shape \(3, 16\)", sdq.qlinear, w, torch.zeros((4, 32)), torch.zeros((3, 16)))
    _raises(r"out: shape \(64,\)", sdq.qlinear, w, torch.zeros((4, 32)), torch.zeros(64))


def test_qlinear_rejects_non_contiguous_input():
    w = _fake_weight(16, 32)
    A = torch.zeros((32, 4)).t()  # [4, 32], column-major
    _raises("A: must be contiguous", sdq.qlinear, w, A, torch.zeros((4, 16)))


def test_qlinear_rejects_wrong_k_dtype_and_operands():
    w = _fake_weight(16, 32)
    A, Y = torch.zeros((4, 32)), torch.zeros((4, 16))
    _raises(r"A: shape \(4, 31\)", sdq.qlinear, w, torch.zeros((4, 31)), Y)
    _raises("A: dtype torch.float64", sdq.qlinear, w, A.double(), Y)
    _raises("out: dtype torch.float32, expected torch.int32", sdq.qlinear, w, A, Y, kind="acc")
    _raises(r"bias: shape \(15,\)", sdq.qlinear, w, A, Y, bias=torch.zeros(15))
    _raises(r"gate: shape \(8,\)", sdq.qlinear, w, A, Y, kind="gated", gate=torch.zeros(8),
            resid=Y)
    _raises(r"resid: shape \(2, 16\)", sdq.qlinear, w, A, Y, kind="resid",
            resid=torch.zeros((2, 16)))
    _raises("expected a torch device tensor", sdq.qlinear, w, A.numpy(), Y)
    dead = _FakeWeight(None, 16, 32)
    _raises("not a live Weight", sdq.qlinear, dead, A, Y)


def test_qgemm_and_act_quant_shapes():
    w = _fake_weight(16, 32)
    _raises(r"out: shape \(4, 8\)", sdq.qgemm, w, torch.zeros((4, 32)), torch.zeros((4, 8)))
    A = torch.zeros((4, 32))
    _raises(r"aq: shape \(4, 16\)", sdq.act_quant, A, torch.zeros((4, 16), dtype=torch.int8),
            torch.zeros(4))
    _raises("aq: dtype torch.uint8", sdq.act_quant, A, torch.zeros((4, 32), dtype=torch.uint8),
            torch.zeros(4))
    _raises(r"as: shape \(3,\)", sdq.act_quant, A, torch.zeros((4, 32), dtype=torch.int8),
            torch.zeros(3))


def test_ffn_shapes():
    fc1, fc2 = _fake_weight(64, 16), _fake_weight(16, 64)
    h, x, g = torch.zeros((4, 16)), torch.zeros((4, 16)), torch.zeros(16)
    _raises(r"hid: shape \(4, 63\)", sdq.ffn, fc1, None, fc2, None, h, g, torch.zeros((4, 63)), x)
    _raises("do not chain", sdq.ffn, fc1, None, _fake_weight(16, 32), None, h, g,
            torch.zeros((4, 64)), x)
    _raises(r"x: shape \(5, 16\)", sdq.ffn, fc1, None, fc2, None, h, g, torch.zeros((4, 64)),
            torch.zeros((5, 16)))
    _raises(r"shift: shape \(8,\)", sdq.ffn_lnmod, fc1, None, fc2, None, x, torch.zeros(8),
            torch.zeros(16), g, torch.zeros((4, 64)))


def test_sdpa_column_bounds_and_rows():
    qkv = torch.zeros((8, 3 * 256))
    out = torch.zeros((8, 256))
    # k block at column 256 + 2 heads of 128 = 512 <= 768: fine; v at 600 is not
    _raises(r"v: columns \[600, 856\)", sdq.sdpa, qkv, qkv, qkv, out, 2, 0, 256, 600)
    _raises(r"out: columns \[0, 256\)", sdq.sdpa, qkv, qkv, qkv, torch.zeros((8, 128)), 2, 0, 256,
            512)
    kv = torch.zeros((5, 512))
    _raises("5 keys, 4 values", sdq.sdpa, qkv, kv, kv[:4], out, 2, 0, 0, 256)
    # strided rows are accepted by the checks (they reach the device check)
    _raises("q: must be on the GPU", sdq.sdpa, qkv[:, 256:], qkv, qkv, out, 2)
    _raises("must be 2-D with contiguous rows", sdq.sdpa, qkv[:, ::2], qkv, qkv, out, 1)


def test_rmsnorm_rope_tables_and_columns():
    qkv = torch.zeros((10, 768))
    w = torch.ones(256)
    cs = torch.zeros((10, 64, 2))
    _raises(r"x: columns \[600, 856\)", sdq.rmsnorm_rope, qkv, 256, w, 2, cs, col0=600)
    _raises("cs: 9 rows of", sdq.rmsnorm_rope, qkv, 256, w, 2, cs[:9])
    _raises(r"w: shape \(255,\)", sdq.rmsnorm_rope, qkv, 256, torch.ones(255), 2, cs)
    _raises(r"cs: shape \(10, 64, 3\)", sdq.rmsnorm_rope, qkv, 256, w, 2,
            torch.zeros((10, 64, 3)))
    _raises("segs.1..cs: 9 rows", sdq.rmsnorm_rope_batch,
            [(qkv, 0, w, cs), (qkv, 256, w, cs[:9])], 256, 2)


def test_layernorm_and_add_shapes():
    x = torch.zeros((4, 32))
    _raises(r"y: shape \(4, 31\)", sdq.layernorm, x, torch.zeros((4, 31)))
    _raises(r"w: shape \(31,\)", sdq.layernorm, x, x, torch.zeros(31))
    _raises(r"y: shape \(4, 16\)", sdq.add_, x, torch.zeros((4, 16)))


def test_block_step_argument_checks():
    blk = _FakeBlock.__new__(_FakeBlock)
    blk.h, blk.fusion, blk.dim, blk.ffn_dim = ctypes.c_void_p(0x1000), True, 256, 512
    blk.workspace_bytes = lambda M, Mc, Mt=0: 1 << 20
    x, ctx, e = torch.zeros((8, 256)), torch.zeros((4, 256)), torch.zeros((6, 256))
    _raises(r"x: shape \(8, 255\)", blk.step, torch.zeros((8, 255)), ctx, e, 2)
    _raises(r"e: shape \(5, 256\)", blk.step, x, ctx, torch.zeros((5, 256)), 2)
    _raises("cs: 7 rows", blk.step, x, ctx, e, 2, cs=torch.zeros((7, 64, 2)))
    _raises("cs_tgt: 2 rows", blk.step, x, ctx, e, 2, cs=torch.zeros((8, 64, 2)),
            target=torch.zeros((3, 256)), cs_tgt=torch.zeros((2, 22, 2)))
    _raises("workspace too small", blk.step, x, ctx, e, 2, ws=torch.zeros(16, dtype=torch.uint8))
    io = dict(M=8, Mc=4, Mt=0, h_sa=x, att=x, gate_sa=torch.zeros(256), xq=x, ctx=ctx, xt=x,
              h_ffn=x, gate_ffn=torch.zeros(256), qkv=torch.zeros((8, 767)))
    _raises(r"qkv: shape \(8, 767\)", blk.forward, **io)


def test_linear_f32_checks():
    x, w, y = torch.zeros((4, 32)), torch.zeros((32, 20)), torch.zeros((4, 20))
    _raises("x: must be on the GPU", sdq.linear_f32, x, w, y)
    _raises(r"w: shape \(31, 20\)", sdq.linear_f32, x, torch.zeros((31, 20)), y)
    _raises(r"out: shape \(4, 19\)", sdq.linear_f32, x, w, torch.zeros((4, 19)))
    _raises(r"bias: shape \(19,\)", sdq.linear_f32, x, w, y, bias=torch.zeros(19))
    _raises("x: dtype", sdq.linear_f32, x.double(), w, y)
    _raises("w: must be contiguous", sdq.linear_f32, x, torch.zeros((20, 32)).t(), y)


def test_group_and_stack_item_checks():
    wa, wb = _fake_weight(16, 32), _fake_weight(24, 32)
    good = [dict(w=wa, A=torch.zeros((4, 32)), out=torch.zeros((4, 16))),
            dict(w=wb, A=torch.zeros((6, 32)), out=torch.zeros((6, 24)), kind="gated",
                 bias=torch.zeros(24), gate=torch.zeros(24), resid=torch.zeros((6, 24)))]
    for fn, extra in ((sdq.qlinear_group, ()), (sdq.qlinear_stack, (1,))):
        _raises(r"items\[0\]\.A: must be on the GPU", fn, good, *extra)
        bad = [dict(good[0], A=torch.zeros((4, 31))), good[1]]
        _raises(r"items\[0\]\.A: shape \(4, 31\)", fn, bad, *extra)
        bad = [good[0], dict(good[1], out=torch.zeros((6, 23)))]
        _raises(r"items\[1\]\.out: shape \(6, 23\)", fn, bad, *extra)
        bad = [good[0], dict(good[1], resid=torch.zeros((5, 24)))]
        _raises(r"items\[1\]\.resid: shape \(5, 24\)", fn, bad, *extra)
        _raises("at most 16 items", fn, good * 9, *extra)


def test_stack_ffn_checks():
    fc1, fc2 = _fake_weight(64, 32), _fake_weight(32, 64)
    M = 6
    ffn = dict(fc1=fc1, fc2=fc2, b1=torch.zeros(64), b2=torch.zeros(32), h=torch.zeros((M, 32)),
               gate=torch.zeros(32), hid=torch.zeros((M, 64)), x=torch.zeros((M, 32)))
    _raises("b1: must be on the GPU", sdq.qlinear_stack, [], 0, ffn)
    _raises(r"h: shape \(6, 31\)", sdq.qlinear_stack, [], 0, dict(ffn, h=torch.zeros((M, 31))))
    _raises(r"hid: shape \(6, 63\)", sdq.qlinear_stack, [], 0, dict(ffn, hid=torch.zeros((M, 63))))
    _raises(r"x: shape \(5, 32\)", sdq.qlinear_stack, [], 0, dict(ffn, x=torch.zeros((5, 32))))
    _raises(r"gate: shape \(31,\)", sdq.qlinear_stack, [], 0, dict(ffn, gate=torch.zeros(31)))
    _raises(r"b2: shape \(33,\)", sdq.qlinear_stack, [], 0, dict(ffn, b2=torch.zeros(33)))
