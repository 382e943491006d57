"""sdq_ffn (ovi_dit.cpp:214-222: fc1 -> GELU -> fc2 -> gated residual) on the
GPU. fc1's epilogue writes the row maxima of the hidden state and fc2's
quantizer uses them instead of its own max pass, so every shape class of
that hand-off is covered: few long rows (the split quantizer's second
kernel alone, 2 and 4 fragment groups per item), rows that fit the
register cache, many rows (the single quantizer with given maxima), and
M <= 64 (fc1 on the skinny kernel, which writes no maxima: fc2 quantizes
from scratch). The results must equal the two separate sdq_qlinear calls
bit for bit (hid and x), and x must equal the oracle's gated fc2 applied to
the GPU's own hidden state."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _lin(oracle, out, inp, seed, zero_bias=False):
    W = oracle.randn(out * inp, seed).reshape(out, inp) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    b = np.zeros(out, np.float32) if zero_bias else oracle.randn(out, seed + 1) * np.float32(0.01)
    return q, s, b


@pytest.mark.parametrize("M,D,F,zero_bias", [
    (157, 3072, 14336, False),   # audio tokens: split emit, 2 groups per item
    (768, 3072, 14336, False),   # config 2: split emit, 4 groups per item
    (300, 512, 1408, True),      # short hidden rows: single quantizer, given maxima
    (40, 512, 1408, False),      # M <= 64: skinny fc1, fc2 quantizes from scratch
    (4500, 256, 3328, False),    # many rows: single quantizer, given maxima
])
def test_ffn_matches_two_linears_and_oracle(sdq_dev, oracle, M, D, F, zero_bias):
    import torch

    import sdq

    print(f"[ffn] M={M} D={D} F={F} zero_bias={zero_bias}", flush=True)
    q1, s1, b1 = _lin(oracle, F, D, 10 + M, zero_bias)
    q2, s2, b2 = _lin(oracle, D, F, 20 + M)
    h = oracle.randn(M * D, 30 + M).reshape(M, D)
    h[3] = 0.0  # with zero bias: an all-zero hidden row (scale 1)
    h[5] *= np.float32(1e4)
    x0 = oracle.randn(M * D, 40 + M).reshape(M, D)
    gate = oracle.randn(D, 50 + M)
    w1, w2 = sdq.Weight.from_host(q1, s1), sdq.Weight.from_host(q2, s2)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    h_d, g_d, b1_d, b2_d = t(h), t(gate), t(b1), t(b2)
    hid = torch.empty((M, F), device=sdq_dev)
    x = t(x0)
    sdq.ffn(w1, b1_d, w2, b2_d, h_d, g_d, hid, x)
    hid2 = torch.empty((M, F), device=sdq_dev)
    x2 = t(x0)
    sdq.qlinear(w1, h_d, hid2, kind="gelu", bias=b1_d)
    sdq.qlinear(w2, hid2, x2, kind="gated", bias=b2_d, gate=g_d, resid=x2)
    torch.cuda.synchronize()
    hid_c = hid.cpu().numpy()
    assert_bitexact(hid_c, hid2.cpu().numpy(), "hid vs two calls")
    assert_bitexact(x.cpu().numpy(), x2.cpu().numpy(), "x vs two calls")
    if zero_bias:
        assert not hid_c[3].any()
    rows = np.unique(np.r_[0, 3, 5, np.arange(0, M, max(1, M // 64)), M - 1])
    want_h = oracle.linear(h[rows], q1, s1, bias=b1, epilogue="gelu")
    err = np.abs(hid_c[rows].astype(np.float64) - want_h.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want_h))), float(err.max())
    want_x = oracle.linear(hid_c[rows], q2, s2, bias=b2, epilogue="gated", gate=gate,
                           resid=x0[rows])
    assert_bitexact(x.cpu().numpy()[rows], want_x, "x vs oracle")


def test_ffn_errors(sdq_dev, oracle):
    import torch

    import sdq

    q1, s1, b1 = _lin(oracle, 256, 64, 1)
    q2, s2, b2 = _lin(oracle, 64, 128, 2)
    w1, w2 = sdq.Weight.from_host(q1, s1), sdq.Weight.from_host(q2, s2)
    h = torch.zeros((8, 64), device=sdq_dev)
    hid = torch.empty((8, 256), device=sdq_dev)
    x = torch.zeros((8, 64), device=sdq_dev)
    g = torch.ones(64, device=sdq_dev)
    with pytest.raises(sdq.SdqError, match="do not chain"):
        sdq.ffn(w1, None, w2, None, h, g, hid, x)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rc = sdq._lib.sdq_ffn(w1.h, None, w2.h, None, P(h), 8, P(g), 1, P(hid), P(x), None)
    assert rc == sdq.ERR_INVALID and b"need fc1" in sdq._lib.sdq_last_error()
    w3 = sdq.Weight.from_host(*_lin(oracle, 64, 256, 3)[:2])
    with pytest.raises(sdq.SdqError, match="gate: required"):
        sdq.ffn(w1, None, w3, None, h, None, hid, x)
    rc = sdq._lib.sdq_ffn(w1.h, None, w3.h, None, P(h), 8, None, 1, P(hid), P(x), None)
    assert rc == sdq.ERR_INVALID and b"null gate" in sdq._lib.sdq_last_error()
