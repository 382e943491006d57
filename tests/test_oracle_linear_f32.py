"""Pins of the oracle's fp32 Linear (orc_linear_f32), the F32 branch of mlin
(src/model/ovi_dit.cpp:80-82 -> blk::linear -> sd::matmul,
src/core/gemm.cpp:115-160), before it serves as the GPU's checker:

* the reference build's own matmul (oracle/_ref) bit for bit, live, on
  ragged shapes and special values;
* committed outputs of the reference build (tests/golden/ref_linear_f32.npz)
  without the reference sources;
* exact rational arithmetic: each output is the chain c = fma(x_k, w_k, c)
  from +0 in k order, every step rounded once to float32 (then + bias). The
  inputs are chosen so that the plausible mistakes (a separate multiply and
  add, another summation order, a dropped last term) give different bits,
  and the test checks that they do;
* exact integer dot products where every partial sum is an integer below
  2^24 (no rounding anywhere)."""
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import assert_bitexact

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _f32_round(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32, ties to even
    (subnormals included; |q| < 2^128)."""
    if q == 0:
        return np.float32(0.0)
    neg = q < 0
    a = -q if neg else q
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp_e = max(e - 23, -149)
    scaled = a / (Fraction(2) ** ulp_e)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = np.float32(float(n) * 2.0 ** ulp_e)
    return np.float32(-v) if neg else v


def _fma_exact(a, b, c) -> np.float32:
    """fmaf(a, b, c): the exact a*b + c rounded once (signed zero as IEEE
    754 addition: an exact zero sum is +0 unless both terms are -0)."""
    a, b, c = np.float32(a), np.float32(b), np.float32(c)
    q = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if q == 0:
        prod_neg = np.signbit(a) != np.signbit(b)
        both_neg = prod_neg and np.signbit(c)
        return np.float32(-0.0) if both_neg else np.float32(0.0)
    return _f32_round(q)


def _chain(x, w, bias, order=None, fused=True, drop_last=False):
    M, K = x.shape
    N = w.shape[1]
    ks = list(range(K)) if order is None else list(order)
    if drop_last:
        ks = ks[:-1]
    y = np.empty((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            c = np.float32(0.0)
            for k in ks:
                if fused:
                    c = _fma_exact(x[i, k], w[k, j], c)
                else:
                    c = np.float32(c + np.float32(x[i, k] * w[k, j]))
            if bias is not None:
                c = np.float32(c + bias[j])
            y[i, j] = c
    return y


def _spread_inputs(seed, M, K, N):
    """Values over many binades, so that rounding after every step matters."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * 2.0 ** rng.integers(-12, 12, (M, K))).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 2.0 ** rng.integers(-12, 12, (K, N))).astype(np.float32)
    b = (rng.standard_normal(N) * 2.0 ** rng.integers(-6, 6, N)).astype(np.float32)
    return x, w, b


def test_linear_f32_exact_fma_chain(oracle):
    x, w, b = _spread_inputs(5, 4, 11, 6)
    want = _chain(x, w, b)
    assert_bitexact(oracle.linear_f32(x, w, b), want, "exact fma chain + bias")
    assert_bitexact(oracle.linear_f32(x, w), _chain(x, w, None), "exact fma chain, no bias")
    # the check discriminates: each plausible mistake changes some output
    for name, alt in (("separate multiply and add", _chain(x, w, b, fused=False)),
                      ("reversed k order", _chain(x, w, b, order=range(10, -1, -1))),
                      ("last term dropped", _chain(x, w, b, drop_last=True))):
        assert not np.array_equal(alt.view(np.uint32), want.view(np.uint32)), name


def test_linear_f32_integer_closed_form(oracle):
    rng = np.random.default_rng(9)
    M, K, N = 13, 200, 37
    x = rng.integers(-8, 9, (M, K)).astype(np.float32)
    w = rng.integers(-8, 9, (K, N)).astype(np.float32)
    b = rng.integers(-1000, 1000, N).astype(np.float32)
    exact = x.astype(np.int64) @ w.astype(np.int64) + b.astype(np.int64)
    assert np.abs(exact).max() < 2 ** 24
    got = oracle.linear_f32(x, w, b)
    assert np.array_equal(got.astype(np.int64), exact)


def test_linear_f32_k0_and_signed_zero(oracle):
    b = np.array([1.5, -0.0, 0.0, -2.0], np.float32)
    y = oracle.linear_f32(np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32), b)
    # 0 + b: the -0 bias gives +0 (round-to-nearest sum of +0 and -0)
    want = np.tile(np.array([1.5, 0.0, 0.0, -2.0], np.float32), (3, 1))
    assert_bitexact(y, want, "K = 0")
    # a product of -0 into the +0 accumulator stays +0
    y = oracle.linear_f32(np.array([[-1.0]], np.float32), np.array([[0.0]], np.float32))
    assert not np.signbit(y[0, 0])


def test_linear_f32_golden_fixture(oracle):
    """Committed outputs of the reference build (make_golden_linear_f32.py)."""
    g = np.load(os.path.join(GOLDEN, "ref_linear_f32.npz"))
    assert_bitexact(oracle.linear_f32(g["head_x"], g["head_w"], g["head_b"]), g["head_y"],
                    "audio-head shape")
    assert_bitexact(oracle.linear_f32(g["head_x"], g["head_w"]), g["head_y_nobias"],
                    "audio-head shape, no bias")
    assert_bitexact(oracle.linear_f32(g["sp_x"], g["sp_w"], g["sp_b"]), g["sp_y"],
                    "zeros, -0, denormals")
    assert_bitexact(oracle.linear_f32(np.zeros((4, 0), np.float32), np.zeros((0, 6), np.float32),
                                      g["k0_b"]), g["k0_y"], "K = 0")


@pytest.mark.parametrize("M,K,N", [(157, 3072, 20), (6, 64, 16), (7, 65, 17), (1, 3, 1),
                                   (50, 513, 100)])
def test_linear_f32_matches_reference_build(oracle, ref, M, K, N):
    x, w, b = _spread_inputs(M * 7 + N, M, K, N)
    assert_bitexact(oracle.linear_f32(x, w, b), ref.matmul(x, w, b), f"{M}x{K}x{N}")
    assert_bitexact(oracle.linear_f32(x, w), ref.matmul(x, w), f"{M}x{K}x{N} no bias")
