"""Pins the CPU oracle (oracle/qgemm_oracle.c) before anything is checked
against it: the reference's own golden vectors, the reference's compiled
sources (oracle/_ref), closed forms, and brute force on small inputs."""
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN, assert_bitexact


def cosine(a, b):
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


# ---------------------------------------------------------------- golden
def test_golden_quantize_rowwise(oracle):
    """tests/test_golden.cpp:64-72: int8 byte-exact, scale within 1e-6."""
    g = np.load(os.path.join(GOLDEN, "basic_golden.npz"))
    q, s = oracle.quantize_rowwise(g["q_w"])
    assert_bitexact(q, g["q_wq"], "quantize_rowwise i8")
    assert np.max(np.abs(s - g["q_scale"])) < 1e-6


def test_golden_qgemm_cosine(oracle):
    """tests/test_golden.cpp:73-81: qgemm vs the fp32 dequant product, cosine > 0.999."""
    g = np.load(os.path.join(GOLDEN, "basic_golden.npz"))
    o = oracle.qgemm(g["qg_a"], g["qg_bq"], g["qg_bs"])
    assert cosine(o, g["qg_out"]) > 0.999


@pytest.mark.parametrize("M,K,N", [(17, 31, 13), (64, 1024, 512)])
def test_core_shapes_cosine(oracle, M, K, N):
    """tests/test_core.cpp:93-118: randu seeds 7+M / 13+N, cosine > 0.999."""
    A = oracle.randu(M * K, 7 + M).reshape(M, K)
    W = oracle.randu(N * K, 13 + N).reshape(N, K)
    q, s = oracle.quantize_rowwise(W)
    o = oracle.qgemm(A, q, s)
    ref = A.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T
    assert cosine(o, ref) > 0.999


def test_ref_fixture_outputs(oracle):
    """Committed outputs of the reference's own compiled qgemm."""
    g = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    for (M, K, N) in [(17, 31, 13), (64, 1024, 512)]:
        A = oracle.randu(M * K, 7 + M).reshape(M, K)
        W = oracle.randu(N * K, 13 + N).reshape(N, K)
        q, s = oracle.quantize_rowwise(W)
        assert_bitexact(oracle.qgemm(A, q, s), g[f"core_{M}x{K}x{N}_out"], f"core {M}x{K}x{N}")
    o = oracle.qgemm(g["special_a"], g["special_bq"], g["special_bs"])
    assert_bitexact(o, g["special_out"], "special rows")


def test_ref_fixture_cfg1_hash(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    M, K, N = 256, 3072, 3072
    A = oracle.randn(M * K, 1001).reshape(M, K)
    W = oracle.randn(N * K, 1002).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    o = oracle.qgemm(A, q, s)
    assert hashlib.sha256(o.tobytes()).digest() == g["cfg1_sha256"].tobytes()


# ------------------------------------------------- reference-compiled oracle
@pytest.mark.parametrize("M,K,N", [(1, 256, 64), (7, 100, 33), (64, 512, 256),
                                   (300, 257, 129), (2048, 192, 96), (2100, 64, 70)])
def test_oracle_matches_reference_build(oracle, ref, M, K, N):
    """Bit-exact vs the reference's own sd::qgemm, both M<2048 (narrow s8
    path) and M>=2048 (widened s16 path), qgemm.cpp:98-138."""
    rng = np.random.default_rng(M * 131 + K * 7 + N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[::5] *= np.float32(37.0)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q, s = oracle.quant_rows(W)
    assert_bitexact(oracle.qgemm(A, q, s), ref.qgemm(A, q, s), f"{M}x{K}x{N}")


def test_oracle_special_rows_match_reference(oracle, ref):
    g = np.load(os.path.join(GOLDEN, "ref_qgemm.npz"))
    assert_bitexact(ref.qgemm(g["special_a"], g["special_bq"], g["special_bs"]),
                    g["special_out"], "special rows (fixture vs live reference)")


def test_quantize_rowwise_matches_reference(oracle, ref):
    W = oracle.randu(37 * 513, 42).reshape(37, 513)
    W[3] = 0.0
    q1, s1 = oracle.quantize_rowwise(W)
    q2, s2 = ref.quantize_rowwise(W)
    assert_bitexact(q1, q2, "q")
    assert_bitexact(s1, s2, "scale")


def test_randu_matches_reference(oracle, ref):
    for seed in (0, 1, 7, 2**40 + 3):
        assert_bitexact(oracle.randu(5000, seed), ref.randu(5000, seed), f"randu {seed}")


# ------------------------------------------------------------- closed forms
def test_act_quant_closed_form(oracle):
    """qgemm.cpp:84-96 restated independently in numpy float32."""
    rng = np.random.default_rng(3)
    A = (rng.standard_normal((50, 200)) * rng.uniform(0.01, 100, (50, 1))).astype(np.float32)
    aq, asc = oracle.act_quant(A)
    mx = np.abs(A).max(axis=1)
    sc = (mx / np.float32(127.0)).astype(np.float32)
    sc[sc == 0] = 1
    inv = (np.float32(1.0) / sc).astype(np.float32)
    y = (A * inv[:, None]).astype(np.float32)
    q = np.clip(np.rint(y), -127, 127).astype(np.int8)
    assert_bitexact(asc, sc, "as")
    assert_bitexact(aq, q, "aq")


def test_act_quant_special_values(oracle):
    assert oracle.round_to_i8(np.nan) == -127
    assert oracle.round_to_i8(np.inf) == -127      # cvtss2si -> INT_MIN -> clamp
    assert oracle.round_to_i8(-np.inf) == -127
    assert oracle.round_to_i8(3e9) == -127         # out of int32 -> INT_MIN
    assert oracle.round_to_i8(2e9) == 127          # fits int32 -> clamp
    assert oracle.round_to_i8(2.5) == 2 and oracle.round_to_i8(3.5) == 4   # ties to even
    assert oracle.round_to_i8(-2.5) == -2
    aq, asc = oracle.act_quant(np.zeros((2, 9), np.float32))
    assert np.all(aq == 0) and np.all(asc == 1.0)
    A = np.array([[1.0, -2.0, 4.0, -4.0]], np.float32)
    aq, asc = oracle.act_quant(A)
    assert list(aq[0]) == [32, -64, 127, -127]     # +-amax -> +-127


def test_qgemm_acc_brute_force(oracle):
    rng = np.random.default_rng(11)
    aq = rng.integers(-127, 128, (9, 77)).astype(np.int8)
    bq = rng.integers(-127, 128, (13, 77)).astype(np.int8)
    want = aq.astype(np.int64) @ bq.astype(np.int64).T
    assert_bitexact(oracle.qgemm_acc(aq, bq), want.astype(np.int32), "acc")
    # extreme values: max |acc| at K=14336 still fits int32
    aq = np.full((2, 14336), 127, np.int8)
    bq = np.full((2, 14336), -127, np.int8)
    assert oracle.qgemm_acc(aq, bq)[0, 0] == -127 * 127 * 14336


def test_linear_at_equals_full_product(oracle):
    """The spot-check form gives the full product's value at every position
    (with and without bias), so it inherits orc_qgemm's pins."""
    M, K, N = 37, 300, 45
    A = oracle.randn(M * K, 71).reshape(M, K)
    q, s = oracle.quant_rows(oracle.randn(N * K, 72).reshape(N, K) * np.float32(0.02))
    bias = oracle.randn(N, 73) * np.float32(0.01)
    aq, asc = oracle.act_quant(A)
    mm, nn = np.meshgrid(np.arange(M), np.arange(N), indexing="ij")
    full = oracle.qgemm(A, q, s)
    assert_bitexact(oracle.linear_at(aq, asc, q, s, mm.ravel(), nn.ravel()).reshape(M, N),
                    full, "linear_at")
    yb = oracle.bias_add(full, bias)
    assert_bitexact(oracle.linear_at(aq, asc, q, s, mm.ravel(), nn.ravel(), bias).reshape(M, N),
                    yb, "linear_at+bias")
    x = oracle.randn(M * N, 74).reshape(M, N)
    g = oracle.randn(N, 75)
    for fma in (True, False):
        got = oracle.linear_at(aq, asc, q, s, mm.ravel(), nn.ravel(), bias, "gated", g, x, fma)
        assert_bitexact(got.reshape(M, N), oracle.gated_add(x, yb, g, fma), f"gated fma={fma}")
    got = oracle.linear_at(aq, asc, q, s, mm.ravel(), nn.ravel(), bias, "resid", resid=x)
    assert_bitexact(got.reshape(M, N), oracle.add(x, yb), "resid")


def test_rescale_two_roundings(oracle):
    """out = fl(fl(acc) * fl(as*bs)), no FMA: differs from the one-rounding
    (double) product on some inputs, which a dropped rounding would fail."""
    rng = np.random.default_rng(5)
    acc = rng.integers(-2**24, 2**24, (64, 64)).astype(np.int32) * 7
    a = rng.uniform(1e-3, 1, 64).astype(np.float32)
    b = rng.uniform(1e-4, 1e-2, 64).astype(np.float32)
    got = oracle.rescale(acc, a, b)
    s = (a[:, None] * b[None, :]).astype(np.float32)
    want = (acc.astype(np.float32) * s).astype(np.float32)
    assert_bitexact(got, want, "rescale")
    one_round = (acc.astype(np.float64) * a[:, None].astype(np.float64)
                 * b[None, :].astype(np.float64)).astype(np.float32)
    assert np.any(bits(one_round) != bits(got))


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def test_bias_and_residual_closed_forms(oracle):
    rng = np.random.default_rng(8)
    y = rng.standard_normal((16, 40)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    g = rng.standard_normal(40).astype(np.float32)
    x = rng.standard_normal((16, 40)).astype(np.float32)
    assert_bitexact(oracle.bias_add(y, b), (y + b).astype(np.float32), "bias")
    assert_bitexact(oracle.add(x, y), (x + y).astype(np.float32), "add")
    # fma: exact product + x rounded once (float64 holds y*g exactly)
    fma = (y.astype(np.float64) * g.astype(np.float64) + x.astype(np.float64)).astype(np.float32)
    got = oracle.gated_add(x, y, g, use_fma=True)
    # float64 sum can round twice; accept only where it is provably exact
    exact = np.abs(fma.astype(np.float64) - (y.astype(np.float64) * g + x)) < 2.0 ** -60
    assert_bitexact(got[exact], fma[exact], "gated fma")
    nofma = oracle.gated_add(x, y, g, use_fma=False)
    assert_bitexact(nofma, (x + (y * g).astype(np.float32)).astype(np.float32), "gated no-fma")
    assert np.any(bits(nofma) != bits(got))


def test_gelu_tanh_tolerance(oracle):
    v = np.linspace(-8, 8, 4001).astype(np.float32)
    d = v.astype(np.float64)
    want = 0.5 * d * (1 + np.tanh(0.7978845608028654 * (d + 0.044715 * d ** 3)))
    got = oracle.gelu_tanh(v)
    assert np.max(np.abs(got - want)) < 1e-5


def test_quant_rows_closed_form(oracle):
    """tools/quantize/pack_sdcpp.py:45-51 evaluated by numpy itself."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((33, 129)) * 0.02).astype(np.float32)
    x[4] = 0.0
    amax = np.abs(x).max(axis=1)
    safe = np.where(amax > 0, amax, np.float32(1.0)).astype(np.float32)
    qn = np.rint(x * (np.float32(127.0) / safe)[:, None])
    np.clip(qn, -127, 127, out=qn)
    q, s = oracle.quant_rows(x)
    assert_bitexact(q, qn.astype(np.int8), "q")
    assert_bitexact(s, (amax / np.float32(127.0)).astype(np.float32), "scale")
    assert s[4] == 0.0


def test_randn_closed_form(oracle):
    """src/pipeline/gen.cpp:88-105: splitmix64 + Box-Muller."""
    mask = (1 << 64) - 1
    s = (7 + 0x9E3779B97F4A7C15) & mask

    def nxt():
        nonlocal s
        s = (s + 0x9E3779B97F4A7C15) & mask
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)

    want = []
    for _ in range(50):
        u1 = ((nxt() >> 11) + 1.0) / 9007199254740993.0
        u2 = (nxt() >> 11) / 9007199254740992.0
        r = np.sqrt(-2.0 * np.log(u1))
        want += [np.float32(r * np.cos(6.283185307179586 * u2)),
                 np.float32(r * np.sin(6.283185307179586 * u2))]
    assert_bitexact(oracle.randn(100, 7), np.array(want, np.float32), "randn")
    x = oracle.randn(200001, 9)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1) < 0.01


def test_oracle_planted_mistakes_are_caught(oracle):
    """A dropped rounding, a transposed operand or an RNE->truncation swap in
    the oracle's formulas would fail the checks above; show each one differs
    on the golden inputs (mistakes planted here on the CPU, not in code)."""
    g = np.load(os.path.join(GOLDEN, "basic_golden.npz"))
    A, q, s = g["qg_a"], g["qg_bq"], g["qg_bs"]
    good = oracle.qgemm(A, q, s)
    aq, asc = oracle.act_quant(A)
    acc = aq.astype(np.int64) @ q.astype(np.int64).T
    one_round = (acc * (asc[:, None].astype(np.float64) * s[None, :])).astype(np.float32)
    assert np.any(bits(one_round) != bits(good))
    trunc = np.clip(np.trunc(A * (np.float32(1) / asc)[:, None]), -127, 127).astype(np.int64)
    assert np.any(trunc != aq)
    assert not np.array_equal(aq @ q.T.astype(np.int64), (aq @ q.T.astype(np.int64))[:, ::-1])


# ------------------------------------------------ DiT glue: layernorm, mod_rows
def _ln_rows(seed, M=24, N=3072):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, N)) * rng.uniform(0.01, 100, (M, 1))).astype(np.float32)
    x[1] = 0.0                      # var = 0: inv = 1/sqrt(eps)
    x[2] = np.float32(3.25)         # constant row
    x[3] *= np.float32(1e-30)       # tiny values
    x[4] *= np.float32(1e15)        # huge values (d*d near the float range)
    x[5, ::7] = -x[5, ::7]
    return x


def _ln_serial_numpy(x, eps, fma_var=False):
    """blocks.cpp:18-43 restated in numpy: serial float32 sums over k,
    vectorized over rows (each step rounds like the C loop)."""
    M, N = x.shape
    mu = np.zeros(M, np.float32)
    for k in range(N):
        mu = mu + x[:, k]
    mu = mu / np.float32(N)
    var = np.zeros(M, np.float32)
    for k in range(N):
        d = x[:, k] - mu
        if fma_var:  # a contracted d*d + var (one rounding), for the planted-mistake check
            var = (d.astype(np.float64) * d + var).astype(np.float32)
        else:
            var = var + d * d
    inv = np.float32(1) / np.sqrt(var / np.float32(N) + np.float32(eps))
    t = (x - mu[:, None]) * inv[:, None]
    return t * np.float32(1) + np.float32(0)


def test_layernorm_matches_reference_build(oracle, ref):
    x = _ln_rows(41)
    want = ref.layernorm(x, 1e-6)
    assert_bitexact(oracle.layernorm(x, 1e-6), want, "layernorm vs reference build")
    assert_bitexact(_ln_serial_numpy(x, 1e-6), want, "numpy serial restatement")
    assert not np.signbit(want[1]).any()  # (x-mu)*inv*1 + 0 turns -0 into +0


def test_layernorm_closed_form_and_planted_mistakes(oracle):
    x = _ln_rows(42)
    y = oracle.layernorm(x, 1e-6)
    assert_bitexact(y, _ln_serial_numpy(x, 1e-6), "numpy serial restatement")
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    yd = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-6)
    ok = np.isfinite(yd).all(1) & (np.abs(x).max(1) < 1e10)
    assert np.allclose(y[ok], yd[ok], rtol=2e-4, atol=2e-4)
    # planted: a contracted variance sum, or float64 sums, differ from the oracle
    assert np.any(bits(_ln_serial_numpy(x, 1e-6, fma_var=True)) != bits(y))
    assert np.any(bits(yd.astype(np.float32)[ok]) != bits(y[ok]))


def test_mod_rows_matches_reference_build_and_closed_form(oracle, ref):
    rng = np.random.default_rng(43)
    x = _ln_rows(44, M=16, N=1024)
    shift = rng.standard_normal(1024).astype(np.float32)
    scale = (rng.standard_normal(1024) * 0.3).astype(np.float32)
    want = ref.mod_rows(x, shift, scale)
    got = oracle.mod_rows(x, shift, scale)
    assert_bitexact(got, want, "mod_rows vs reference build")
    a = (np.float32(1) + scale).astype(np.float64)
    once = (x.astype(np.float64) * a + shift).astype(np.float32)  # x*a exact in float64
    fin = np.isfinite(once)
    assert (bits(got[fin]) == bits(once[fin])).mean() > 0.9999
    two = (x * (np.float32(1) + scale) + shift).astype(np.float32)  # planted: two roundings
    assert np.any(bits(two) != bits(got))


def test_rmsnorm_matches_reference_build(oracle, ref):
    x = _ln_rows(45, M=16, N=3072)
    w = np.random.default_rng(46).standard_normal(3072).astype(np.float32)
    want = ref.rmsnorm(x, w, 1e-6)
    got = oracle.rmsnorm(x, w, 1e-6)
    assert_bitexact(got, want, "rmsnorm vs reference build")
    xd = x.astype(np.float64)
    yd = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w
    ok = np.isfinite(yd).all(1) & (np.abs(x).max(1) < 1e10)
    assert np.allclose(got[ok], yd[ok], rtol=2e-4, atol=2e-4)
    # planted: a contracted sum of squares differs (on plain random rows)
    xr = oracle.randn(64 * 3072, 48).reshape(64, 3072)
    good = oracle.rmsnorm(xr, w, 1e-6)
    fused = np.zeros(64, np.float32)
    for k in range(3072):
        fused = (xr[:, k].astype(np.float64) * xr[:, k] + fused).astype(np.float32)
    inv = np.float32(1) / np.sqrt(fused / np.float32(3072) + np.float32(1e-6))
    assert np.any(bits((xr * inv[:, None]) * w) != bits(good))


def test_rope_tables_and_rotation_match_reference_build(oracle, ref):
    # video: T x H x W tokens, audio: 1-D with the temporal scaling factor
    a3 = oracle.rope_freqs_3d(3, 4, 5, 128, 10000.0)
    assert_bitexact(a3, ref.rope_freqs_3d(3, 4, 5, 128, 10000.0), "rope_freqs_3d")
    a1 = oracle.rope_freqs_1d(157, 128, 10000.0, 0.19676)
    assert_bitexact(a1, ref.rope_freqs_1d(157, 128, 10000.0, 0.19676), "rope_freqs_1d")
    assert a3.shape[1] == 64 and a1.shape[1] == 22
    heads, hd = 24, 128
    for ang in (a3, a1):
        L = ang.shape[0]
        x = oracle.randn(L * heads * hd, 47).reshape(L, heads * hd)
        want = ref.apply_rope(x, ang, heads)
        got = oracle.rope(x, oracle.rope_cs(ang), heads)
        assert_bitexact(got, want, "apply_rope")
        # a rotation keeps each pair's length; angle 0 (token 0) is the identity
        nr = ang.shape[1]
        p0 = x.reshape(L, heads, hd)[:, :, :2 * nr].astype(np.float64).reshape(L, heads, nr, 2)
        p1 = got.reshape(L, heads, hd)[:, :, :2 * nr].astype(np.float64).reshape(L, heads, nr, 2)
        assert np.allclose((p0 ** 2).sum(-1), (p1 ** 2).sum(-1), rtol=1e-5, atol=1e-6)
        assert_bitexact(got[0], x[0], "angle 0")
        assert_bitexact(got.reshape(L, heads, hd)[:, :, 2 * nr:], x.reshape(L, heads, hd)[:, :, 2 * nr:],
                        "unrotated pairs")


def test_sdpa_matches_reference_build(oracle, ref):
    heads, hd = 4, 128
    for (Lq, Lk, seed) in ((37, 53, 60), (64, 7, 61), (5, 130, 62)):
        rng = np.random.default_rng(seed)
        q = (rng.standard_normal((Lq, heads * hd)) * 0.5).astype(np.float32)
        k = (rng.standard_normal((Lk, heads * hd)) * 0.5).astype(np.float32)
        v = rng.standard_normal((Lk, heads * hd)).astype(np.float32)
        got = oracle.sdpa(q, k, v, heads)
        assert_bitexact(got, ref.sdpa(q, k, v, heads), f"sdpa {Lq}x{Lk}")
        # float64 softmax attention
        want = np.empty_like(got, np.float64)
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T / np.sqrt(hd)
            pr = np.exp(s - s.max(1, keepdims=True))
            pr /= pr.sum(1, keepdims=True)
            want[:, sl] = pr @ v[:, sl]
        assert np.allclose(got, want, rtol=1e-4, atol=1e-5)


def test_affine_layernorm_matches_reference_build(oracle, ref):
    x = _ln_rows(49)
    rng = np.random.default_rng(50)
    w = rng.standard_normal(3072).astype(np.float32)
    b = rng.standard_normal(3072).astype(np.float32)
    want = ref.layernorm(x, 1e-6, w, b)
    got = oracle.layernorm(x, 1e-6, w, b)
    assert_bitexact(got, want, "affine layernorm vs reference build")
    t = oracle.layernorm(x, 1e-6)  # the no-affine output is t + 0 = fmaf(t, 1, 0)
    two = (t * w + b).astype(np.float32)  # planted: two roundings
    assert np.any(bits(two) != bits(got))


def test_ref_glue_fixture_outputs(oracle):
    """Committed outputs of the reference's own block glue (layernorm with and
    without affine, mod_rows, rmsnorm, the 3-D / 1-D rope angles and
    apply_rope, sdpa; tests/golden/make_golden_glue.py): the oracle's
    restatements reproduce them bit for bit, without the reference sources."""
    g = np.load(os.path.join(GOLDEN, "ref_glue.npz"))
    x, w, b = g["x"], g["w"], g["b"]
    assert_bitexact(oracle.layernorm(x, 1e-6), g["layernorm"], "layernorm")
    assert_bitexact(oracle.layernorm(x, 1e-6, w, b), g["layernorm_affine"], "layernorm affine")
    assert_bitexact(oracle.mod_rows(g["layernorm"], g["shift"], g["scale"]), g["mod_rows"],
                    "mod_rows")
    assert_bitexact(oracle.rmsnorm(x, w, 1e-6), g["rmsnorm"], "rmsnorm")
    assert_bitexact(oracle.rope_freqs_3d(2, 3, 4, 128, 10000.0), g["ang3"], "rope_freqs_3d")
    assert_bitexact(oracle.rope_freqs_1d(24, 128, 10000.0, 0.19676), g["ang1"], "rope_freqs_1d")
    assert_bitexact(oracle.rope(x, oracle.rope_cs(g["ang3"]), 2), g["rope3"], "apply_rope 3-D")
    assert_bitexact(oracle.rope(x, oracle.rope_cs(g["ang1"]), 2), g["rope1"], "apply_rope 1-D")
    assert_bitexact(oracle.sdpa(g["q"], g["k"], g["v"], 2), g["sdpa"], "sdpa")


def test_reference_build_block_chain_equals_oracle_chain(oracle, ref):
    """The block chain the GPU drift test runs on the reference build's own
    functions (qgemm, sdpa, layernorm, mod_rows, rmsnorm) gives the oracle
    chain's bits: two fusion layers of a twin backbone at small widths."""
    from test_gpu_block_full import _norms, _ref_block, _weights
    from test_gpu_drift import _RefOps

    dim, heads, Mv, Ma, Mc = 256, 2, 48, 20, 16
    ops = _RefOps(oracle, ref)
    xv = oracle.randn(Mv * dim, 1).reshape(Mv, dim)
    xa = oracle.randn(Ma * dim, 2).reshape(Ma, dim)
    cv = oracle.randn(Mc * dim, 3).reshape(Mc, dim)
    ca = oracle.randn(Mc * dim, 4).reshape(Mc, dim)
    cs_v = oracle.rope_cs(oracle.rope_freqs_3d(1, 12, 4, 128))
    cs_a = oracle.rope_cs(oracle.rope_freqs_1d(Ma, 128, 10000.0, 0.19676))
    chains = []
    for o in (oracle, ops):
        a, v = xa, xv
        for i in range(2):
            lv, la = _weights(oracle, dim, 512, 10 + i, True), _weights(oracle, dim, 512, 50 + i, True)
            nv, na = _norms(oracle, dim, 20 + i), _norms(oracle, dim, 30 + i)
            ev = (oracle.randn(6 * dim, 40 + i) * np.float32(0.3)).reshape(6, dim)
            ea = (oracle.randn(6 * dim, 60 + i) * np.float32(0.3)).reshape(6, dim)
            a1 = _ref_block(o, a, ca, ea, la, na, heads, cs_a, True, phases=1)
            v1 = _ref_block(o, v, cv, ev, lv, nv, heads, cs_v, True, phases=1)
            a = _ref_block(o, a1, ca, ea, la, na, heads, cs_a, True, v1, cs_v, 2)
            v = _ref_block(o, v1, cv, ev, lv, nv, heads, cs_v, True, a1, cs_a, 2)
        chains.append((v, a))
    assert_bitexact(chains[1][0], chains[0][0], "video chain")
    assert_bitexact(chains[1][1], chains[0][1], "audio chain")
