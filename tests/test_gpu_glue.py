"""Block glue on the GPU against the oracle (pinned to the reference build):
sdq_rmsnorm_rope = rmsnorm (tensor.cpp:112-123) then apply_rope
(blocks.cpp:86-100) on the q / k columns of a q|k|v row, bit-exact, with the
(cosf, sinf) table of the reference's rope angles."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("L,rope", [(60, "3d"), (157, "1d"), (300, "none"), (27280, "3d")])
def test_rmsnorm_rope_bitexact(sdq_dev, oracle, L, rope):
    import torch

    import sdq

    heads, hd = 24, 128
    C = heads * hd
    print(f"[rmsnorm_rope] L={L} rope={rope}", flush=True)
    rng = np.random.default_rng(L)
    qkv = (oracle.randn(L * 3 * C, 50 + L).reshape(L, 3 * C)
           * rng.uniform(0.1, 30, (L, 1)).astype(np.float32)).astype(np.float32)
    qkv[min(3, L - 1), :C] = 0.0  # zero q row: ss = 0, inv = 1/sqrt(eps)
    wq = oracle.randn(C, 60)
    wk = oracle.randn(C, 61)
    if rope == "3d":
        T = max(1, L // 20)
        ang = oracle.rope_freqs_3d(T, 4, 5, hd, 10000.0)
        ang = np.resize(ang, (L, ang.shape[1])).astype(np.float32)
    elif rope == "1d":
        ang = oracle.rope_freqs_1d(L, hd, 10000.0, 0.19676)
    else:
        ang = None
    cs = None if ang is None else oracle.rope_cs(ang)
    d = torch.from_numpy(qkv).to(sdq_dev)
    cs_d = None if cs is None else torch.from_numpy(cs).to(sdq_dev)
    sdq.rmsnorm_rope(d, C, torch.from_numpy(wq).to(sdq_dev), heads, cs_d, col0=0)
    sdq.rmsnorm_rope(d, C, torch.from_numpy(wk).to(sdq_dev), heads, cs_d, col0=C)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    rows = np.arange(L) if L <= 400 else np.r_[0:8, 255:258, L // 2, L - 2, L - 1]
    for part, w in ((0, wq), (1, wk)):
        x = qkv[rows, part * C:(part + 1) * C]
        want = oracle.rmsnorm(x, w, 1e-6)
        if cs is not None:
            want = oracle.rope(want, cs[rows], heads)
        assert_bitexact(got[rows, part * C:(part + 1) * C], want, f"part {part}")
    assert_bitexact(got[:, 2 * C:], qkv[:, 2 * C:], "v untouched")


def test_rmsnorm_rope_errors(sdq_dev):
    import torch

    import sdq

    x = torch.zeros((4, 96), device=sdq_dev)
    w = torch.ones(96, device=sdq_dev)
    with pytest.raises(sdq.SdqError, match="head_dim"):
        sdq.rmsnorm_rope(x, 96, w, 5)  # 96 columns do not split into 5 heads


@pytest.mark.parametrize("Lq,Lk,heads", [(37, 53, 2), (300, 300, 3), (157, 512, 2), (1100, 157, 2),
                                         (64, 1, 1), (157, 768, 24), (768, 768, 24)])
def test_sdpa_matches_oracle(sdq_dev, oracle, Lq, Lk, heads):
    """Attention on q|k|v-style strided inputs against the oracle (bit-exact
    with the reference build's sdpa): within 2e-5 of the output scale (QK^T
    as three fp16 MFMA products per fp32 product of power-of-two-scaled rows,
    PV as three bf16 MFMA products, and an online softmax sum in another
    order). Few queries run as key splits
    merged afterwards (here 300x300, 157x512, and the twin backbone's audio
    fusion and video self-attention shapes)."""
    import torch

    import sdq

    print(f"[sdpa] Lq={Lq} Lk={Lk} heads={heads}", flush=True)
    C = heads * 128
    rng = np.random.default_rng(Lq * 7 + Lk)
    q = (rng.standard_normal((Lq, C)) * 0.6).astype(np.float32)
    kv = rng.standard_normal((Lk, 2 * C)).astype(np.float32)
    kv[:, :C] *= np.float32(0.6)
    want = oracle.sdpa(q, kv[:, :C], kv[:, C:], heads)
    qd = torch.from_numpy(q).to(sdq_dev)
    kvd = torch.from_numpy(kv).to(sdq_dev)
    out = torch.full((Lq, C), float("nan"), device=sdq_dev)
    sdq.sdpa(qd, kvd, kvd, out, heads, kcol=0, vcol=C)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got.astype(np.float64) - want) / (np.abs(want).max() + 1e-30)
    print(f"  max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5, float(err.max())


@pytest.mark.parametrize("qs,ks", [(3e4, 1e-4), (1e-6, 1e6), (1.0, 1.0)])
def test_sdpa_element_range(sdq_dev, oracle, qs, ks):
    """q and k elements far outside the fp16 range (up to ~1e5, down to
    ~1e-6), with logits of ordinary size, and rows whose magnitudes differ by
    2^-12..2^12 inside one key block: the scores' fp16 parts are taken of
    rows scaled by powers of two, which come back out exactly."""
    import torch

    import sdq

    Lq, Lk, heads = 100, 300, 2
    C = heads * 128
    print(f"[sdpa-range] q*{qs} k*{ks}", flush=True)
    rng = np.random.default_rng(17)
    q = (rng.standard_normal((Lq, C)) * 0.6 * qs).astype(np.float32)
    kv = rng.standard_normal((Lk, 2 * C)).astype(np.float32)
    kv[:, :C] *= np.float32(0.6 * ks)
    if qs == 1.0:
        # key rows 2^-12..2^12; q small enough that the largest rows' logits
        # stay ordinary (std ~6)
        rs = np.exp2(rng.integers(-12, 13, Lk)).astype(np.float32)
        kv[:, :C] *= rs[:, None]
        q *= np.float32(2.0 ** -8)
    want = oracle.sdpa(q, kv[:, :C], kv[:, C:], heads)
    qd = torch.from_numpy(q).to(sdq_dev)
    kvd = torch.from_numpy(kv).to(sdq_dev)
    out = torch.full((Lq, C), float("nan"), device=sdq_dev)
    sdq.sdpa(qd, kvd, kvd, out, heads, kcol=0, vcol=C)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got.astype(np.float64) - want) / (np.abs(want).max() + 1e-30)
    print(f"  max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5, float(err.max())


@pytest.mark.parametrize("Lq,Lk", [(157, 512), (768, 768)])
def test_sdpa_split_stacked_equals_separate(sdq_dev, oracle, Lq, Lk):
    """Key-split shapes (24 heads): two sequences stacked in one call give
    the bits of two separate calls (the split factor depends on the sequence,
    not on the batch), and forcing no split stays within the tolerance."""
    import os

    import torch

    import sdq

    from conftest import assert_bitexact

    heads, B = 24, 2
    C = heads * 128
    rng = np.random.default_rng(Lq + 3 * Lk)
    q = torch.from_numpy((rng.standard_normal((B * Lq, C)) * 0.6).astype(np.float32)).to(sdq_dev)
    kv = torch.from_numpy(rng.standard_normal((B * Lk, 2 * C)).astype(np.float32)).to(sdq_dev)
    out = torch.empty((B * Lq, C), device=sdq_dev)
    sdq.sdpa(q, kv, kv, out, heads, kcol=0, vcol=C, batch=B)
    for b in range(B):
        one = torch.empty((Lq, C), device=sdq_dev)
        qs, ks = q[b * Lq:(b + 1) * Lq], kv[b * Lk:(b + 1) * Lk]
        sdq.sdpa(qs, ks, ks, one, heads, kcol=0, vcol=C)
        torch.cuda.synchronize()
        assert_bitexact(out[b * Lq:(b + 1) * Lq].cpu().numpy(), one.cpu().numpy(), f"seq {b}")
    os.environ["SDQ_SDPA_SPLIT"] = "1"
    try:
        whole = torch.empty((Lq, C), device=sdq_dev)
        sdq.sdpa(q[:Lq], kv[:Lk], kv[:Lk], whole, heads, kcol=0, vcol=C)
        torch.cuda.synchronize()
    finally:
        del os.environ["SDQ_SDPA_SPLIT"]
    a, w = out[:Lq].cpu().numpy().astype(np.float64), whole.cpu().numpy().astype(np.float64)
    assert np.abs(a - w).max() / np.abs(w).max() <= 2e-5


def test_sdpa_fullsize_sampled(sdq_dev, oracle):
    """Self-attention at 720p/121 frames: 27280 tokens, 24 heads, q, k, v as
    the column blocks of one q|k|v tensor; sampled query rows (all heads)."""
    import torch

    import sdq

    L, heads = 27280, 24
    C = heads * 128
    print(f"[sdpa-full] L={L} heads={heads}", flush=True)
    g = torch.Generator(device=sdq_dev)
    g.manual_seed(3)
    qkv = torch.randn((L, 3 * C), generator=g, device=sdq_dev) * 0.5
    out = torch.empty((L, C), device=sdq_dev)
    sdq.sdpa(qkv, qkv, qkv, out, heads, qcol=0, kcol=C, vcol=2 * C)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 31, 32, 4097, L // 2, L - 33, L - 1])
    h = qkv.cpu().numpy()
    want = oracle.sdpa(h[rows, :C], h[:, C:2 * C], h[:, 2 * C:], heads)
    got = out[torch.from_numpy(rows).to(sdq_dev)].cpu().numpy()
    err = np.abs(got.astype(np.float64) - want) / (np.abs(want).max() + 1e-30)
    print(f"  max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5, float(err.max())


def test_sdpa_errors(sdq_dev):
    import torch

    import sdq

    q = torch.zeros((4, 96), device=sdq_dev)
    # the binding sees the short rows; the C ABI rejects them too
    with pytest.raises(sdq.SdqError, match="outside its 96 columns"):
        sdq.sdpa(q, q, q, q, 1)  # 96 columns < one head of 128
    p = ctypes.c_void_p(q.data_ptr())
    rc = sdq._lib.sdq_sdpa(p, 96, p, 96, p, 96, p, 96, 4, 4, 1, 128, None)
    assert rc == sdq.ERR_INVALID and b"row strides" in sdq._lib.sdq_last_error()


@pytest.mark.parametrize("M,K,affine", [(1, 3072, True), (157, 3072, True), (300, 3072, False),
                                        (77, 100, True), (2000, 3072, True)])
def test_layernorm_bitexact(sdq_dev, oracle, M, K, affine):
    """sdq_layernorm against the oracle's layernorm (pinned to the reference
    build's blk::layernorm, affine output fmaf(t, w, b)), bit-exact; ragged K,
    a constant row (variance 0) and large offsets included."""
    import torch

    import sdq

    print(f"[layernorm] M={M} K={K} affine={affine}", flush=True)
    rng = np.random.default_rng(M * 3 + K)
    x = (oracle.randn(M * K, 70 + M).reshape(M, K)
         * rng.uniform(0.1, 20, (M, 1)) + rng.uniform(-50, 50, (M, 1))).astype(np.float32)
    x[M // 2] = np.float32(3.25)
    w = oracle.randn(K, 71) if affine else None
    b = oracle.randn(K, 72) if affine else None
    want = oracle.layernorm(x, 1e-6, w, b)
    xd = torch.from_numpy(x).to(sdq_dev)
    y = torch.full_like(xd, float("nan"))
    dev = (lambda a: None if a is None else torch.from_numpy(a).to(sdq_dev))
    sdq.layernorm(xd, y, dev(w), dev(b), 1e-6)
    sdq.layernorm(xd, xd, dev(w), dev(b), 1e-6)  # in place
    torch.cuda.synchronize()
    assert_bitexact(y.cpu().numpy(), want, "layernorm")
    assert_bitexact(xd.cpu().numpy(), want, "layernorm in place")


@pytest.mark.parametrize("M,nt", [(1, 1), (9, 2), (13, 11), (8, 12), (15, 13), (17, 25), (5, 96)])
def test_row_stats_tile_counts(sdq_dev, oracle, M, nt):
    """The row sums of whole 32-column tiles (K = 32*nt, aligned rows) at tile
    counts below, at and past the loads kept in flight, rows past M in the
    last group of 8, and a row whose last tile ends the allocation: layernorm
    and rmsnorm (rows of stride ld = C + 32, the weight-less rest of the row
    never read) bit-exact against the oracle; the same rows at an unaligned
    start (the per-column path) give the same bits."""
    import torch

    import sdq

    K = 32 * nt
    print(f"[row stats] M={M} K={K}", flush=True)
    rng = np.random.default_rng(nt * 7 + M)
    x = (oracle.randn(M * K, 90 + nt).reshape(M, K) * rng.uniform(0.1, 20, (M, 1))
         + rng.uniform(-9, 9, (M, 1))).astype(np.float32)
    x[0, 0] = np.float32(-0.0)
    want = oracle.layernorm(x, 1e-6, None, None)
    xd = torch.from_numpy(x).to(sdq_dev)
    y = torch.full_like(xd, float("nan"))
    sdq.layernorm(xd, y, None, None, 1e-6)
    # the same rows one float into a larger buffer: not 16-byte aligned
    big = torch.zeros(M * K + 1, device=sdq_dev)
    big[1:].copy_(xd.reshape(-1))
    xu = big[1:].view(M, K)
    yu = torch.full_like(xd, float("nan"))
    sdq.layernorm(xu, yu, None, None, 1e-6)
    torch.cuda.synchronize()
    assert_bitexact(y.cpu().numpy(), want, "layernorm, whole tiles")
    assert_bitexact(yu.cpu().numpy(), want, "layernorm, unaligned rows")

    heads = 1 if nt < 4 else nt // 2 if nt % 2 == 0 else nt
    C, ld = K, K + 32
    w = oracle.randn(C, 91)
    rows = np.zeros((M, ld), np.float32)
    rows[:, 32:] = x  # the normalised block ends each row (and the last one the buffer)
    d = torch.from_numpy(rows).to(sdq_dev)
    sdq.rmsnorm_rope(d, C, torch.from_numpy(w).to(sdq_dev), heads, None, col0=32)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    assert_bitexact(got[:, 32:], oracle.rmsnorm(x, w, 1e-6), "rmsnorm, whole tiles")
    assert_bitexact(got[:, :32], rows[:, :32], "columns before the block untouched")


def test_rope_only_and_add(sdq_dev, oracle):
    """The fusion attention's late rotation of q (no rmsnorm, w = NULL) and
    the x += y of its two attention outputs, bit-exact."""
    import torch

    import sdq

    heads, hd, L = 3, 128, 130
    C = heads * hd
    x = oracle.randn(L * C, 80).reshape(L, C) * np.float32(4.0)
    y = oracle.randn(L * C, 81).reshape(L, C)
    cs = oracle.rope_cs(oracle.rope_freqs_1d(L, hd, 10000.0, 1.0))
    xd = torch.from_numpy(x).to(sdq_dev)
    sdq.rmsnorm_rope(xd, C, None, heads, torch.from_numpy(cs).to(sdq_dev))
    torch.cuda.synchronize()
    assert_bitexact(xd.cpu().numpy(), oracle.rope(x, cs, heads), "rope only")
    xd = torch.from_numpy(x).to(sdq_dev)
    sdq.add_(xd, torch.from_numpy(y).to(sdq_dev))
    torch.cuda.synchronize()
    assert_bitexact(xd.cpu().numpy(), oracle.add(x, y), "add")
    with pytest.raises(sdq.SdqError, match="nothing to do"):
        sdq.rmsnorm_rope(xd, C, None, heads, None)


def test_rmsnorm_rope_batch_equals_single_calls(sdq_dev, oracle):
    """sdq_rmsnorm_rope_batch over the q and k blocks of q|k|v (own weights,
    3-D table), a 2C-stride context k block without rotation, a rotation-only
    block and an empty one: bit-identical to one sdq_rmsnorm_rope call each."""
    import torch

    import sdq

    heads, C = 3, 384
    L, Lc = 300, 77
    qkv = oracle.randn(L * 3 * C, 90).reshape(L, 3 * C) * np.float32(3.0)
    kv = oracle.randn(Lc * 2 * C, 91).reshape(Lc, 2 * C)
    q2 = oracle.randn(L * C, 92).reshape(L, C)
    wq, wk, wc = oracle.randn(C, 93), oracle.randn(C, 94), oracle.randn(C, 95)
    cs = oracle.rope_cs(oracle.rope_freqs_1d(L, 128, 10000.0, 1.0))
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    wq_d, wk_d, wc_d, cs_d = dv(wq), dv(wk), dv(wc), dv(cs)
    a = [dv(qkv), dv(kv), dv(q2)]
    b = [dv(qkv), dv(kv), dv(q2)]
    empty = torch.zeros((0, C), device=sdq_dev)
    sdq.rmsnorm_rope_batch([(a[0], 0, wq_d, cs_d), (a[0], C, wk_d, cs_d), (a[1], 0, wc_d, None),
                            (empty, 0, wc_d, None)], C, heads)
    sdq.rmsnorm_rope_batch([(a[2], 0, None, cs_d)], C, heads)
    sdq.rmsnorm_rope(b[0], C, wq_d, heads, cs_d, col0=0)
    sdq.rmsnorm_rope(b[0], C, wk_d, heads, cs_d, col0=C)
    sdq.rmsnorm_rope(b[1], C, wc_d, heads, None, col0=0)
    sdq.rmsnorm_rope(b[2], C, None, heads, cs_d)
    torch.cuda.synchronize()
    for x, y, name in zip(a, b, ("qkv", "ctx kv", "rope only")):
        assert_bitexact(x.cpu().numpy(), y.cpu().numpy(), name)
    want = oracle.rope(oracle.rmsnorm(qkv[:, :C], wq, 1e-6), cs, heads)
    assert_bitexact(a[0].cpu().numpy()[:, :C], want, "q vs oracle")
    with pytest.raises(sdq.SdqError, match="0 to 4 segments"):
        sdq.rmsnorm_rope_batch([(a[2], 0, wq_d, None)] * 5, C, heads)
