"""The whole DiT block on the GPU (sd_dit_block_step_forward: norms,
modulation, RoPE, attention and the int8 Linears) against the oracle's
restatement of the reference's block (ovi_dit.cpp:205-268): block_self_fwd,
then block_vanilla_fwd's cross attention + FFN, or fusion_cross_ffn.

Every step of the oracle chain is pinned to the reference build; the GPU's
steps are each bit-exact with it except the attention (split-fp16 scores,
split bf16 P.V, online softmax: within 2e-5 of the output scale) and GELU's tanhf, both tested on
their own against the oracle. Two checks per case:
  * bit-exact: the oracle chain with its sdpa and fc1+GELU steps replaced by
    the GPU's own kernels (sdq.sdpa, sdq.qlinear_host with the GELU
    epilogue) on the oracle's (bit-exact) inputs. Every other step, and the
    order and wiring of all of them, must then agree bit for bit.
  * pure oracle, to a relative tolerance: the attention's small differences
    move a few int8 rounding decisions of the next Linear's quantizer (one
    flip moves a whole output row by a weight times a quantum, ~1e-3 of the
    scale), and the FFN amplifies them: 1e-2 of the residual stream's scale
    at small widths, 5e-2 at dim 3072 / ffn 14336 (measured 1e-7 to 1.6e-3
    and 1.3e-2). Wiring mistakes move it by O(0.1-1) and fail the bit-exact
    check outright."""
import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "kf", "vf", "fc1", "fc2")


def _weights(oracle, dim, ffn, seed, fusion):
    lin = {}
    for i, n in enumerate(NAMES):
        if n in ("kf", "vf") and not fusion:
            continue
        out, inp = (ffn, dim) if n == "fc1" else ((dim, ffn) if n == "fc2" else (dim, dim))
        W = oracle.randn(out * inp, seed + 10 * i).reshape(out, inp) * np.float32(0.05)
        q, s = oracle.quant_rows(W)
        lin[n] = (q, s, oracle.randn(out, seed + 10 * i + 1) * np.float32(0.02))
    return lin


def _norms(oracle, dim, seed):
    r = lambda k, a, b: (oracle.randu(dim, seed + k) * np.float32(b - a) + np.float32(a))  # noqa
    return dict(sa_nq=r(1, 0.5, 1.5), sa_nk=r(2, 0.5, 1.5), ca_nq=r(3, 0.5, 1.5),
                ca_nk=r(4, 0.5, 1.5), ln3_w=r(5, 0.5, 1.5), ln3_b=r(6, -0.2, 0.2),
                nk_fusion=r(7, 0.5, 1.5), pnf_w=r(8, 0.5, 1.5), pnf_b=r(9, -0.2, 0.2))


def _gpu_sdpa(dev):
    def run(q, k, v, heads):
        import torch

        import sdq

        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa
        out = torch.empty((q.shape[0], q.shape[1]), device=dev)
        sdq.sdpa(t(q), t(k), t(v), out, heads)
        torch.cuda.synchronize()
        return out.cpu().numpy()
    return run


def _gpu_fc1_gelu(lin):
    import sdq

    w = sdq.Weight.from_host(lin["fc1"][0], lin["fc1"][1])
    return lambda h: sdq.qlinear_host(w, h, kind="gelu", bias=lin["fc1"][2])


def _ref_block(o, x, ctx, e, lin, nm, heads, cs, fusion, target=None, cs_tgt=None, phases=3,
               sdpa=None, fc1_gelu=None):
    """ovi_dit.cpp:205-268 on the oracle, step by step (sdpa, fc1_gelu:
    replacements for those two steps)."""
    x = x.copy()
    C = x.shape[1]
    L = lambda A, n, **kw: o.linear(A, lin[n][0], lin[n][1], bias=lin[n][2], **kw)  # noqa
    if sdpa is None:
        sdpa = lambda q, k, v, h: o.sdpa(q, k, v, h).astype(np.float32)  # noqa
    if fc1_gelu is None:
        fc1_gelu = lambda h: o.gelu_tanh(L(h, "fc1"))  # noqa
    if phases & 1:  # block_self_fwd + self_attn_fwd
        h = o.mod_rows(o.layernorm(x, 1e-6), e[0], e[1])
        q, k, v = L(h, "q"), L(h, "k"), L(h, "v")
        q, k = o.rmsnorm(q, nm["sa_nq"]), o.rmsnorm(k, nm["sa_nk"])
        if cs is not None:
            q, k = o.rope(q, cs, heads), o.rope(k, cs, heads)
        att = sdpa(q, k, v, heads)
        x = L(att, "o", epilogue="gated", gate=e[2], resid=x)
    if phases & 2:
        xin = x if fusion else o.layernorm(x, 1e-6, nm["ln3_w"], nm["ln3_b"])
        q = o.rmsnorm(L(xin, "cq"), nm["ca_nq"])
        k = o.rmsnorm(L(ctx, "ck"), nm["ca_nk"])
        xt = sdpa(q, k, L(ctx, "cv"), heads)
        if fusion:
            tn = o.layernorm(target, 1e-6, nm["pnf_w"], nm["pnf_b"])
            kt = o.rmsnorm(L(tn, "kf"), nm["nk_fusion"])
            if cs is not None:
                q = o.rope(q, cs, heads)
            if cs_tgt is not None:
                kt = o.rope(kt, cs_tgt, heads)
            xt = o.add(xt, sdpa(q, kt, L(tn, "vf"), heads))
        x = L(xt, "co", epilogue="resid", resid=x)
        h = o.mod_rows(o.layernorm(x, 1e-6), e[3], e[4])
        x = L(fc1_gelu(h), "fc2", epilogue="gated", gate=e[5], resid=x)
    return x


def _case(sdq_dev, oracle, dim, ffn, heads, M, Mc, Mt, fusion, rope, seed, phases=3, tol=1e-2):
    import torch

    import sdq

    print(f"[block-full] dim={dim} ffn={ffn} M={M} Mc={Mc} Mt={Mt} fusion={fusion} "
          f"rope={rope} phases={phases}", flush=True)
    lin = _weights(oracle, dim, ffn, seed, fusion)
    nm = _norms(oracle, dim, seed + 500)
    x = oracle.randn(M * dim, seed + 1).reshape(M, dim)
    ctx = oracle.randn(Mc * dim, seed + 2).reshape(Mc, dim)
    e = (oracle.randn(6 * dim, seed + 3).reshape(6, dim) * np.float32(0.3)).astype(np.float32)
    target = oracle.randn(Mt * dim, seed + 4).reshape(Mt, dim) if fusion else None
    if rope == "3d":
        cs = sdq.rope_table_3d(1, M // 4, 4)[:M] if M % 4 == 0 else sdq.rope_table_1d(M)
        cs_t = sdq.rope_table_1d(Mt, 128, 10000.0, 0.19676) if fusion else None
    elif rope in ("video", "audio"):
        # the 256x256/9-frame grids: video latents 3x16x16 = 768 tokens (RoPE-3D),
        # audio 157 tokens (RoPE-1D with the audio backbone's scaling,
        # ovi_dit.cpp:330, 656-658)
        vid = lambda n: sdq.rope_table_3d(3, 16, 16)[:n]  # noqa: E731
        aud = lambda n: sdq.rope_table_1d(n, 128, 10000.0, 0.19676)  # noqa: E731
        cs, cs_t = (vid(M), aud(Mt)) if rope == "video" else (aud(M), vid(Mt))
    else:
        cs, cs_t = None, None
    want = _ref_block(oracle, x, ctx, e, lin, nm, heads, cs, fusion, target, cs_t, phases)
    exact = _ref_block(oracle, x, ctx, e, lin, nm, heads, cs, fusion, target, cs_t, phases,
                       sdpa=_gpu_sdpa(sdq_dev), fc1_gelu=_gpu_fc1_gelu(lin))

    blk = sdq.DitBlock(lin, fusion)
    blk.set_norms(nm)
    dv = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa
    xd = dv(x)
    blk.step(xd, dv(ctx), dv(e), heads, cs=dv(cs), target=dv(target), cs_tgt=dv(cs_t),
             phases=phases)
    torch.cuda.synchronize()
    got = xd.cpu().numpy()
    assert np.isfinite(got).all()
    assert_bitexact(got, exact, "block vs oracle chain with the GPU's sdpa and GELU")
    err = np.abs(got.astype(np.float64) - want) / (np.abs(want).max() + 1e-30)
    print(f"  max rel err vs pure oracle {err.max():.3e}", flush=True)
    assert err.max() <= tol, float(err.max())
    assert np.abs(want - x).max() > 0.05 * np.abs(want).max()  # x moved far beyond the tolerance
    blk.free()


@pytest.mark.parametrize("fusion", [False, True])
def test_block_small(sdq_dev, oracle, fusion):
    _case(sdq_dev, oracle, 256, 512, 2, 100, 37, 60, fusion, "3d", 11 + fusion)


@pytest.mark.parametrize("phases", [1, 2])
def test_block_phases(sdq_dev, oracle, phases):
    _case(sdq_dev, oracle, 256, 512, 2, 64, 20, 33, True, "3d", 40 + phases, phases)


def test_block_no_rope_ragged(sdq_dev, oracle):
    _case(sdq_dev, oracle, 384, 768, 3, 77, 5, 0, False, "none", 61)


def test_block_real_width(sdq_dev, oracle):
    """dim 3072, ffn 14336, 24 heads (the Wan2.2 5B width), audio-sized rows
    against video-sized fusion target."""
    _case(sdq_dev, oracle, 3072, 14336, 24, 157, 64, 300, True, "3d", 71, tol=5e-2)


@pytest.mark.parametrize("M,Mt,rope", [(768, 157, "video"), (157, 768, "audio")])
def test_block_cfg5_real_width(sdq_dev, oracle, M, Mt, rope):
    """Config 5's fusion block whole at the real widths: the video branch
    (768 tokens, RoPE-3D on the 3x16x16 grid) against the 157 audio tokens,
    and the audio branch (157 tokens, RoPE-1D) against the 768 video tokens;
    text context 512 rows, 24 heads."""
    _case(sdq_dev, oracle, 3072, 14336, 24, M, 512, Mt, True, rope, 91 + M, tol=5e-2)


def test_block_fusion_no_rope(sdq_dev, oracle):
    _case(sdq_dev, oracle, 256, 512, 2, 48, 9, 20, True, "none", 81)


def test_block_step_errors(sdq_dev, oracle):
    import torch

    import sdq

    lin = _weights(oracle, 256, 512, 5, False)
    blk = sdq.DitBlock(lin, False)
    x = torch.zeros((8, 256), device=sdq_dev)
    ctx = torch.zeros((4, 256), device=sdq_dev)
    e = torch.zeros((6, 256), device=sdq_dev)
    with pytest.raises(RuntimeError, match="norm weights not set"):
        blk.step(x, ctx, e, 2)
    nm = _norms(oracle, 256, 9)
    blk.set_norms(nm)
    with pytest.raises(RuntimeError, match="head_dim must be 128"):
        blk.step(x, ctx, e, 4)
    small = torch.empty(16, dtype=torch.uint8, device=sdq_dev)
    with pytest.raises(RuntimeError, match="workspace too small"):
        blk.step(x, ctx, e, 2, ws=small)
    bad = dict(nm)
    bad.pop("ln3_b")
    with pytest.raises(RuntimeError, match="norm3"):
        blk.set_norms(bad)


def test_fusion_layer_two_branches(sdq_dev, oracle):
    """One fusion layer the way ovi_dit.cpp:726-734 runs it: audio self, video
    self, a snapshot of the audio tokens, audio cross+FFN against the video
    tokens, video cross+FFN against the snapshot. The GPU runs the two
    branches' phases on two streams with snapshots of both; bit-exact against
    the oracle chain in the reference's order (GPU attention and GELU steps)."""
    import torch

    import sdq

    dim, ffn, heads, Mv, Ma, Mc = 256, 512, 2, 64, 40, 24
    print(f"[fusion-layer] dim={dim} Mv={Mv} Ma={Ma}", flush=True)
    lin_v, lin_a = _weights(oracle, dim, ffn, 300, True), _weights(oracle, dim, ffn, 400, True)
    nm_v, nm_a = _norms(oracle, dim, 500), _norms(oracle, dim, 600)
    xv = oracle.randn(Mv * dim, 1).reshape(Mv, dim)
    xa = oracle.randn(Ma * dim, 2).reshape(Ma, dim)
    cv = oracle.randn(Mc * dim, 3).reshape(Mc, dim)
    ca = oracle.randn(Mc * dim, 4).reshape(Mc, dim)
    ev = (oracle.randn(6 * dim, 5).reshape(6, dim) * np.float32(0.3)).astype(np.float32)
    ea = (oracle.randn(6 * dim, 6).reshape(6, dim) * np.float32(0.3)).astype(np.float32)
    cs_v = sdq.rope_table_3d(4, 4, 4)
    cs_a = sdq.rope_table_1d(Ma, 128, 10000.0, 0.19676)
    run = dict(sdpa=_gpu_sdpa(sdq_dev))

    # the reference's order, on the oracle
    ra = _ref_block(oracle, xa, ca, ea, lin_a, nm_a, heads, cs_a, True, phases=1,
                    fc1_gelu=_gpu_fc1_gelu(lin_a), **run)
    rv = _ref_block(oracle, xv, cv, ev, lin_v, nm_v, heads, cs_v, True, phases=1,
                    fc1_gelu=_gpu_fc1_gelu(lin_v), **run)
    og_audio = ra.copy()
    ra = _ref_block(oracle, ra, ca, ea, lin_a, nm_a, heads, cs_a, True, rv, cs_v, phases=2,
                    fc1_gelu=_gpu_fc1_gelu(lin_a), **run)
    rv = _ref_block(oracle, rv, cv, ev, lin_v, nm_v, heads, cs_v, True, og_audio, cs_a, phases=2,
                    fc1_gelu=_gpu_fc1_gelu(lin_v), **run)

    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    bv, ba = sdq.DitBlock(lin_v, True), sdq.DitBlock(lin_a, True)
    bv.set_norms(nm_v)
    ba.set_norms(nm_a)
    gxv, gxa, gcv, gca, gev, gea = dv(xv), dv(xa), dv(cv), dv(ca), dv(ev), dv(ea)
    gcs_v, gcs_a = dv(cs_v), dv(cs_a)
    wsv = torch.empty(bv.workspace_bytes(Mv, Mc, Ma), dtype=torch.uint8, device=sdq_dev)
    wsa = torch.empty(ba.workspace_bytes(Ma, Mc, Mv), dtype=torch.uint8, device=sdq_dev)
    sv, sa = torch.cuda.Stream(), torch.cuda.Stream()
    cur = torch.cuda.current_stream()
    sv.wait_stream(cur)
    sa.wait_stream(cur)
    ba.step(gxa, gca, gea, heads, cs=gcs_a, ws=wsa, phases=sdq.SELF, stream=sa.cuda_stream)
    bv.step(gxv, gcv, gev, heads, cs=gcs_v, ws=wsv, phases=sdq.SELF, stream=sv.cuda_stream)
    with torch.cuda.stream(sa):
        og_a = gxa.clone()
    with torch.cuda.stream(sv):
        og_v = gxv.clone()
    sv.wait_stream(sa)
    sa.wait_stream(sv)
    ba.step(gxa, gca, gea, heads, cs=gcs_a, target=og_v, cs_tgt=gcs_v, ws=wsa,
            phases=sdq.CROSS_FFN, stream=sa.cuda_stream)
    bv.step(gxv, gcv, gev, heads, cs=gcs_v, target=og_a, cs_tgt=gcs_a, ws=wsv,
            phases=sdq.CROSS_FFN, stream=sv.cuda_stream)
    cur.wait_stream(sv)
    cur.wait_stream(sa)
    torch.cuda.synchronize()
    assert_bitexact(gxa.cpu().numpy(), ra, "audio branch")
    assert_bitexact(gxv.cpu().numpy(), rv, "video branch")
    bv.free()
    ba.free()
