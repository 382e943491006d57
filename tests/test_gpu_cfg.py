"""Classifier-free guidance as one stacked forward: the conditional and the
unconditional passes of a denoise step (denoise.cpp:95-98; the same latents
and time, different text contexts, skip-layer guidance on the unconditional
pass only, ovi_dit.cpp:713) run as one pass over both sets of rows.

The twin-backbone layer loop of OviDit::forward (ovi_dit.cpp:712-739) is
run both ways on small widths: two separate passes, and one stacked pass
(sd_dit_block_step_forward_batched: every Linear, norm and residual on the
stacked rows, the attention inside each half; the SLG layer on the
conditional half alone). The stacked pass must reproduce both passes bit for
bit, and each half must equal the oracle's layer loop for its pass (the
unconditional one skipping the SLG layer) with the GPU's sdpa and fc1 + GELU
substituted, the two steps that are not bit-exact by construction."""
import numpy as np
import pytest

from conftest import assert_bitexact
from test_gpu_block_full import _gpu_fc1_gelu, _gpu_sdpa, _norms, _ref_block, _weights

pytestmark = pytest.mark.gpu


def test_sdpa_batched_equals_separate(sdq_dev, oracle):
    import torch

    import sdq

    heads, Lq, Lk, B = 2, 50, 37, 3
    C = heads * 128
    q = torch.from_numpy(oracle.randn(B * Lq * C, 1).reshape(B * Lq, C)).to(sdq_dev)
    kv = torch.from_numpy(oracle.randn(B * Lk * 2 * C, 2).reshape(B * Lk, 2 * C)).to(sdq_dev)
    out = torch.empty((B * Lq, C), device=sdq_dev)
    sdq.sdpa(q, kv, kv, out, heads, kcol=0, vcol=C, batch=B)
    for b in range(B):
        one = torch.empty((Lq, C), device=sdq_dev)
        sdq.sdpa(q[b * Lq:(b + 1) * Lq], kv[b * Lk:(b + 1) * Lk], kv[b * Lk:(b + 1) * Lk], one,
                 heads, kcol=0, vcol=C)
        torch.cuda.synchronize()
        assert_bitexact(out[b * Lq:(b + 1) * Lq].cpu().numpy(), one.cpu().numpy(), f"seq {b}")


def _twin_pass(sdq, torch, layers, xv, xa, cv, ca, ev, ea, cs_v, cs_a, heads, slg, batch):
    """One OviDit::forward layer loop on the GPU (fusion layers): audio self,
    video self, snapshot of the audio tokens, audio cross+FFN against the
    video tokens, video cross+FFN against the snapshot. batch == 2: rows hold
    the conditional then the unconditional pass; the SLG layer runs on the
    conditional half only (the unconditional pass skips it)."""
    Mv, Ma = xv.shape[0] // batch, xa.shape[0] // batch
    Mcv, Mca = cv.shape[0] // batch, ca.shape[0] // batch
    for i, (bv, ba) in enumerate(layers):
        if batch == 1 and i == slg:
            continue  # the reference's `continue` (ovi_dit.cpp:713)
        n = 1 if (batch == 2 and i == slg) else batch
        xv_, xa_ = xv[:n * Mv], xa[:n * Ma]
        cv_, ca_ = cv[:n * Mcv], ca[:n * Mca]
        tv, ta = cs_v[:n * Mv], cs_a[:n * Ma]
        ba.step(xa_, ca_, ea[i], heads, cs=ta, phases=sdq.SELF, batch=n)
        bv.step(xv_, cv_, ev[i], heads, cs=tv, phases=sdq.SELF, batch=n)
        og_a = xa_.clone()
        ba.step(xa_, ca_, ea[i], heads, cs=ta, target=xv_, cs_tgt=tv, phases=sdq.CROSS_FFN,
                batch=n)
        bv.step(xv_, cv_, ev[i], heads, cs=tv, target=og_a, cs_tgt=ta, phases=sdq.CROSS_FFN,
                batch=n)
    torch.cuda.synchronize()


@pytest.mark.parametrize("slg", [1, -1])
def test_cfg_stacked_pass_equals_two_passes(sdq_dev, oracle, slg):
    import torch

    import sdq

    dim, ffn, heads, L = 256, 512, 2, 3
    Mv, Ma, Mc = 64, 20, 16
    print(f"[cfg] layers={L} slg={slg} Mv={Mv} Ma={Ma}", flush=True)
    layers, host = [], []
    for i in range(L):
        pair, hpair = [], []
        for j in range(2):
            lin = _weights(oracle, dim, ffn, 1000 + 100 * i + 50 * j, True)
            nm = _norms(oracle, dim, 3000 + 100 * i + 50 * j)
            blk = sdq.DitBlock(lin, True)
            blk.set_norms(nm)
            pair.append(blk)
            hpair.append((lin, nm))
        layers.append(tuple(pair))
        host.append(tuple(hpair))
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(sdq_dev)  # noqa
    r = lambda n, s: oracle.randn(n * dim, s).reshape(n, dim)  # noqa: E731
    xv0, xa0 = r(Mv, 1), r(Ma, 2)
    ctx = {k: r(Mc, 10 + i) for i, k in enumerate(("v_pos", "a_pos", "v_neg", "a_neg"))}
    hev = [(oracle.randn(6 * dim, 20 + i) * np.float32(0.3)).reshape(6, dim) for i in range(L)]
    hea = [(oracle.randn(6 * dim, 30 + i) * np.float32(0.3)).reshape(6, dim) for i in range(L)]
    ev, ea = [dv(e) for e in hev], [dv(e) for e in hea]
    cs_v = sdq.rope_table_3d(1, Mv // 4, 4)
    cs_a = sdq.rope_table_1d(Ma, 128, 10000.0, 0.19676)

    # two separate passes
    sep = {}
    for name, vk, ak, s in (("pos", "v_pos", "a_pos", -1), ("neg", "v_neg", "a_neg", slg)):
        xv, xa = dv(xv0), dv(xa0)
        _twin_pass(sdq, torch, layers, xv, xa, dv(ctx[vk]), dv(ctx[ak]), ev, ea, dv(cs_v),
                   dv(cs_a), heads, s, 1)
        sep[name] = (xv.cpu().numpy(), xa.cpu().numpy())
    # one stacked pass: rows [conditional; unconditional]
    xv = dv(np.concatenate([xv0, xv0]))
    xa = dv(np.concatenate([xa0, xa0]))
    cv = dv(np.concatenate([ctx["v_pos"], ctx["v_neg"]]))
    ca = dv(np.concatenate([ctx["a_pos"], ctx["a_neg"]]))
    _twin_pass(sdq, torch, layers, xv, xa, cv, ca, ev, ea, dv(np.concatenate([cs_v, cs_v])),
               dv(np.concatenate([cs_a, cs_a])), heads, slg, 2)
    gv, ga = xv.cpu().numpy(), xa.cpu().numpy()
    assert_bitexact(gv[:Mv], sep["pos"][0], "video, conditional half")
    assert_bitexact(gv[Mv:], sep["neg"][0], "video, unconditional half")
    assert_bitexact(ga[:Ma], sep["pos"][1], "audio, conditional half")
    assert_bitexact(ga[Ma:], sep["neg"][1], "audio, unconditional half")
    # the halves did diverge (different contexts, and SLG when on)
    assert np.abs(sep["pos"][0] - sep["neg"][0]).max() > 1e-2
    # each half against the oracle's layer loop for its own pass
    gsd = _gpu_sdpa(sdq_dev)
    fc1 = [(_gpu_fc1_gelu(lv), _gpu_fc1_gelu(la)) for (lv, _), (la, _) in host]
    for half, vk, ak, skip in ((0, "v_pos", "a_pos", -1), (1, "v_neg", "a_neg", slg)):
        xv, xa = xv0, xa0
        for i, ((lv, nv), (la, na)) in enumerate(host):
            if i == skip:
                continue  # skip-layer guidance, ovi_dit.cpp:713
            kv = dict(sdpa=gsd, fc1_gelu=fc1[i][0])
            ka = dict(sdpa=gsd, fc1_gelu=fc1[i][1])
            xa1 = _ref_block(oracle, xa, ctx[ak], hea[i], la, na, heads, cs_a, True, phases=1, **ka)
            xv1 = _ref_block(oracle, xv, ctx[vk], hev[i], lv, nv, heads, cs_v, True, phases=1, **kv)
            xa = _ref_block(oracle, xa1, ctx[ak], hea[i], la, na, heads, cs_a, True, xv1, cs_v, 2,
                            **ka)
            xv = _ref_block(oracle, xv1, ctx[vk], hev[i], lv, nv, heads, cs_v, True, xa1, cs_a, 2,
                            **kv)
        tag = "conditional" if half == 0 else f"unconditional (SLG layer {slg})"
        assert_bitexact(gv[half * Mv:(half + 1) * Mv], xv, f"video, {tag} half vs the oracle")
        assert_bitexact(ga[half * Ma:(half + 1) * Ma], xa, f"audio, {tag} half vs the oracle")
    for pair in layers:
        for b in pair:
            b.free()
