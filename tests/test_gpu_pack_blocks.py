"""Whole DiT blocks loaded from a .sdcpp pack (sd_dit_blocks_from_pack: the
12 int8 Linears, the norm vectors and modulation.modulation, with
OviDit::load_impl's names and checks, ovi_dit.cpp:397-415, 505-537) and run
as the reference's layer loop runs them (ovi_dit.cpp:712-739): per layer
e = time rows + the block's modulation bias, then the block forward.

The pack is written by the oracle's restatement of the packer
(pack_sdcpp.py:75-124); both loading paths (sequential file reads into the
pinned ring, and load_sdcpp's mapping) must give the same blocks. The chain
of layers is checked bit for bit against the oracle's reference block chain
with the GPU's own attention and fc1 + GELU substituted (the two steps that
are tolerance-only), and to a tolerance against the pure oracle chain."""
import numpy as np
import pytest

from conftest import assert_bitexact
from test_gpu_block_full import _gpu_fc1_gelu, _gpu_sdpa, _ref_block

pytestmark = pytest.mark.gpu

LIN = {"q": "self_attn.q", "k": "self_attn.k", "v": "self_attn.v", "o": "self_attn.o",
       "cq": "cross_attn.q", "ck": "cross_attn.k", "cv": "cross_attn.v", "co": "cross_attn.o",
       "kf": "cross_attn.k_fusion", "vf": "cross_attn.v_fusion", "fc1": "ffn.0", "fc2": "ffn.2"}
NORM = {"sa_nq": "self_attn.norm_q.weight", "sa_nk": "self_attn.norm_k.weight",
        "ca_nq": "cross_attn.norm_q.weight", "ca_nk": "cross_attn.norm_k.weight",
        "ln3_w": "norm3.weight", "ln3_b": "norm3.bias",
        "nk_fusion": "cross_attn.norm_k_fusion.weight",
        "pnf_w": "cross_attn.pre_attn_norm_fusion.weight",
        "pnf_b": "cross_attn.pre_attn_norm_fusion.bias"}


def _write_pack(oracle, path, prefix, layers, dim, ffn, fusion, seed):
    """float32 tensors of `layers` blocks under load_impl's names, packed."""
    t = {}
    for li in range(layers):
        B = f"{prefix}blocks.{li}."
        for j, (k, n) in enumerate(LIN.items()):
            if k in ("kf", "vf") and not fusion:
                continue
            out, inp = (ffn, dim) if k == "fc1" else ((dim, ffn) if k == "fc2" else (dim, dim))
            s = seed + 100 * li + 2 * j
            t[B + n + ".weight"] = oracle.randn(out * inp, s).reshape(out, inp) * np.float32(0.05)
            t[B + n + ".bias"] = oracle.randn(out, s + 1) * np.float32(0.02)
        for j, (k, n) in enumerate(NORM.items()):
            if k in ("nk_fusion", "pnf_w", "pnf_b") and not fusion:
                continue
            base = oracle.randu(dim, seed + 100 * li + 50 + j)
            t[B + n] = (base * np.float32(0.2) if k.endswith("_b") else
                        base * np.float32(0.5) + np.float32(1.0)).astype(np.float32)
        t[B + "modulation.modulation"] = (oracle.randn(6 * dim, seed + 100 * li + 70)
                                          * np.float32(0.1)).reshape(1, 6, dim)
    return oracle.write_sdcpp(path, t)


def _layer(written, prefix, li, fusion):
    B = f"{prefix}blocks.{li}."
    lin = {}
    for k, n in LIN.items():
        if k in ("kf", "vf") and not fusion:
            continue
        code, q, s = written[B + n + ".weight"]
        assert code == 0, f"{n} must be an int8 pack entry"
        lin[k] = (q, s, written[B + n + ".bias"][1])
    nm = {k: written[B + n][1] for k, n in NORM.items() if (B + n) in written}
    mod = written[B + "modulation.modulation"][1].reshape(6, -1)
    return lin, nm, mod


@pytest.mark.parametrize("fusion", [False, True])
def test_pack_blocks_chain(sdq_dev, oracle, tmp_path, fusion):
    import torch

    import sdq

    dim, ffn, heads, layers = 256, 512, 2, 2
    M, Mc, Mt = 96, 40, 33
    prefix = "audio_model." if fusion else "video_model."
    path = str(tmp_path / "blocks.sdcpp")
    print(f"[pack-blocks] fusion={fusion} layers={layers}", flush=True)
    written = _write_pack(oracle, path, prefix, layers, dim, ffn, fusion, 900 + 7 * fusion)
    by_file = sdq.DitBlock.from_pack(path, prefix, list(range(layers)), dim, ffn, fusion, True)
    by_map = sdq.DitBlock.from_pack(path, prefix, list(range(layers)), dim, ffn, fusion, False)

    x0 = oracle.randn(M * dim, 11).reshape(M, dim)
    ctx = oracle.randn(Mc * dim, 12).reshape(Mc, dim)
    t6 = (oracle.randn(6 * dim, 13) * np.float32(0.3)).reshape(6, dim)
    target = oracle.randn(Mt * dim, 14).reshape(Mt, dim) if fusion else None
    cs = sdq.rope_table_1d(M, 128, 10000.0, 0.19676)
    cs_t = sdq.rope_table_3d(1, Mt, 1) if fusion else None

    dv = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa
    results = []
    for blocks in (by_file, by_map):
        x = dv(x0)
        e = torch.empty((6, dim), device=sdq_dev)
        for blk in blocks:
            blk.modulation(dv(t6), e)
            blk.step(x, dv(ctx), e, heads, cs=dv(cs), target=dv(target), cs_tgt=dv(cs_t))
        torch.cuda.synchronize()
        results.append(x.cpu().numpy())
    assert_bitexact(results[0], results[1], "file-read blocks vs mapped blocks")

    want, exact = x0.copy(), x0.copy()
    for li in range(layers):
        lin, nm, mod = _layer(written, prefix, li, fusion)
        e = (t6 + mod).astype(np.float32)  # the reference's pv[k] += bv[k]
        want = _ref_block(oracle, want, ctx, e, lin, nm, heads, cs, fusion, target, cs_t)
        exact = _ref_block(oracle, exact, ctx, e, lin, nm, heads, cs, fusion, target, cs_t,
                           sdpa=_gpu_sdpa(sdq_dev), fc1_gelu=_gpu_fc1_gelu(lin))
    got = results[0]
    assert np.isfinite(got).all()
    assert_bitexact(got, exact, "pack blocks vs oracle chain with the GPU's sdpa and GELU")
    err = np.abs(got.astype(np.float64) - want) / (np.abs(want).max() + 1e-30)
    print(f"  max rel err vs pure oracle {err.max():.3e}", flush=True)
    assert err.max() <= 1e-2
    for b in by_file + by_map:
        b.free()
