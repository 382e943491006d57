"""The DiT block's int8 linear stack on the GPU (sd::gpu::DitBlock, the C++
host mirror's driver of ovi_dit.cpp:176-259) against the oracle.

Every GEMM output is bit-exact against the oracle's mlin restatement: the
concatenated q|k|v, cross k|v and k_fusion|v_fusion GEMMs against the three
(two) separate Linears, and the residual stream x after o (gated), cross o
(plain add) and fc2 (gated). The FFN hidden state is GELU-tanh, a tolerance
check (device tanhf vs libm); fc2 is then checked bit-exactly on the GPU's
own hidden state, so the chain fc1 -> GELU -> fc2 -> residual is covered
end to end. The full-size case (720p/121-frame token count, real widths)
checks sampled rows of every output."""
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
        W = oracle.randn(out * inp, seed + 10 * i).reshape(out, inp) * np.float32(0.02)
        q, s = oracle.quant_rows(W)
        b = oracle.randn(out, seed + 10 * i + 1) * np.float32(0.01)
        lin[n] = (q, s, b)
    return lin


def _inputs(oracle, M, Mc, Mt, dim, seed):
    r = lambda rows, k: oracle.randn(rows * dim, seed + k).reshape(rows, dim)  # noqa: E731
    return dict(h_sa=r(M, 1), att=r(M, 2), xq=r(M, 3), ctx=r(Mc, 4), tn=r(Mt, 5), xt=r(M, 6),
                h_ffn=r(M, 7), x=r(M, 8), gate_sa=oracle.randn(dim, seed + 9),
                gate_ffn=oracle.randn(dim, seed + 10))


def _run_block(blk, dev, inp, M, Mc, Mt, dim, ffn, fusion):
    import torch

    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in inp.items()}
    outs = dict(qkv=torch.empty((M, 3 * dim), device=dev), cq=torch.empty((M, dim), device=dev),
                ckv=torch.empty((Mc, 2 * dim), device=dev),
                kvt=torch.empty((max(Mt, 1), 2 * dim), device=dev),
                hid=torch.empty((M, ffn), device=dev))
    blk.forward(M=M, Mc=Mc, Mt=Mt if fusion else 0, **d, **outs)
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in outs.items()}
    res["x"] = d["x"].cpu().numpy()
    return res


def _check_small(oracle, got, lin, inp, fusion, Mt):
    L = lambda A, n, **kw: oracle.linear(A, lin[n][0], lin[n][1], bias=lin[n][2], **kw)  # noqa
    assert_bitexact(got["qkv"], np.concatenate([L(inp["h_sa"], n) for n in "qkv"], 1), "q|k|v")
    assert_bitexact(got["cq"], L(inp["xq"], "cq"), "cross q")
    assert_bitexact(got["ckv"], np.concatenate([L(inp["ctx"], n) for n in ("ck", "cv")], 1),
                    "cross k|v")
    if fusion:
        assert_bitexact(got["kvt"][:Mt],
                        np.concatenate([L(inp["tn"], n) for n in ("kf", "vf")], 1), "fusion k|v")
    want_hid = L(inp["h_ffn"], "fc1", epilogue="gelu")
    err = np.abs(got["hid"].astype(np.float64) - want_hid.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want_hid))), float(err.max())
    x = L(inp["att"], "o", epilogue="gated", gate=inp["gate_sa"], resid=inp["x"])
    x = L(inp["xt"], "co", epilogue="resid", resid=x)
    x = L(got["hid"], "fc2", epilogue="gated", gate=inp["gate_ffn"], resid=x)
    assert_bitexact(got["x"], x, "residual stream x")


@pytest.mark.parametrize("fusion", [True, False])
def test_block_stack_bitexact(sdq_dev, oracle, fusion):
    import sdq

    dim, ffn, M, Mc, Mt = 512, 1408, 300, 77, 45
    print(f"[block] dim={dim} ffn={ffn} M={M} Mc={Mc} Mt={Mt} fusion={fusion}", flush=True)
    lin = _weights(oracle, dim, ffn, 100, fusion)
    inp = _inputs(oracle, M, Mc, Mt, dim, 200)
    blk = sdq.DitBlock(lin, fusion)
    got = _run_block(blk, sdq_dev, inp, M, Mc, Mt, dim, ffn, fusion)
    _check_small(oracle, got, lin, inp, fusion, Mt)
    blk.free()


@pytest.mark.parametrize("M,Mt", [(768, 157), (157, 768)])
def test_block_stack_cfg5_real_width(sdq_dev, oracle, M, Mt):
    """Config 5's fusion-layer linear stack at the real widths (dim 3072, FFN
    14336, text context 512): the video branch (M=768 tokens, the 157 audio
    tokens as fusion target) and the audio branch (M=157, target 768), every
    output against the oracle."""
    import sdq

    dim, ffn, Mc = 3072, 14336, 512
    print(f"[block-cfg5] M={M} Mc={Mc} Mt={Mt}", flush=True)
    lin = _weights(oracle, dim, ffn, 600, True)
    inp = _inputs(oracle, M, Mc, Mt, dim, 700 + M)
    blk = sdq.DitBlock(lin, True)
    got = _run_block(blk, sdq_dev, inp, M, Mc, Mt, dim, ffn, True)
    _check_small(oracle, got, lin, inp, True, Mt)
    blk.free()


def test_block_device_weights_match_host_weights(sdq_dev, oracle):
    """The on-device construction path (concatenation + repack on the GPU)
    gives the same block as the host path, bit for bit."""
    import torch

    import sdq

    dim, ffn, M, Mc, Mt = 384, 1024, 130, 33, 20
    lin = _weights(oracle, dim, ffn, 300, True)
    inp = _inputs(oracle, M, Mc, Mt, dim, 400)
    host = sdq.DitBlock(lin, True)
    dlin = {n: tuple(torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev) for a in t)
            for n, t in lin.items()}
    devb = sdq.DitBlock(dlin, True)
    a = _run_block(host, sdq_dev, inp, M, Mc, Mt, dim, ffn, True)
    b = _run_block(devb, sdq_dev, inp, M, Mc, Mt, dim, ffn, True)
    for k in a:
        assert_bitexact(b[k][:Mt] if k == "kvt" else b[k], a[k][:Mt] if k == "kvt" else a[k], k)
    _check_small(oracle, a, lin, inp, True, Mt)


def test_block_errors(sdq_dev, oracle):
    import sdq

    lin = _weights(oracle, 64, 128, 500, False)
    bad = dict(lin)
    bad["o"] = (lin["o"][0][:, :32], lin["o"][1], lin["o"][2])
    with pytest.raises(sdq.SdqError, match="attention Linears"):
        sdq.DitBlock(bad, False)
    with pytest.raises(ValueError, match="missing Linear kf"):
        sdq.DitBlock(lin, True)


def test_block_fullsize_sampled(sdq_dev, oracle):
    """720p/121-frame video tokens (M=27280), dim 3072, FFN 14336, text
    context 512, fusion target 157 rows: every output checked bit-exactly at
    sampled rows (GELU: tolerance), the residual stream through all three
    updates."""
    import torch

    import sdq

    dim, ffn, M, Mc, Mt = 3072, 14336, 27280, 512, 157
    print(f"[block-full] dim={dim} ffn={ffn} M={M} Mc={Mc} Mt={Mt}", flush=True)
    lin = _weights(oracle, dim, ffn, 600, True)
    inp = _inputs(oracle, M, Mc, Mt, dim, 700)
    blk = sdq.DitBlock(lin, True)
    d = {k: torch.from_numpy(v).to(sdq_dev) for k, v in inp.items()}
    qkv = torch.empty((M, 3 * dim), device=sdq_dev)
    cq = torch.empty((M, dim), device=sdq_dev)
    ckv = torch.empty((Mc, 2 * dim), device=sdq_dev)
    kvt = torch.empty((Mt, 2 * dim), device=sdq_dev)
    hid = torch.empty((M, ffn), device=sdq_dev)
    blk.forward(M=M, Mc=Mc, Mt=Mt, qkv=qkv, cq=cq, ckv=ckv, kvt=kvt, hid=hid, **d)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 127, 128, 4097, M // 2, M - 129, M - 1], np.int64)
    rt = torch.from_numpy(rows).to(sdq_dev)
    L = lambda A, n, **kw: oracle.linear(A, lin[n][0], lin[n][1], bias=lin[n][2], **kw)  # noqa
    sub = {k: v[rows] for k, v in inp.items() if k in ("h_sa", "att", "xq", "xt", "h_ffn", "x")}
    assert_bitexact(qkv[rt].cpu().numpy(),
                    np.concatenate([L(sub["h_sa"], n) for n in "qkv"], 1), "q|k|v rows")
    assert_bitexact(cq[rt].cpu().numpy(), L(sub["xq"], "cq"), "cross q rows")
    assert_bitexact(ckv.cpu().numpy(),
                    np.concatenate([L(inp["ctx"], n) for n in ("ck", "cv")], 1), "cross k|v")
    assert_bitexact(kvt.cpu().numpy(),
                    np.concatenate([L(inp["tn"], n) for n in ("kf", "vf")], 1), "fusion k|v")
    h = hid[rt].cpu().numpy()
    want_h = L(sub["h_ffn"], "fc1", epilogue="gelu")
    err = np.abs(h.astype(np.float64) - want_h.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want_h))), float(err.max())
    x = L(sub["att"], "o", epilogue="gated", gate=inp["gate_sa"], resid=sub["x"])
    x = L(sub["xt"], "co", epilogue="resid", resid=x)
    x = L(h, "fc2", epilogue="gated", gate=inp["gate_ffn"], resid=x)
    assert_bitexact(d["x"][rt].cpu().numpy(), x, "residual stream rows")
    blk.free()


def test_block_with_norms_folded(sdq_dev, oracle):
    """The block with its norm1 / norm2 + modulation folded into q|k|v's and
    fc1's quantizers (io shift_sa/scale_sa, shift_ffn/scale_ffn): q|k|v read
    mod_rows(layernorm(x)) at block entry, fc1 the same of x after the
    cross-attention update; bit-exact against the oracle's layernorm,
    mod_rows and Linears (GELU hidden state: tolerance, then fc2 on it)."""
    import torch

    import sdq

    dim, ffn, M, Mc, Mt = 512, 1408, 300, 77, 45
    lin = _weights(oracle, dim, ffn, 900, True)
    inp = _inputs(oracle, M, Mc, Mt, dim, 1000)
    e = [oracle.randn(dim, 1100 + i) * np.float32(0.3) for i in range(4)]
    blk = sdq.DitBlock(lin, True)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(sdq_dev) for k, v in inp.items()}
    ed = [torch.from_numpy(a).to(sdq_dev) for a in e]
    outs = dict(qkv=torch.empty((M, 3 * dim), device=sdq_dev), cq=torch.empty((M, dim), device=sdq_dev),
                ckv=torch.empty((Mc, 2 * dim), device=sdq_dev),
                kvt=torch.empty((Mt, 2 * dim), device=sdq_dev),
                hid=torch.empty((M, ffn), device=sdq_dev))
    blk.forward(M=M, Mc=Mc, Mt=Mt, **d, **outs, shift_sa=ed[0], scale_sa=ed[1], shift_ffn=ed[2],
                scale_ffn=ed[3], eps=1e-6)
    torch.cuda.synchronize()
    L = lambda A, n, **kw: oracle.linear(A, lin[n][0], lin[n][1], bias=lin[n][2], **kw)  # noqa
    h_sa = oracle.mod_rows(oracle.layernorm(inp["x"], 1e-6), e[0], e[1])
    assert_bitexact(outs["qkv"].cpu().numpy(), np.concatenate([L(h_sa, n) for n in "qkv"], 1),
                    "q|k|v of the normed x")
    x = L(inp["att"], "o", epilogue="gated", gate=inp["gate_sa"], resid=inp["x"])
    x = L(inp["xt"], "co", epilogue="resid", resid=x)
    h_ffn = oracle.mod_rows(oracle.layernorm(x, 1e-6), e[2], e[3])
    hid = outs["hid"].cpu().numpy()
    want_hid = L(h_ffn, "fc1", epilogue="gelu")
    err = np.abs(hid.astype(np.float64) - want_hid.astype(np.float64))
    assert np.all(err <= 1e-6 * (1.0 + np.abs(want_hid))), float(err.max())
    x = L(hid, "fc2", epilogue="gated", gate=inp["gate_ffn"], resid=x)
    assert_bitexact(d["x"].cpu().numpy(), x, "residual stream with folded norms")
    blk.free()


def test_block_create_many_matches_single(sdq_dev, oracle):
    """Blocks built in one streamed upload (sd_dit_block_create_many) compute
    what blocks built one by one compute, bit for bit."""
    dim, ffn, M, Mc, Mt = 384, 1024, 130, 33, 20
    lins = [_weights(oracle, dim, ffn, 1200 + 50 * b, True) for b in range(3)]
    inp = _inputs(oracle, M, Mc, Mt, dim, 1400)
    import sdq

    many = sdq.DitBlock.create_many(lins, True)
    for b in range(3):
        one = sdq.DitBlock(lins[b], True)
        a = _run_block(many[b], sdq_dev, inp, M, Mc, Mt, dim, ffn, True)
        c = _run_block(one, sdq_dev, inp, M, Mc, Mt, dim, ffn, True)
        for k in a:
            assert_bitexact(a[k][:Mt] if k == "kvt" else a[k], c[k][:Mt] if k == "kvt" else c[k],
                            f"block {b} {k}")
        one.free()
    _check_small(oracle, _run_block(many[0], sdq_dev, inp, M, Mc, Mt, dim, ffn, True), lins[0],
                 inp, True, Mt)
    for blk in many:
        blk.free()


def _outs(torch, dev, M, Mc, Mt, dim, ffn):
    return dict(qkv=torch.empty((M, 3 * dim), device=dev), cq=torch.empty((M, dim), device=dev),
                ckv=torch.empty((Mc, 2 * dim), device=dev),
                kvt=torch.empty((max(Mt, 1), 2 * dim), device=dev),
                hid=torch.empty((M, ffn), device=dev))


@pytest.mark.parametrize("streams", [1, 2])
@pytest.mark.parametrize("dim,ffn,Mv,Ma,Mc", [(512, 1408, 300, 90, 77), (3072, 14336, 768, 157, 512)])
def test_block_pair_equals_oracle(sdq_dev, oracle, dim, ffn, Mv, Ma, Mc, streams):
    """forward_pair: the video and audio blocks of one twin layer with their
    attention Linears (and the two cross-o projections) grouped; every output
    of both blocks against the oracle. streams=2: the pair split over two
    streams (forward_pair2): the video block's own Linears on one, the audio
    block's and the video block's text / fusion k|v on the other."""
    import torch

    import sdq

    print(f"[block-pair] dim={dim} Mv={Mv} Ma={Ma} Mc={Mc} streams={streams}", flush=True)
    lv, la = _weights(oracle, dim, ffn, 900, True), _weights(oracle, dim, ffn, 950, True)
    iv, ia = _inputs(oracle, Mv, Mc, Ma, dim, 300), _inputs(oracle, Ma, Mc, Mv, dim, 400)
    bv, ba = sdq.DitBlock(lv, True), sdq.DitBlock(la, True)
    t = lambda inp: {k: torch.from_numpy(np.ascontiguousarray(v)).to(sdq_dev)  # noqa: E731
                     for k, v in inp.items()}
    dv, da = t(iv), t(ia)
    ov, oa = _outs(torch, sdq_dev, Mv, Mc, Ma, dim, ffn), _outs(torch, sdq_dev, Ma, Mc, Mv, dim, ffn)
    bv.forward_pair(ba, dict(M=Mv, Mc=Mc, Mt=Ma, **dv, **ov), dict(M=Ma, Mc=Mc, Mt=Mv, **da, **oa),
                    stream2=torch.cuda.Stream() if streams == 2 else None)
    torch.cuda.synchronize()
    for got_o, d, lin, inp, Mt in ((ov, dv, lv, iv, Ma), (oa, da, la, ia, Mv)):
        got = {k: v.cpu().numpy() for k, v in got_o.items()}
        got["x"] = d["x"].cpu().numpy()
        _check_small(oracle, got, lin, inp, True, Mt)
    bv.free()
    ba.free()


def test_block_pair_shared_hidden_buffer_stays_in_order(sdq_dev, oracle):
    """forward_pair with a second stream but one hidden-state buffer shared by
    both blocks: the two sides may not run side by side, so the pair runs in
    order on the first stream; x of both blocks equals the separate-buffer
    results."""
    import torch

    import sdq

    dim, ffn, Mv, Ma, Mc = 512, 1408, 200, 90, 64
    lv, la = _weights(oracle, dim, ffn, 1400, True), _weights(oracle, dim, ffn, 1450, True)
    iv, ia = _inputs(oracle, Mv, Mc, Ma, dim, 1500), _inputs(oracle, Ma, Mc, Mv, dim, 1600)
    bv, ba = sdq.DitBlock(lv, True), sdq.DitBlock(la, True)
    t = lambda inp: {k: torch.from_numpy(np.ascontiguousarray(v)).to(sdq_dev)  # noqa: E731
                     for k, v in inp.items()}
    xs = []
    for shared in (False, True):
        dv, da = t(iv), t(ia)
        ov, oa = _outs(torch, sdq_dev, Mv, Mc, Ma, dim, ffn), _outs(torch, sdq_dev, Ma, Mc, Mv, dim, ffn)
        if shared:
            oa["hid"] = ov["hid"][:Ma]  # the first Ma rows of the video block's buffer
        bv.forward_pair(ba, dict(M=Mv, Mc=Mc, Mt=Ma, **dv, **ov),
                        dict(M=Ma, Mc=Mc, Mt=Mv, **da, **oa), stream2=torch.cuda.Stream())
        torch.cuda.synchronize()
        xs.append((dv["x"].cpu().numpy(), da["x"].cpu().numpy()))
    assert_bitexact(xs[1][0], xs[0][0], "video x, shared hid")
    assert_bitexact(xs[1][1], xs[0][1], "audio x, shared hid")
    bv.free()
    ba.free()


def test_block_aliased_cross_q_runs_in_order(sdq_dev, oracle):
    """Cross q reading x itself (as a fusion block's q does): the o projection
    writes x, so the Linears may not be grouped; cross q must see x after
    x += o(att) * gate, exactly as the reference order has it."""
    import torch

    import sdq

    dim, ffn, M, Mc, Mt = 512, 1408, 200, 64, 40
    lin = _weights(oracle, dim, ffn, 1200, True)
    inp = _inputs(oracle, M, Mc, Mt, dim, 1300)
    blk = sdq.DitBlock(lin, True)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(sdq_dev) for k, v in inp.items()}
    d["xq"] = d["x"]  # the same tensor
    outs = _outs(torch, sdq_dev, M, Mc, Mt, dim, ffn)
    blk.forward(M=M, Mc=Mc, Mt=Mt, **d, **outs)
    torch.cuda.synchronize()
    L = lambda A, n, **kw: oracle.linear(A, lin[n][0], lin[n][1], bias=lin[n][2], **kw)  # noqa
    x1 = L(inp["att"], "o", epilogue="gated", gate=inp["gate_sa"], resid=inp["x"])
    assert_bitexact(outs["cq"].cpu().numpy(), L(x1, "cq"), "cross q on the updated x")
    x2 = L(inp["xt"], "co", epilogue="resid", resid=x1)
    x3 = L(outs["hid"].cpu().numpy(), "fc2", epilogue="gated", gate=inp["gate_ffn"], resid=x2)
    assert_bitexact(d["x"].cpu().numpy(), x3, "residual stream x")
    blk.free()
