#!/usr/bin/env python3
"""Benchmark of the int8 qGEMM hot path on one MI355X.

Workload (the headline metric, the north star): one int8 Linear of the Ovi DiT
FFN up-projection at 720p/121 frames, M=27280 tokens, K=3072, N=14336:
  Y[M,N] = qgemm(A, W) + bias  (sd::qgemm + mlin's bias pass, fused),
including the per-row activation quantizer pre-pass, fp32 output.
Inputs are synthetic and resident in HBM before timing: A ~ N(0,1),
W ~ N(0,0.02) quantized row-wise with the .sdcpp packer convention,
bias ~ N(0,0.01). A "step" is one full call (quantizer + GEMM).

Prints ONE JSON line (rank 0): value = TOPS = 2*M*N*K / (ms_per_step),
plus `roofline` for the dominant kernel (the GEMM, timed with HIP events on
its launch stream inside libsdq) and `cpu_baseline` (the reference's own
sd::qgemm compiled from its sources, oracle/_ref, timed on this host's cores
on a bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "self-evolve-diffusion-cpp_amd"))

M_NS, K_NS, N_NS = 27280, 3072, 14336
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--M", type=int, default=M_NS)
    ap.add_argument("--K", type=int, default=K_NS)
    ap.add_argument("--N", type=int, default=N_NS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-rows", type=int, default=0,
                    help="rows of the CPU baseline's sample (0: all M rows, the full workload)")
    ap.add_argument("--settle-ms", type=float, default=600.0,
                    help="after the W warmup steps, further untimed steps until this much wall "
                         "time has passed since the first warmup step (the shader clock's "
                         "power-limit transient; 0 = none)")
    ap.add_argument("--counters-json", default=os.path.join(ROOT, "profiles", "qgemm_ns_counters.json"),
                    help="rocprofv3 counter summary (written by --summarize-counters); its "
                         "figures are reported only when it was recorded on this library build")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="read rocprofv3 --pmc output directories (FETCH_SIZE, WRITE_SIZE, "
                         "MFMA busy, L2 hit passes of --profile-pass) and write --counters-json")
    ap.add_argument("--kernel-counters", nargs="+", metavar="DIR",
                    help="read rocprofv3 --pmc output directories of any bench.py run and print "
                         "per-kernel means (dispatches, FETCH_SIZE / WRITE_SIZE in bytes with the "
                         "--calibrate copy's scale, MFMA busy fraction, duration) as JSON")
    ap.add_argument("--calibrate", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="--kernel-counters: FETCH_SIZE and WRITE_SIZE runs of --profile-pass, "
                         "whose 1 GiB copy gives the bytes-per-KiB scale of each counter")
    ap.add_argument("--config", default="ns",
                    choices=["ns", "block", "blockfull", "ffn", "cross", "twin", "load"],
                    help="ns: the north-star qGEMM (the driver's bench line); block: one DiT "
                         "block's linear stack at 720p/121f; ffn: the 256x256/9f FFN pair; "
                         "cross: text/cross-attention and AdaLN projections; twin: the "
                         "full twin-backbone linear stack (28 and 30 layers); load: weight "
                         "upload of 8 blocks from host memory")
    ap.add_argument("--pack-dir", default=None,
                    help="--config load: directory for the temporary .sdcpp file (default: the "
                         "system temp directory)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="run a few steps plus a 1 GiB torch copy (the counter calibration "
                         "kernel) and exit; used under rocprofv3 --pmc")
    return ap.parse_args()


def profile_pass(torch, sdq, args):
    """Workload for `rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE -- python bench.py
    --profile-pass`: a few qgemm steps, then a plain 1 GiB device copy whose
    known traffic calibrates the counters."""
    dev = torch.device("cuda:0")
    sdq.init(0)
    A, q, s, bias = make_inputs(torch, dev, args.M, args.K, args.N)
    w = sdq.Weight.from_device(q, s)
    Y = torch.empty((args.M, args.N), device=dev, dtype=torch.float32)
    for _ in range(max(args.steps, 1)):
        sdq.qlinear(w, A, Y, kind="none", bias=bias)
    torch.cuda.synchronize()
    src = torch.ones(1 << 28, device=dev, dtype=torch.float32)  # 1 GiB
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": True, "copy_bytes": src.numel() * 4, "M": args.M,
                      "K": args.K, "N": args.N, "library": sdq.version(),
                      "cu_count": sdq.device_info()["cu_count"],
                      "plan": sdq.qlinear_plan(w, args.M)}), flush=True)


def make_inputs(torch, dev, M, K, N, seed=1234):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    A = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    W = torch.randn((N, K), generator=g, device=dev, dtype=torch.float32) * 0.02
    bias = torch.randn((N,), generator=g, device=dev, dtype=torch.float32) * 0.01
    # .sdcpp packer convention (tools/quantize/pack_sdcpp.py:45-51)
    amax = W.abs().amax(dim=1)
    safe = torch.where(amax > 0, amax, torch.ones_like(amax))
    q = torch.clamp(torch.round(W * (127.0 / safe)[:, None]), -127, 127).to(torch.int8)
    s = (amax / 127.0).to(torch.float32)
    del W
    return A, q.contiguous(), s.contiguous(), bias


def _dev_weights(torch, dev, out, inp, seed):
    """Synthetic packed int8 weights on the device: values in [-127, 127] and
    per-row scales ~ 0.02*max|N(0,1)|/127 (timing only; parity is tested)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randint(-127, 128, (out, inp), generator=g, device=dev, dtype=torch.int8)
    s = (torch.rand((out,), generator=g, device=dev) * 2e-4 + 4e-4).float()
    b = torch.randn((out,), generator=g, device=dev) * 0.01
    return q, s, b


def _block_weights(torch, dev, dim, ffn, seed, fusion=True):
    names = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "kf", "vf", "fc1", "fc2")
    lin = {}
    for i, n in enumerate(names):
        if n in ("kf", "vf") and not fusion:
            continue
        out, inp = (ffn, dim) if n == "fc1" else ((dim, ffn) if n == "fc2" else (dim, dim))
        lin[n] = _dev_weights(torch, dev, out, inp, seed + i)
    return lin


def _block_io(torch, dev, M, Mc, Mt, dim, ffn):
    r = lambda rows: torch.randn((rows, dim), device=dev)  # noqa: E731
    return dict(M=M, Mc=Mc, Mt=Mt, h_sa=r(M), att=r(M), xq=r(M), ctx=r(Mc), tn=r(max(Mt, 1)),
                xt=r(M), h_ffn=r(M), x=r(M), gate_sa=torch.randn(dim, device=dev),
                gate_ffn=torch.randn(dim, device=dev),
                qkv=torch.empty((M, 3 * dim), device=dev), cq=torch.empty((M, dim), device=dev),
                ckv=torch.empty((Mc, 2 * dim), device=dev),
                kvt=torch.empty((max(Mt, 1), 2 * dim), device=dev),
                hid=torch.empty((M, ffn), device=dev))


def _timed(torch, fn, warmup, steps):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def _kernel_split(sdq, fn, steps):
    sdq.profile_begin()
    for _ in range(steps):
        fn()
    prof = sdq.profile_end()
    return {k: round(t / steps, 5) for k, (n, t) in prof.items()}


def _block_full(torch, sdq, blk, io, dim, M, Mc, Mt, steps=3):
    """The whole block (sd_dit_block_step_forward): norms, RoPE on the
    31x22x40 token grid, the three attentions and the Linears, the audio rows
    as fusion target. Returns (ms per block, kernel split, ops)."""
    import numpy as np

    dev = torch.device("cuda:0")
    blk.set_norms({n: np.ones(dim, np.float32) for n in sdq.NORM_NAMES})
    heads = dim // 128
    cs = torch.from_numpy(sdq.rope_table_3d(31, 22, 40)).to(dev)
    cs_a = torch.from_numpy(sdq.rope_table_1d(Mt, 128, 10000.0, 0.19676)).to(dev)
    e6 = torch.randn((6, dim), device=dev) * 0.3
    ws = torch.empty(blk.workspace_bytes(M, Mc, Mt), dtype=torch.uint8, device=dev)
    xf = torch.randn((M, dim), device=dev)
    fn = lambda: blk.step(xf, io["ctx"], e6, heads, cs=cs, target=io["tn"][:Mt],  # noqa: E731
                          cs_tgt=cs_a, ws=ws)
    ms = _timed(torch, fn, 1, steps)
    return ms, _kernel_split(sdq, fn, 1), blk.step_ops(M, Mc, Mt)


def bench_block_full(torch, sdq, args):
    """Config 3 as a whole block: M=27280 video tokens (31x22x40), text
    context 512 rows, 157 audio rows as fusion target, 24 heads."""
    dev = torch.device("cuda:0")
    dim, ffn, M, Mc, Mt = 3072, 14336, 27280, 512, 157
    blk = sdq.DitBlock(_block_weights(torch, dev, dim, ffn, 11), True)
    io = _block_io(torch, dev, M, Mc, Mt, dim, ffn)
    ms, split, ops = _block_full(torch, sdq, blk, io, dim, M, Mc, Mt, max(args.steps // 20, 3))
    return {"metric": "DiT block forward incl. attention (config 3), TFLOP/s",
            "value": round(ops / ms / 1e9, 2), "unit": "TFLOP/s (int8 Linears + fp32 attention)",
            "ms_per_block": round(ms, 3), "ops": ops, "dtype": "int8+f32",
            "config": {"workload": "whole DiT block M=27280 (31x22x40) dim=3072 ffn=14336 "
                                   "heads=24 ctx=512 fusion=157", "kernel_ms_per_block": split}}


def bench_block(torch, sdq, args):
    """Config 3: one DiT block's linear stack at 720p/121 frames (M=27280
    video tokens, dim 3072, FFN 14336), text context 512 rows, fusion target
    157 audio rows; q|k|v, cross k|v and k_fusion|v_fusion as single GEMMs."""
    dev = torch.device("cuda:0")
    dim, ffn, M, Mc, Mt = 3072, 14336, 27280, 512, 157
    blk = sdq.DitBlock(_block_weights(torch, dev, dim, ffn, 11), True)
    io = _block_io(torch, dev, M, Mc, Mt, dim, ffn)
    fn = lambda: blk.forward(**io)  # noqa: E731
    ms = _timed(torch, fn, max(args.warmup // 5, 2), max(args.steps // 10, 3))
    ops = blk.ops(M, Mc, Mt)
    split = _kernel_split(sdq, fn, 2)
    # the same block with norm1/norm2 + modulation folded into q|k|v's and
    # fc1's quantizers (x is normalized in place of the given h_sa / h_ffn)
    mods = {k: torch.randn(dim, device=dev) * 0.3
            for k in ("shift_sa", "scale_sa", "shift_ffn", "scale_ffn")}
    fn_ln = lambda: blk.forward(**io, **mods, eps=1e-6)  # noqa: E731
    ms_ln = _timed(torch, fn_ln, max(args.warmup // 5, 2), max(args.steps // 10, 3))
    split_ln = _kernel_split(sdq, fn_ln, 2)
    ms_full, split_full, ops_full = _block_full(torch, sdq, blk, io, dim, M, Mc, Mt)
    return {"metric": "DiT block int8 linear stack (config 3), TOPS", "value": round(ops / ms / 1e9, 2),
            "unit": "TOPS", "ms_per_block": round(ms, 4), "ops": ops, "dtype": "int8",
            "config": {"workload": "DiT block linears M=27280 dim=3072 ffn=14336 ctx=512 "
                                   "fusion=157", "kernel_ms_per_block": split,
                       "ms_per_block_norms_folded": round(ms_ln, 4),
                       "kernel_ms_per_block_norms_folded": split_ln,
                       "ms_per_block_full": round(ms_full, 3),
                       "ops_block_full": ops_full,
                       "kernel_ms_per_block_full": split_full}}


def bench_ffn(torch, sdq, args):
    """Config 2: the FFN pair at 256x256/9 frames as the config states it
    (M=768): up 14336x3072 + GELU, then down 3072x14336 + gated residual."""
    dev = torch.device("cuda:0")
    M, dim, ffn = 768, 3072, 14336
    q1, s1, b1 = _dev_weights(torch, dev, ffn, dim, 21)
    q2, s2, b2 = _dev_weights(torch, dev, dim, ffn, 22)
    w1, w2 = sdq.Weight.from_device(q1, s1), sdq.Weight.from_device(q2, s2)
    x, h = torch.randn((M, dim), device=dev), torch.randn((M, dim), device=dev)
    hid = torch.empty((M, ffn), device=dev)
    gate = torch.randn(dim, device=dev)

    def fn():  # sdq_ffn: fc1's epilogue hands hid's row maxima to fc2's quantizer
        sdq.ffn(w1, b1, w2, b2, h, gate, hid, x)

    def fn_pair():  # the same as two separate Linears
        sdq.qlinear(w1, h, hid, kind="gelu", bias=b1)
        sdq.qlinear(w2, hid, x, kind="gated", bias=b2, gate=gate, resid=x)
    ms = _timed(torch, fn, args.warmup, args.steps)
    ms_pair = _timed(torch, fn_pair, args.warmup, args.steps)
    ops = 2.0 * 2 * M * dim * ffn
    return {"metric": "FFN pair int8 (config 2), TOPS", "value": round(ops / ms / 1e9, 2),
            "unit": "TOPS", "ms_per_pair": round(ms, 5), "dtype": "int8",
            "config": {"workload": "FFN up+GELU, down+gated residual, M=768 (sdq_ffn)",
                       "kernel_ms": _kernel_split(sdq, fn, 5),
                       "two_qlinear_calls_ms": round(ms_pair, 5),
                       "two_qlinear_calls_kernel_ms": _kernel_split(sdq, fn_pair, 5)}}


def bench_cross(torch, sdq, args):
    """Config 4: text_embedding.0 [512,4096]x[3072,4096], the real cross k|v
    [512,3072]x[6144,3072], video-token Q [27280,3072]x[3072,3072], and the
    AdaLN time projection [1,3072]x[18432,3072] (HBM-bound: reported in GB/s)."""
    dev = torch.device("cuda:0")
    out = {"metric": "cross-attention / AdaLN projections (config 4)", "unit": "us", "dtype": "int8",
           "ops": {}}
    for name, (M, K, N) in {"text_embedding.0": (512, 4096, 3072), "cross_kv": (512, 3072, 6144),
                            "video_q": (27280, 3072, 3072), "adaln_tp1": (1, 3072, 18432)}.items():
        q, s, b = _dev_weights(torch, dev, N, K, 31)
        w = sdq.Weight.from_device(q, s)
        A = torch.randn((M, K), device=dev)
        Y = torch.empty((M, N), device=dev)
        fn = lambda: sdq.qlinear(w, A, Y, kind="none", bias=b)  # noqa: E731
        ms = _timed(torch, fn, args.warmup, args.steps)
        bytes_ = 4.0 * M * K + N * K + 8.0 * N + 4.0 * M * N
        out["ops"][name] = {"M": M, "K": K, "N": N, "us": round(ms * 1e3, 2),
                            "TOPS": round(2.0 * M * N * K / ms / 1e9, 2),
                            "GBps": round(bytes_ / ms / 1e6, 1)}
        w.free()
    out["value"] = out["ops"]["adaln_tp1"]["us"]
    return out


def bench_twin(torch, sdq, args):
    """Config 5: the twin-backbone linear stack at 256x256/9 frames: video
    M=768 and audio M=157 tokens, dim 3072, FFN 14336, text context 512, every
    layer a fusion layer (k_fusion|v_fusion on the other branch's tokens);
    28 layers (as stated) and 30 (the real model). Weights are device-resident
    (10.2 / 10.95 GB int8): the pass streams them once, an HBM-bound stack.
    The branches run on two streams, joined after every layer (the one-stream
    time is reported beside it). The one-time GPU repack of all blocks is
    timed separately."""
    dev = torch.device("cuda:0")
    dim, ffn, Mv, Ma, Mc = 3072, 14336, 768, 157, 512
    res = {"metric": "twin-backbone int8 linear stack (config 5)", "unit": "ms", "dtype": "int8",
           "layers": {}}
    blocks = []
    wbytes = 0
    t_repack = 0.0
    sv, sa = torch.cuda.Stream(), torch.cuda.Stream()
    for layers in (28, 30):
        while len(blocks) < 2 * layers:
            lin = _block_weights(torch, dev, dim, ffn, 1000 + len(blocks))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            blocks.append(sdq.DitBlock(lin, True))
            torch.cuda.synchronize()
            t_repack += time.perf_counter() - t0
            wbytes += sum(q.numel() for q, _, _ in lin.values())
            del lin
        iov = _block_io(torch, dev, Mv, Mc, Ma, dim, ffn)
        ioa = _block_io(torch, dev, Ma, Mc, Mv, dim, ffn)

        def fn():
            for i in range(layers):
                blocks[2 * i].forward(**iov)
                blocks[2 * i + 1].forward(**ioa)

        # The two branches of a layer are independent given the previous
        # layer's outputs (each reads the other's tokens only through the
        # fusion k|v, computed from layer inputs): run them on two streams
        # (default priority, created once), joined after every layer.
        def fn2():
            cur = torch.cuda.current_stream()
            sv.wait_stream(cur)
            sa.wait_stream(cur)
            for i in range(layers):
                blocks[2 * i].forward(stream=sv.cuda_stream, **iov)
                blocks[2 * i + 1].forward(stream=sa.cuda_stream, **ioa)
                sv.wait_stream(sa)
                sa.wait_stream(sv)
            cur.wait_stream(sv)
            cur.wait_stream(sa)
        # Both blocks of a layer through forward_pair (one stream): their
        # attention Linears and the two cross-attention output projections
        # each as one grouped launch (sdq_qlinear_group).
        def fn3():
            for i in range(layers):
                blocks[2 * i].forward_pair(blocks[2 * i + 1], iov, ioa)

        # forward_pair on two streams: the video block's own Linears on one,
        # the audio block's and the video block's text / fusion k|v on the
        # other (forked and joined inside every layer)
        def fn4():
            for i in range(layers):
                blocks[2 * i].forward_pair(blocks[2 * i + 1], iov, ioa, stream2=sa)

        ms_seq = _timed(torch, fn, 2, max(args.steps // 10, 3))
        ms_two = _timed(torch, fn2, 2, max(args.steps // 10, 3))
        ms_grp = _timed(torch, fn3, 2, max(args.steps // 10, 3))
        ms_grp2 = _timed(torch, fn4, 2, max(args.steps // 10, 3))
        ms = min(ms_two, ms_grp, ms_grp2)
        ops = sum(blocks[2 * i].ops(Mv, Mc, Ma) + blocks[2 * i + 1].ops(Ma, Mc, Mv)
                  for i in range(layers))
        lw = wbytes * (2 * layers) / len(blocks)  # bytes of the blocks this pass uses
        res["layers"][str(layers)] = {"ms_per_pass": round(ms, 4), "TOPS": round(ops / ms / 1e9, 2),
                                      "ms_per_pass_grouped_pair": round(ms_grp, 4),
                                      "ms_per_pass_pair_two_streams": round(ms_grp2, 4),
                                      "ms_per_pass_two_streams": round(ms_two, 4),
                                      "ms_per_pass_one_stream": round(ms_seq, 4),
                                      "kernel_ms_grouped_pair": (_kernel_split(sdq, fn3, 1)
                                                                 if layers == 28 else None),
                                      "weight_GB": round(lw / 1e9, 3),
                                      "weight_stream_GBps": round(lw / ms / 1e6, 1),
                                      "repack_ms_total": round(t_repack * 1e3, 1)}
    # The whole twin backbone on the GPU (sd_dit_block_step_forward): norms,
    # RoPE, the attentions and the Linears of every layer, in the order of a
    # fusion layer (ovi_dit.cpp:726-734): both self phases (two streams),
    # snapshots of both branches, then both cross+FFN phases, each reading
    # the other's snapshot (two streams). 30 layers.
    import numpy as np

    layers, slg = 30, 9  # gen.cpp:258: skip-layer guidance at layer 9
    heads = dim // 128
    ones = {n: np.ones(dim, np.float32) for n in sdq.NORM_NAMES}
    for b in blocks[:2 * layers]:
        b.set_norms(ones)
    tab_v = sdq.rope_table_3d(3, 16, 16)  # 768 video tokens
    tab_a = sdq.rope_table_1d(Ma, 128, 10000.0, 0.19676)
    e_v = [torch.randn((6, dim), device=dev) * 0.1 for _ in range(layers)]
    e_a = [torch.randn((6, dim), device=dev) * 0.1 for _ in range(layers)]

    def whole(batch, skip):
        """The 30-layer forward over `batch` stacked passes (batch 2: the
        conditional and unconditional forwards of one guidance step, each with
        its own text context; the unconditional half skips layer `skip`,
        which then runs on the conditional half alone)."""
        cs_v = torch.from_numpy(np.concatenate([tab_v] * batch)).to(dev)
        cs_a = torch.from_numpy(np.concatenate([tab_a] * batch)).to(dev)
        xv = torch.randn((batch * Mv, dim), device=dev)
        xa = torch.randn((batch * Ma, dim), device=dev)
        og_v, og_a = torch.empty_like(xv), torch.empty_like(xa)
        ctx_v = torch.randn((batch * Mc, dim), device=dev)
        ctx_a = torch.randn((batch * Mc, dim), device=dev)
        ws_v = torch.empty(blocks[0].workspace_bytes(batch * Mv, batch * Mc, batch * Ma),
                           dtype=torch.uint8, device=dev)
        ws_a = torch.empty(blocks[1].workspace_bytes(batch * Ma, batch * Mc, batch * Mv),
                           dtype=torch.uint8, device=dev)

        def fn():
            cur = torch.cuda.current_stream()
            sv.wait_stream(cur)
            sa.wait_stream(cur)
            for i in range(layers):
                n = batch
                if i == skip:
                    if batch == 1:
                        continue  # the reference's `continue` (ovi_dit.cpp:713)
                    n = 1
                bv, ba = blocks[2 * i], blocks[2 * i + 1]
                xv_, xa_, ov, oa = xv[:n * Mv], xa[:n * Ma], og_v[:n * Mv], og_a[:n * Ma]
                cv, ca = ctx_v[:n * Mc], ctx_a[:n * Mc]
                tv, ta = cs_v[:n * Mv], cs_a[:n * Ma]
                ba.step(xa_, ca, e_a[i], heads, cs=ta, ws=ws_a, phases=sdq.SELF,
                        stream=sa.cuda_stream, batch=n)
                bv.step(xv_, cv, e_v[i], heads, cs=tv, ws=ws_v, phases=sdq.SELF,
                        stream=sv.cuda_stream, batch=n)
                with torch.cuda.stream(sa):
                    oa.copy_(xa_)
                with torch.cuda.stream(sv):
                    ov.copy_(xv_)
                sv.wait_stream(sa)
                sa.wait_stream(sv)
                ba.step(xa_, ca, e_a[i], heads, cs=ta, target=ov, cs_tgt=tv, ws=ws_a,
                        phases=sdq.CROSS_FFN, stream=sa.cuda_stream, batch=n)
                bv.step(xv_, cv, e_v[i], heads, cs=tv, target=oa, cs_tgt=ta, ws=ws_v,
                        phases=sdq.CROSS_FFN, stream=sv.cuda_stream, batch=n)
                sv.wait_stream(sa)
                sa.wait_stream(sv)
            cur.wait_stream(sv)
            cur.wait_stream(sa)
        ms = _timed(torch, fn, 2, max(args.steps // 10, 3))
        assert bool(torch.isfinite(xv).all()) and bool(torch.isfinite(xa).all())
        return ms, fn

    ms_full, fn_full = whole(1, -1)
    ops_full = sum(blocks[2 * i].step_ops(Mv, Mc, Ma) + blocks[2 * i + 1].step_ops(Ma, Mc, Mv)
                   for i in range(layers))
    res["whole_blocks_30"] = {"ms_per_pass": round(ms_full, 4),
                              "TFLOPs": round(ops_full / ms_full / 1e9, 2),
                              "kernel_ms_per_pass": _kernel_split(sdq, fn_full, 1)}
    # Classifier-free guidance (denoise.cpp:95-98 runs the conditional pass,
    # then the unconditional one with SLG): both passes' rows stacked through
    # the whole forward (sd_dit_block_step_forward_batched; bit-identical to
    # the two passes), against the two passes one after the other.
    ms_uncond, _ = whole(1, slg)
    ms_pair, fn_pair = whole(2, slg)
    res["cfg_pair_whole_30"] = {"ms_per_cond_uncond_pair": round(ms_pair, 4),
                                "two_separate_passes_ms": round(ms_full + ms_uncond, 4),
                                "slg_layer": slg,
                                "kernel_ms_per_pair": _kernel_split(sdq, fn_pair, 1)}
    res["value"] = res["layers"]["28"]["ms_per_pass"]
    return res


def bench_load(torch, sdq, args):
    """Weight upload from host memory (the streaming loader): 8 DiT blocks at the real
    widths (dim 3072, FFN 14336, fusion: 1.46 GB of int8 + scales, host arrays
    like load_sdcpp's views), one block at a time (per Linear: host concat,
    pageable copy, repack) vs one streamed upload (pinned ring, async copies,
    repack overlap)."""
    import numpy as np

    dim, ffn, nb = 3072, 14336, 8
    rng = np.random.default_rng(5)
    names = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "kf", "vf", "fc1", "fc2")
    lins = []
    for b in range(nb):
        lin = {}
        for n in names:
            out, inp = (ffn, dim) if n == "fc1" else ((dim, ffn) if n == "fc2" else (dim, dim))
            lin[n] = (rng.integers(-127, 128, (out, inp), dtype=np.int8),
                      rng.uniform(1e-4, 1e-3, out).astype(np.float32),
                      rng.standard_normal(out).astype(np.float32))
        lins.append(lin)
    nbytes = sum(q.nbytes + s.nbytes for lin in lins for q, s, _ in lin.values())
    sdq.DitBlock(lins[0], True).free()  # warm up the path
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    one = [sdq.DitBlock(lin, True) for lin in lins]
    torch.cuda.synchronize()
    t_one = time.perf_counter() - t0
    for blk in one:
        blk.free()
    t0 = time.perf_counter()
    many = sdq.DitBlock.create_many(lins, True)
    torch.cuda.synchronize()
    t_many = time.perf_counter() - t0
    for blk in many:
        blk.free()
    files = _bench_pack_file(torch, sdq, args, lins, dim, ffn, nbytes)
    return {"metric": "DiT block weight upload from host memory", "unit": "GB/s",
            "value": round(nbytes / t_many / 1e9, 2), "dtype": "int8",
            "config": {"workload": f"{nb} blocks dim={dim} ffn={ffn} fusion, {nbytes / 1e9:.2f} GB",
                       "streamed_s": round(t_many, 3), "block_by_block_s": round(t_one, 3),
                       "block_by_block_GBps": round(nbytes / t_one / 1e9, 2),
                       "from_pack_file": files}}


_PACK_NAMES = {"q": "self_attn.q", "k": "self_attn.k", "v": "self_attn.v", "o": "self_attn.o",
               "cq": "cross_attn.q", "ck": "cross_attn.k", "cv": "cross_attn.v",
               "co": "cross_attn.o", "kf": "cross_attn.k_fusion", "vf": "cross_attn.v_fusion",
               "fc1": "ffn.0", "fc2": "ffn.2"}
_PACK_VECS = ("self_attn.norm_q.weight", "self_attn.norm_k.weight", "cross_attn.norm_q.weight",
              "cross_attn.norm_k.weight", "norm3.weight", "norm3.bias",
              "cross_attn.norm_k_fusion.weight", "cross_attn.pre_attn_norm_fusion.weight",
              "cross_attn.pre_attn_norm_fusion.bias")


def _write_int8_pack(path, lins, dim):
    """A .sdcpp v1 file (src/serde/sdcpp.cpp:1-8) of already-quantized blocks
    under load_impl's names: each Linear's int8 rows then its f32 scales
    (code 0), biases / norms / modulation raw f32 (code 1), back to back."""
    import struct

    import numpy as np

    ents = []
    for b, lin in enumerate(lins):
        B = f"video_model.blocks.{b}."
        for k, (q, s, bias) in lin.items():
            ents.append((B + _PACK_NAMES[k] + ".weight", 0, q.shape, [q, s]))
            ents.append((B + _PACK_NAMES[k] + ".bias", 1, bias.shape, [bias]))
        for n in _PACK_VECS:
            ents.append((B + n, 1, (dim,), [np.ones(dim, np.float32)]))
        ents.append((B + "modulation.modulation", 1, (1, 6, dim), [np.zeros(6 * dim, np.float32)]))
    with open(path, "wb") as f:
        f.write(b"SDCP" + struct.pack("<II", 1, len(ents)))
        off = 0
        for name, code, dims, parts in ents:
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<BI", code, len(dims)))
            f.write(struct.pack(f"<{len(dims)}q", *dims) + struct.pack("<Q", off))
            off += sum(p.nbytes for p in parts)
        for _, _, _, parts in ents:
            for p in parts:
                f.write(np.ascontiguousarray(p).tobytes())
        f.flush()
        os.fsync(f.fileno())


def _drop_cache(path):
    """Evicts the file's clean pages from the page cache (no privileges
    needed for a file of one's own); False when the filesystem keeps them."""
    fd = os.open(path, os.O_RDONLY)
    try:
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    finally:
        os.close(fd)


def _fs_type(path):
    best, fs = "", "?"
    try:
        with open("/proc/mounts") as f:
            for ln in f:
                dev, mnt, typ = ln.split()[:3]
                if path.startswith(mnt) and len(mnt) > len(best):
                    best, fs = mnt, typ
    except OSError:
        pass
    return fs


def _bench_pack_file(torch, sdq, args, lins, dim, ffn, nbytes):
    """The same blocks loaded whole from a .sdcpp file (sd_dit_blocks_from_pack):
    sequential file reads into the pinned ring vs load_sdcpp's mapping, each
    from a cold page cache (the file's pages evicted first) and warm."""
    import tempfile

    d = args.pack_dir or tempfile.gettempdir()
    path = os.path.join(d, f"sdq_bench_{os.getpid()}.sdcpp")
    _write_int8_pack(path, lins, dim)
    try:
        out = {"file_bytes": os.path.getsize(path), "filesystem": _fs_type(os.path.abspath(path))}
        layers = list(range(len(lins)))
        for mode, file_reads in (("file_reads", True), ("mapped", False)):
            for temp in ("cold", "warm"):
                if temp == "cold":
                    _drop_cache(path)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                blocks = sdq.DitBlock.from_pack(path, "video_model.", layers, dim, ffn, True,
                                                file_reads)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                for b in blocks:
                    b.free()
                out[f"{mode}_{temp}_s"] = round(dt, 3)
                out[f"{mode}_{temp}_GBps"] = round(nbytes / dt / 1e9, 2)
        return out
    finally:
        os.unlink(path)


def cpu_baseline(args, K, N):
    """The reference's sd::qgemm (oracle/_ref) on a row sample of the same
    workload; best of 3 after one warmup (tests/test_core.cpp:40-49)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import pyoracle

    rows = args.cpu_sample_rows if args.cpu_sample_rows > 0 else args.M
    rng = np.random.default_rng(7)
    A = rng.standard_normal((rows, K), dtype=np.float32)
    W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    if pyoracle.Ref.available():
        ref = pyoracle.Ref()
        q, s = pyoracle.quant_rows(W)
        fn, kind, cores = (lambda: ref.qgemm(A, q, s)), "reference", ref.nthreads
    else:
        q, s = pyoracle.quant_rows(W)
        cores = pyoracle.nthreads_default()
        fn, kind = (lambda: pyoracle.qgemm(A, q, s, cores)), "port"
    def best_of_3():
        fn()
        best = 1e30
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - t0)
        return best

    best = best_of_3()
    tops = 2.0 * rows * K * N / best / 1e12
    # the same at 8 threads, the thread count of the reference's own figures
    tops8 = None
    if kind == "reference" and int(cores) != 8:
        ref.set_nthreads(8)
        tops8 = round(2.0 * rows * K * N / best_of_3() / 1e12, 5)
        ref.set_nthreads(int(cores))
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(tops, 5), "unit": "TOPS", "cores": int(cores), "kind": kind,
            "value_8_threads": tops8,
            "sample": (f"the full {args.M}x{K}x{N} qgemm" if rows == args.M else
                       f"M={rows} rows of the {args.M}x{K}x{N} qgemm (same K,N; M>=2048 keeps "
                       f"the reference's widened-s16 path)") +
                      f", best of 3 after 1 warmup, {best * 1e3:.1f} ms/call, host CPU: {cpu}"}


def main():
    args = parse()
    if args.kernel_counters:
        kernel_counters(args)
        return
    if args.summarize_counters:
        summarize_counters(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (every GPU box here has one); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import sdq

    if args.profile_pass:
        profile_pass(torch, sdq, args)
        return
    if args.config != "ns":
        sdq.init(0)
        fn = {"block": bench_block, "blockfull": bench_block_full, "ffn": bench_ffn, "cross": bench_cross,
              "twin": bench_twin, "load": bench_load}[args.config]
        line = fn(torch, sdq, args)
        line.update({"n_gpus": 1, "data": "synthetic, host memory" if args.config == "load"
                     else "synthetic, resident in HBM"})
        print(json.dumps(line), flush=True)
        return
    M, K, N = args.M, args.K, args.N
    dev = torch.device("cuda:0")
    sdq.init(0)
    info = sdq.device_info()
    A, q, s, bias = make_inputs(torch, dev, M, K, N)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    w = sdq.Weight.from_device(q, s)
    torch.cuda.synchronize()
    repack_ms = (time.perf_counter() - t0) * 1e3
    del q
    Y = torch.empty((M, N), device=dev, dtype=torch.float32)

    def step():
        sdq.qlinear(w, A, Y, kind="none", bias=bias)

    t_warm = time.perf_counter()
    for _ in range(args.warmup):
        step()
    settle = _settle(torch, step, args.settle_ms, t_warm)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12

    # per-kernel device time with HIP events on the launch stream, for the
    # kernels the library's plan names (the 256x256 launch and, when the
    # last round of tiles is split off, the 128x128 tail launch)
    plan = sdq.qlinear_plan(w, M)
    sdq.profile_begin()
    for _ in range(args.steps):
        step()
    prof = sdq.profile_end()
    kern = {}
    for name, r0, rows in plan:
        n_launch, tot = prof[name]
        kms = tot / n_launch
        kops = 2.0 * rows * N * K
        kern[name] = {"rows": rows, "ms": round(kms, 5), "tops": round(kops / kms / 1e9, 2),
                      "ops": kops}
    main_name = plan[0][0]
    main = kern[main_name]
    gemm_ms = sum(k["ms"] for k in kern.values())
    q_launch, q_ms = prof.get("act_quant", (1, 0.0))

    counters, stamp = _load_counters(args.counters_json, sdq.version(), f"{M}x{K}x{N}")
    traffic = None
    if counters:
        kc = counters["kernels"].get(main_name, {})
        traffic = kc.get("hbm_bytes_per_launch")
    line = {
        "metric": "int8 qGEMM TOPS + % of MI355X MFMA peak at M=27280,K=3072,N=14336",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (A~N(0,1), W~N(0,0.02) packer-quantized, bias~N(0,0.01)), "
                "resident in HBM",
        "config": {"workload": f"qgemm+bias M={M} K={K} N={N} (DiT FFN up, 720p/121f)",
                   "M": M, "K": K, "N": N, "output": "fp32", "epilogue": "bias",
                   "pct_of_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
                   "settle": {"extra_untimed_steps": settle,
                              "why": f"untimed steps after the {args.warmup} warmup steps until "
                                     f"{args.settle_ms:.0f} ms had passed: the shader clock "
                                     "overshoots and settles under the power limit over the "
                                     "first ~25 calls"},
                   "act_quant_ms": round(q_ms / max(q_launch, 1), 5),
                   "gemm_kernels": kern, "gemm_ms": round(gemm_ms, 5),
                   "weight_repack_ms": round(repack_ms, 3),
                   "library": sdq.version(), "counters": stamp, "device": info},
        "roofline": {"bound": "mfma", "kernel": main_name, "achieved": main["tops"],
                     "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(main["tops"] / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "algorithmic_ops": main["ops"],
                     "algorithmic_bytes": _gemm_bytes(main["rows"], K, N)},
    }
    if counters:
        kc = counters["kernels"].get(main_name, {})
        if "mfma_busy_frac" in kc:
            line["config"]["mfma_busy_frac_pmc"] = kc["mfma_busy_frac"]
        if "l2_hit_frac" in kc:
            line["config"]["l2_hit_frac_pmc"] = kc["l2_hit_frac"]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args, K, N)
    print(json.dumps(line), flush=True)


def _settle(torch, step, settle_ms, t_start):
    """Untimed steps until settle_ms of wall time have passed since t_start,
    synchronizing every few steps so the host does not run ahead of the GPU;
    returns the number of extra steps."""
    n = 0
    torch.cuda.synchronize()
    while (time.perf_counter() - t_start) * 1e3 < settle_ms:
        for _ in range(4):
            step()
        n += 4
        torch.cuda.synchronize()
    return n


def _gemm_bytes(rows, K, N):
    """Algorithmic HBM bytes of one GEMM launch over `rows` activation rows:
    int8 activations (rows*K), int8 weights (N*K), weight scales + bias
    (8N), fp32 output (4*rows*N)."""
    return rows * K + N * K + 8 * N + 4 * rows * N


def _load_counters(path, library, key):
    """The counter summary for workload `key`, if it was recorded on this
    library build (same source fingerprint); else (None, reason)."""
    try:
        with open(path) as f:
            cj = json.load(f)
    except (OSError, ValueError):
        return None, "no counter summary"
    if cj.get("workload") != key:
        return None, f"counter summary is for {cj.get('workload')}, not {key}"
    if cj.get("library") != library:
        return None, (f"counter summary recorded on '{cj.get('library')}', this run loads "
                      f"'{library}': not reported")
    return cj, f"recorded on this build ({cj.get('commit', '?')}, {cj.get('source', '')})"


def _short_kernel(name):
    """rocprofv3 kernel name -> the library's record name (north-star pass)."""
    if "qgemm_persist<256, 256" in name:
        return "qgemm_tile256x256"
    if "qgemm_persist<128, 128" in name:
        return "qgemm_tail128"
    if "act_quant_units_kernel" in name:
        return "act_quant"
    if "copyBuffer" in name:  # the runtime's device-to-device copy (the 1 GiB calibration)
        return "copy"
    return None


def _counter_rows(dirs):
    """(kernel name without arguments, counter) -> per-dispatch values, and
    kernel name -> per-dispatch durations in us, from rocprofv3 --pmc CSVs."""
    import csv
    import glob

    vals, dur = {}, {}
    for d in dirs:
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(fn, newline="") as f:
                for row in csv.DictReader(f):
                    name = row["Kernel_Name"].replace("(anonymous namespace)::", "")
                    name = name.replace("void ", "").split("(")[0]
                    vals.setdefault((name, row["Counter_Name"]), []).append(
                        float(row["Counter_Value"]))
                    if row.get("Start_Timestamp") and row.get("End_Timestamp"):
                        key = (name, row["Dispatch_Id"])
                        dur[key] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
    per = {}
    for (name, _), us in dur.items():
        per.setdefault(name, []).append(us)
    return vals, per


def kernel_counters(args):
    """Per-kernel means of rocprofv3 --pmc runs of any bench.py config:
    FETCH_SIZE and WRITE_SIZE scaled to bytes by the --profile-pass copy
    (see summarize_counters), the MFMA busy fraction over the kernel's active
    cycles, and the mean duration under the profiler (kernels serialized)."""
    vals, dur = _counter_rows(args.kernel_counters)
    scale = {}
    if args.calibrate:
        for d, c in zip(args.calibrate, ("FETCH_SIZE", "WRITE_SIZE")):
            cv, _ = _counter_rows([d])
            copy = [v for (k, cc), v in cv.items() if "copyBuffer" in k and cc == c]
            if copy:
                scale[c] = (1 << 30) / (max(copy[0]) * 1024)
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    names = sorted({k for k, _ in vals})
    out = {"calibration": scale, "kernels": {}}
    for k in names:
        kc = {"dispatches": max(len(v) for (kk, _), v in vals.items() if kk == k)}
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            if (k, c) in vals and c in scale:
                kc[c.lower().replace("_size", "_bytes")] = round(mean(vals[(k, c)]) * 1024 * scale[c])
        busy, act = vals.get((k, "SQ_VALU_MFMA_BUSY_CYCLES")), vals.get((k, "GRBM_GUI_ACTIVE"))
        if busy and act:
            # GRBM_GUI_ACTIVE is summed over the 8 XCDs; 256 CUs x 4 SIMDs
            kc["mfma_busy_frac"] = round(mean(busy) / ((mean(act) / 8) * 256 * 4), 4)
        # where the waves' time goes: the share of wave cycles spent waiting on
        # an instruction dependency (s_waitcnt, barrier), the mean L2 read
        # latency seen by the L1, LDS bank-conflict cycles per LDS instruction
        for key, num, den in (("wait_frac", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES"),
                              ("l2_read_latency_cycles", "TCP_TCC_READ_REQ_LATENCY_sum",
                               "TCP_TCC_READ_REQ_sum"),
                              ("lds_conflict_cycles_per_inst", "SQ_LDS_BANK_CONFLICT",
                               "SQ_INSTS_LDS")):
            a, b = vals.get((k, num)), vals.get((k, den))
            if a and b and mean(b) > 0:
                kc[key] = round(mean(a) / mean(b), 4)
        if k in dur:
            kc["us_mean"] = round(mean(dur[k]), 2)
        out["kernels"][k] = kc
    print(json.dumps(out, indent=1))


def summarize_counters(args):
    """Reads the counter_collection.csv files of rocprofv3 --pmc runs of
    `bench.py --profile-pass` and writes the per-kernel summary bench.py
    reports: HBM bytes per launch (FETCH_SIZE and WRITE_SIZE, each scaled by
    what the counter reads for the pass's plain copy of known size), MFMA busy
    fraction (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs) and L2
    hit fraction (TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum))."""
    import csv
    import glob
    import subprocess

    vals = {}  # (kernel, counter) -> [per-dispatch values]
    meta = None
    for d in args.summarize_counters:
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(fn, newline="") as f:
                for row in csv.DictReader(f):
                    k = _short_kernel(row["Kernel_Name"])
                    if k:
                        vals.setdefault((k, row["Counter_Name"]), []).append(
                            float(row["Counter_Value"]))
        for fn in glob.glob(os.path.join(d, "**", "*.log"), recursive=True) + \
                glob.glob(os.path.join(d + ".log")):
            with open(fn) as f:
                for ln in f:
                    if ln.startswith("{") and "profile_pass" in ln:
                        meta = json.loads(ln)
    if meta is None:
        sys.exit("summarize: no --profile-pass output line found (pass the .log beside each dir)")
    mean = lambda k, c: (sum(vals[(k, c)]) / len(vals[(k, c)])) if (k, c) in vals else None  # noqa
    copy_bytes = meta["copy_bytes"]
    cf, cw = mean("copy", "FETCH_SIZE"), mean("copy", "WRITE_SIZE")
    fscale = copy_bytes / (cf * 1024) if cf else None
    wscale = copy_bytes / (cw * 1024) if cw else None
    info_cus = int(meta.get("cu_count", 256))
    out = {"workload": f"{meta['M']}x{meta['K']}x{meta['N']}", "library": meta["library"],
           "plan": meta["plan"], "calibration": {"copy_bytes": copy_bytes,
                                                  "fetch_scale": fscale, "write_scale": wscale},
           "kernels": {}}
    try:
        out["commit"] = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"],
                                       capture_output=True, text=True).stdout.strip()
    except OSError:
        out["commit"] = "?"
    for k in ("qgemm_tile256x256", "qgemm_tail128", "act_quant"):
        kc = {}
        f, wr = mean(k, "FETCH_SIZE"), mean(k, "WRITE_SIZE")
        if f is not None and fscale:
            kc["fetch_bytes"] = round(f * 1024 * fscale)
        if wr is not None and wscale:
            kc["write_bytes"] = round(wr * 1024 * wscale)
        if "fetch_bytes" in kc and "write_bytes" in kc:
            kc["hbm_bytes_per_launch"] = kc["fetch_bytes"] + kc["write_bytes"]
        busy, act = mean(k, "SQ_VALU_MFMA_BUSY_CYCLES"), mean(k, "GRBM_GUI_ACTIVE")
        if busy is not None and act:
            # GRBM_GUI_ACTIVE is summed over the 8 XCDs; 4 SIMDs per CU
            kc["mfma_busy_frac"] = round(busy / ((act / 8) * info_cus * 4), 4)
            kc["active_cycles_per_xcd"] = round(act / 8)
        hit, miss = mean(k, "TCC_HIT_sum"), mean(k, "TCC_MISS_sum")
        if hit is not None and miss is not None and hit + miss > 0:
            kc["l2_hit_frac"] = round(hit / (hit + miss), 4)
            kc["l2_requests"] = round(hit + miss)
        if kc:
            kc["dispatches"] = max(len(v) for (kk, c), v in vals.items() if kk == k)
            out["kernels"][k] = kc
    out["source"] = os.path.relpath(args.counters_json, ROOT).replace(".json", ".md")
    with open(args.counters_json, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
