#!/usr/bin/env python3
"""Benchmark of the int8 qGEMM hot path on one MI355X.

Workload (BASELINE.json metric, north star): one int8 Linear of the Ovi DiT
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
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--M", type=int, default=M_NS)
    ap.add_argument("--K", type=int, default=K_NS)
    ap.add_argument("--N", type=int, default=N_NS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-rows", type=int, default=4096)
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="rocprofv3 FETCH/WRITE_SIZE summary used for roofline.traffic")
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
                      "K": args.K, "N": args.N}), flush=True)


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


def cpu_baseline(args, K, N):
    """The reference's sd::qgemm (oracle/_ref) on a row sample of the same
    workload; best of 3 after one warmup (tests/test_core.cpp:40-49)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import pyoracle

    rows = args.cpu_sample_rows
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
    fn()
    best = 1e30
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    tops = 2.0 * rows * K * N / best / 1e12
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
            "sample": f"M={rows} rows of the {args.M}x{K}x{N} qgemm (same K,N; M>=2048 keeps "
                      f"the reference's widened-s16 path), best of 3 after 1 warmup, "
                      f"{best * 1e3:.1f} ms/call, host CPU: {cpu}"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (every GPU box here has one); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import sdq

    if args.profile_pass:
        profile_pass(torch, sdq, args)
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

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12

    # per-kernel device time with HIP events on the launch stream
    sdq.profile_begin()
    for _ in range(args.steps):
        step()
    prof = sdq.profile_end()
    gemm_name = next(k for k in prof if k.startswith("qgemm"))
    g_launch, g_ms = prof[gemm_name]
    gemm_ms = g_ms / g_launch
    q_launch, q_ms = prof.get("act_quant", (1, 0.0))
    achieved = ops / (gemm_ms * 1e-3) / 1e12
    traffic = None
    try:
        with open(args.traffic_json) as f:
            tj = json.load(f)
        key = f"{M}x{K}x{N}"
        if key in tj:
            traffic = tj[key]["qgemm_hbm_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        traffic = None

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
                   "gemm_kernel": gemm_name, "pct_of_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
                   "act_quant_ms": round(q_ms / max(q_launch, 1), 5),
                   "gemm_ms": round(gemm_ms, 5), "weight_repack_ms": round(repack_ms, 3),
                   "device": info},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8_TOPS, 4),
                     "traffic": traffic},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args, K, N)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
