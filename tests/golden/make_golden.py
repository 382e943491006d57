#!/usr/bin/env python3
"""Write the committed golden fixtures under tests/golden/.

basic_golden.npz
    The reference's own golden vectors for the qgemm path: the draw order and
    closed forms of tools/golden/gen_basic.py (numpy default_rng(5)), restated
    here (not imported): quantize_rowwise inputs + exact int8/scale replica
    (gen_basic.py:44-50) and the qgemm inputs + fp32 dequant product that the
    reference checks with cosine > 0.999 (gen_basic.py:52-58,
    tests/test_golden.cpp:64-81).

ref_qgemm.npz
    Outputs of the REFERENCE's own sd::qgemm / quantize_rowwise / randu,
    compiled from its sources into oracle/_ref (oracle/Makefile), on
    - the test_core.cpp shapes {17,31,13}, {64,1024,512} with randu seeds
      7+M / 13+N and quantize_rowwise weights (tests/test_core.cpp:93-118);
      {3072,5120,5120} is stored as a SHA-256 of the output bytes;
    - the BASELINE cfg1 shape 256x3072x3072 with N(0,1) activations and
      packer-quantized N(0,0.02) weights (SHA-256 of the output bytes);
    - a small matrix of special activation rows (zeros, NaN, +-Inf,
      denormals, huge values, ties) that pins the quantizer's edge cases.
Run from the repo root after __graft_entry__.build():  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def lround(v):
    v = v.astype(np.float64)
    return np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5))


def basic_golden():
    rng = np.random.default_rng(5)
    # draws in gen_basic.py's order (only the qgemm-path arrays are kept)
    rng.uniform(-1, 1, (64, 128))
    rng.uniform(0.5, 1.5, 128)
    rng.uniform(-3, 3, 256)
    rng.uniform(-1, 1, (17, 31))
    rng.uniform(-1, 1, (31, 13))
    rng.uniform(-1, 1, 1000)
    W = rng.uniform(-1, 1, (64, 256)).astype(np.float32)
    sc = np.abs(W).max(axis=1) / np.float32(127.0)
    sc = np.where(sc == np.float32(0), np.float32(1), sc).astype(np.float32)
    qa = rng.standard_normal((64, 256)).astype(np.float32)
    qb = rng.integers(-127, 128, (128, 256)).astype(np.int8)
    qs = rng.uniform(0.001, 0.01, 128).astype(np.float32)
    out = dict(
        q_w=W,
        q_wq=lround(W / sc[:, None]).astype(np.int8),
        q_scale=sc,
        qg_a=qa,
        qg_bq=qb,
        qg_bs=qs,
        qg_out=(qa @ (qb.T.astype(np.float32) * qs[None, :])).astype(np.float32),
    )
    np.savez(os.path.join(OUT, "basic_golden.npz"), **out)


def special_rows(K=96):
    """Activation rows exercising every branch of the reference quantizer."""
    f32 = np.float32
    rows = []
    rng = np.random.default_rng(123)
    base = rng.standard_normal(K).astype(f32)
    rows.append(np.zeros(K, f32))                              # sc == 0 -> 1
    r = base.copy(); r[3] = np.nan; rows.append(r)              # NaN ignored by max, -> -127
    r = base.copy(); r[5] = np.inf; rows.append(r)              # mx = inf, inv = 0
    r = base.copy(); r[7] = -np.inf; rows.append(r)
    rows.append((base * f32(1e-39)).astype(f32))                # denormal amax -> inv overflow
    rows.append((base * f32(1e-41)).astype(f32))                # deeper denormals
    rows.append((base * f32(3e38)).astype(f32))                 # near FLT_MAX
    r = np.zeros(K, f32); r[0] = f32(127.0); r[1:64] = np.arange(-63, 0, dtype=f32) + f32(0.5)
    rows.append(r)                                              # exact .5 ties (RNE)
    r = np.full(K, f32(-2.5)); r[0] = f32(127.0); rows.append(r)
    rows.append(-np.abs(base))                                  # all negative
    r = np.zeros(K, f32); r[10] = f32(1e-45); rows.append(r)    # single smallest denormal
    r = base.copy(); r[::2] = np.nan; rows.append(r)
    return np.stack(rows).astype(f32)


def ref_golden():
    ref = pyoracle.Ref()
    out = {}
    for (M, K, N) in [(17, 31, 13), (64, 1024, 512), (3072, 5120, 5120)]:
        A = ref.randu(M * K, 7 + M).reshape(M, K)
        W = ref.randu(N * K, 13 + N).reshape(N, K)
        q, s = ref.quantize_rowwise(W)
        o = ref.qgemm(A, q, s)
        tag = f"core_{M}x{K}x{N}"
        if M * N <= 64 * 512:
            out[tag + "_out"] = o
        out[tag + "_sha256"] = np.frombuffer(hashlib.sha256(o.tobytes()).digest(), np.uint8)
    # cfg1: N(0,1) activations, packer-quantized N(0,0.02) weights
    M, K, N = 256, 3072, 3072
    A = pyoracle.randn(M * K, 1001).reshape(M, K)
    W = pyoracle.randn(N * K, 1002).reshape(N, K) * np.float32(0.02)
    q, s = pyoracle.quant_rows(W)
    o = ref.qgemm(A, q, s)
    out["cfg1_sha256"] = np.frombuffer(hashlib.sha256(o.tobytes()).digest(), np.uint8)
    # special rows
    A = special_rows()
    Wf = pyoracle.randn(40 * A.shape[1], 77).reshape(40, A.shape[1]) * np.float32(0.02)
    q, s = pyoracle.quant_rows(Wf)
    out["special_a"] = A
    out["special_bq"] = q
    out["special_bs"] = s
    out["special_out"] = ref.qgemm(A, q, s)
    np.savez(os.path.join(OUT, "ref_qgemm.npz"), **out)


if __name__ == "__main__":
    basic_golden()
    ref_golden()
    print("wrote", os.listdir(OUT))
