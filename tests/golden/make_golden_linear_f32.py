#!/usr/bin/env python3
"""Write tests/golden/ref_linear_f32.npz: outputs of the REFERENCE's own fp32
matmul (src/core/gemm.cpp:115-160, the F32 branch of mlin through
blk::linear, src/model/blocks.cpp:14-16), compiled from its sources into
oracle/_ref (oracle/Makefile), on small seeded inputs:
  - an audio-head-shaped product (N = 20 < the 16-column panels' multiple,
    M not a multiple of the 6-row groups) with and without bias,
  - a product whose weights hold zeros, -0 and denormals, and a bias with -0,
  - K = 0 (zero output plus bias).
The oracle's C restatement is pinned to these bit for bit without needing the
reference sources (tests/test_oracle_linear_f32.py).
Run from the repo root after __graft_entry__.build():
    python tests/golden/make_golden_linear_f32.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def main():
    if not pyoracle.Ref.available():
        sys.exit("oracle/_ref is not built (needs the reference sources)")
    ref = pyoracle.Ref()
    rng = np.random.default_rng(77)
    f = {}
    x = rng.standard_normal((23, 384)).astype(np.float32)
    w = (rng.standard_normal((384, 20)) * 0.05).astype(np.float32)
    b = rng.standard_normal(20).astype(np.float32)
    f.update(head_x=x, head_w=w, head_b=b)
    f["head_y"] = ref.matmul(x, w, b)
    f["head_y_nobias"] = ref.matmul(x, w)
    x2 = (rng.standard_normal((9, 40)) * np.float32(3.0)).astype(np.float32)
    w2 = rng.standard_normal((40, 35)).astype(np.float32)
    w2[::3, ::2] = 0.0
    w2[1::5, 1::3] = -0.0
    w2[2::7, :] *= np.float32(1e-39)  # denormal weights, products underflow
    b2 = rng.standard_normal(35).astype(np.float32)
    b2[::4] = -0.0
    f.update(sp_x=x2, sp_w=w2, sp_b=b2)
    f["sp_y"] = ref.matmul(x2, w2, b2)
    x3 = np.zeros((4, 0), np.float32)
    w3 = np.zeros((0, 6), np.float32)
    b3 = np.array([1.5, -0.0, 0.0, -2.0, 3.25, 1e-40], np.float32)
    f.update(k0_b=b3)
    f["k0_y"] = ref.matmul(x3, w3, b3)
    np.savez_compressed(os.path.join(OUT, "ref_linear_f32.npz"), **f)
    print("wrote ref_linear_f32.npz:", {n: a.shape for n, a in f.items()})


if __name__ == "__main__":
    main()
