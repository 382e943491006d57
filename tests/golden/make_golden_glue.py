#!/usr/bin/env python3
"""Write tests/golden/ref_glue.npz: outputs of the REFERENCE's own block glue,
compiled from its sources into oracle/_ref (oracle/Makefile, the shim over
src/model/ovi_dit.cpp and blocks.cpp), on small seeded inputs:
  - blk::layernorm without and with affine weights (blocks.cpp:18-43),
  - mod_rows (ovi_dit.cpp:161-172),
  - rmsnorm (src/core/tensor.cpp:112-123),
  - rope_freqs_3d / rope_freqs_1d angles (blocks.cpp:46-84) and apply_rope
    with them (blocks.cpp:86-100),
  - sdpa (blocks.cpp:112-199), two heads of 128, Lq != Lk.
The oracle's C restatement is pinned to these bit for bit without needing the
reference sources (tests/test_oracle.py::test_ref_glue_fixture_outputs).
Run from the repo root after __graft_entry__.build():
    python tests/golden/make_golden_glue.py
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
    rng = np.random.default_rng(2024)
    f = {}
    x = (rng.standard_normal((24, 256)) * rng.uniform(0.1, 20, (24, 1))
         + rng.uniform(-30, 30, (24, 1))).astype(np.float32)
    x[5] = np.float32(1.5)  # constant row: variance 0
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, 256).astype(np.float32)
    shift = rng.standard_normal(256).astype(np.float32) * np.float32(0.3)
    scale = rng.standard_normal(256).astype(np.float32) * np.float32(0.3)
    f.update(x=x, w=w, b=b, shift=shift, scale=scale)
    f["layernorm"] = ref.layernorm(x, 1e-6)
    f["layernorm_affine"] = ref.layernorm(x, 1e-6, w, b)
    f["mod_rows"] = ref.mod_rows(f["layernorm"], shift, scale)
    f["rmsnorm"] = ref.rmsnorm(x, w, 1e-6)
    ang3 = ref.rope_freqs_3d(2, 3, 4, 128, 10000.0)
    ang1 = ref.rope_freqs_1d(24, 128, 10000.0, 0.19676)
    f["ang3"], f["ang1"] = ang3, ang1
    f["rope3"] = ref.apply_rope(x, ang3, 2)
    f["rope1"] = ref.apply_rope(x, ang1, 2)
    q = (rng.standard_normal((20, 256)) * 0.7).astype(np.float32)
    k = (rng.standard_normal((37, 256)) * 0.7).astype(np.float32)
    v = rng.standard_normal((37, 256)).astype(np.float32)
    f.update(q=q, k=k, v=v)
    f["sdpa"] = ref.sdpa(q, k, v, 2)
    np.savez_compressed(os.path.join(OUT, "ref_glue.npz"), **f)
    print("wrote ref_glue.npz:", {n: a.shape for n, a in f.items()})


if __name__ == "__main__":
    main()
