"""Writes tests/golden/fullsize_sha256.json: SHA-256 of the WHOLE output of the
reference's own sd::qgemm (oracle/_ref, compiled from src/core/qgemm.cpp) at
the headline shapes, so the GPU can be checked on every one of their outputs
(391M at the north star) without the reference tree on the GPU box.

  north star   A [27280, 3072]  x W [14336, 3072]  (FFN up, 720p/121 frames)
  FFN down     A [27280, 14336] x W [3072, 14336]
  cross q      A [27280, 3072]  x W [3072, 3072]   (config 4's video-token q)

Inputs are the oracle's seeded generators (splitmix64 + Box-Muller, gen.cpp:
88-105; the packer's row-wise quantizer, pack_sdcpp.py:45-51): A ~ N(0,1),
W ~ N(0, 0.02). The hashes of A and of (Wq, scale) are recorded too, so the
GPU test can confirm it regenerated the same inputs. The oracle's own C
restatement is run as well and must give the same output hash.

Run in the build container (needs oracle/_ref):
    python tests/golden/make_fullsize_hashes.py [name ...]
A few minutes of CPU per shape.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle  # noqa: E402

SHAPES = {
    "ns_27280x3072x14336": dict(M=27280, K=3072, N=14336, seed_a=101, seed_w=202),
    "ffn_down_27280x14336x3072": dict(M=27280, K=14336, N=3072, seed_a=303, seed_w=404),
    # config 4's video-token cross-attention q projection
    "cross_q_27280x3072x3072": dict(M=27280, K=3072, N=3072, seed_a=505, seed_w=606),
}


def inputs(M, K, N, seed_a, seed_w):
    """The seeded inputs the GPU test regenerates (same calls, same order)."""
    A = pyoracle.randn(M * K, seed_a).reshape(M, K)
    W = pyoracle.randn(N * K, seed_w).reshape(N, K) * np.float32(0.02)
    q, s = pyoracle.quant_rows(W)
    return A, q, s


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).data)
    return h.hexdigest()


def main():
    """python make_fullsize_hashes.py [name ...]: (re)records the named shapes
    (default all), keeping the other entries of the JSON file."""
    ref = pyoracle.Ref()
    path = os.path.join(HERE, "fullsize_sha256.json")
    out = {}
    if os.path.exists(path):
        with open(path) as f:
            out = json.load(f)
    for name in sys.argv[1:] or list(SHAPES):
        c = SHAPES[name]
        t0 = time.time()
        A, q, s = inputs(**c)
        y = ref.qgemm(A, q, s)
        h_ref = sha(y)
        del y
        y = pyoracle.qgemm(A, q, s)
        h_orc = sha(y)
        del y
        if h_ref != h_orc:
            sys.exit(f"{name}: the oracle's restatement differs from the reference build")
        out[name] = dict(c, sha256_A=sha(A), sha256_W=sha(q, s), sha256_out=h_ref,
                         producer="oracle/_ref sd::qgemm (reference src/core/qgemm.cpp)")
        print(f"{name}: {h_ref} ({time.time() - t0:.1f} s)", flush=True)
    with open(path, "w") as f:
        json.dump({k: out[k] for k in SHAPES if k in out}, f, indent=1)


if __name__ == "__main__":
    main()
