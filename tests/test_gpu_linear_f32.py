"""The F32 branch of mlin on the GPU (sdq_linear_f32): blk::linear ->
sd::matmul (src/core/gemm.cpp:115-160), bit-exact against the oracle's
restatement (itself pinned to the reference build) and against the committed
outputs of the reference build, at the audio head's shape ([20, 3072] on the
157 audio tokens, ovi_dit.cpp:313), ragged shapes, K = 0 and the many-rows
launch form (four rows per lane)."""
import os

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _run(sdq, torch, dev, x, w, b):
    M, N = x.shape[0], w.shape[1]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa: E731
    out = torch.full((M, N), float("nan"), device=dev)
    sdq.linear_f32(t(x), t(w), out, bias=None if b is None else t(b))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("M,K,N", [(157, 3072, 20), (768, 3072, 20), (1, 256, 3072),
                                   (77, 1000, 130), (1, 1, 1), (3000, 96, 130),
                                   (5000, 64, 16)])
def test_linear_f32_matches_oracle(sdq_dev, oracle, M, K, N):
    import torch

    import sdq

    print(f"[linear_f32] {M}x{K}x{N}", flush=True)
    x = oracle.randn(M * K, M + 1).reshape(M, K)
    w = (oracle.randn(K * N, N + 2) * np.float32(0.05)).reshape(K, N)
    b = oracle.randn(N, 3)
    assert_bitexact(_run(sdq, torch, sdq_dev, x, w, b), oracle.linear_f32(x, w, b),
                    f"{M}x{K}x{N}")
    assert_bitexact(_run(sdq, torch, sdq_dev, x, w, None), oracle.linear_f32(x, w),
                    f"{M}x{K}x{N} no bias")


def test_linear_f32_reference_outputs(sdq_dev):
    """Committed outputs of the reference build's matmul
    (tests/golden/make_golden_linear_f32.py): audio-head shape, zeros / -0 /
    denormal weights with a -0 bias, K = 0."""
    import torch

    import sdq

    g = np.load(os.path.join(GOLDEN, "ref_linear_f32.npz"))
    assert_bitexact(_run(sdq, torch, sdq_dev, g["head_x"], g["head_w"], g["head_b"]),
                    g["head_y"], "audio-head shape")
    assert_bitexact(_run(sdq, torch, sdq_dev, g["head_x"], g["head_w"], None),
                    g["head_y_nobias"], "audio-head shape, no bias")
    assert_bitexact(_run(sdq, torch, sdq_dev, g["sp_x"], g["sp_w"], g["sp_b"]), g["sp_y"],
                    "zeros, -0, denormals")
    assert_bitexact(_run(sdq, torch, sdq_dev, np.zeros((4, 0), np.float32),
                         np.zeros((0, 6), np.float32), g["k0_b"]), g["k0_y"], "K = 0")


def test_linear_f32_raw_abi_errors(sdq_dev):
    import sdq

    lib = sdq.load_library()
    assert lib.sdq_linear_f32(None, -1, 4, None, 4, None, None, None) == sdq.ERR_INVALID
    assert lib.sdq_linear_f32(None, 2, 4, None, 4, None, None, None) == sdq.ERR_INVALID
    # M == 0 / N == 0: nothing to do
    assert lib.sdq_linear_f32(None, 0, 4, None, 4, None, None, None) == 0
    assert lib.sdq_linear_f32(None, 3, 4, None, 0, None, None, None) == 0
