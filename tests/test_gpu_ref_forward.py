"""The reference's own DiT forward with sd::qgemm on the GPU.

oracle/Makefile builds tests/cpp/ref_forward.cpp (OviDit::forward from the
reference's model/ovi_dit.cpp, blocks.cpp, gemm.cpp, tensor.cpp and
sdcpp.cpp, compiled where they lie) twice: with the reference's qgemm.cpp
(ref_forward_cpu) and with libsd_qgemm.so in its place (ref_forward_gpu: the
reference's own link line with -lsd_qgemm -lsdq for qgemm.cpp). Every int8
Linear of the forward (ovi_dit.cpp:66-84, mlin: text embedding te0/te2
662-673, the M=1 time MLP tm2 and AdaLN projection tp1 678-700, every block
Linear, the video head 298-314) then goes through the GPU. Both builds run OviDitCfg::test()
(ovi_dit.cpp:336-342) on one int8 pack and the same inputs; their outputs
must be bit-identical. As in tests/test_ovit8.cpp:83-125, the int8 forward
is also gated against the fp32 forward of the same weights (the pack written
with every tensor raw f32): cosine > 0.99."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact

pytestmark = pytest.mark.gpu

REF_DIR = os.path.join(ROOT, "oracle", "_ref")
DIM, FFN, HEADS, LAYERS, FREQ, TEXT_DIM = 384, 1792, 3, 2, 32, 512  # OviDitCfg::test()
FUSION = {1}
HIDDEN = 1024  # audio ConvMLP hidden: round256(int(2 * 4 * dim / 3)) (model.py:144-145)


def _tensors(oracle):
    """Every tensor OviDit::load_impl reads at OviDitCfg::test()
    (ovi_dit.cpp:466-537), seeded."""
    t, seed = {}, [10]

    def put(name, shape, std, mean=0.0):
        seed[0] += 1
        n = int(np.prod(shape))
        t[name] = (oracle.randn(n, seed[0]) * np.float32(std) + np.float32(mean)).reshape(shape)

    def lin(base, i, o):
        put(base + ".weight", (o, i), 1.0 / np.sqrt(i))
        put(base + ".bias", (o,), 0.02)

    for pfx, in_dim, out_dim in (("video_model.", 48, 48), ("audio_model.", 20, 20)):
        if pfx[0] == "a":
            put(pfx + "patch_embedding.0.weight", (DIM, in_dim, 7), 1.0 / np.sqrt(in_dim * 7))
            put(pfx + "patch_embedding.0.bias", (DIM,), 0.02)
            put(pfx + "patch_embedding.2.w1.weight", (HIDDEN, DIM, 7), 1.0 / np.sqrt(DIM * 7))
            put(pfx + "patch_embedding.2.w2.weight", (DIM, HIDDEN, 7), 1.0 / np.sqrt(HIDDEN * 7))
            put(pfx + "patch_embedding.2.w3.weight", (HIDDEN, DIM, 7), 1.0 / np.sqrt(DIM * 7))
            pout = out_dim
        else:
            put(pfx + "patch_embedding.weight", (DIM, in_dim, 1, 2, 2), 1.0 / np.sqrt(in_dim * 4))
            put(pfx + "patch_embedding.bias", (DIM,), 0.02)
            pout = 4 * out_dim
        lin(pfx + "text_embedding.0", TEXT_DIM, DIM)
        lin(pfx + "text_embedding.2", DIM, DIM)
        lin(pfx + "time_embedding.0", FREQ, DIM)
        lin(pfx + "time_embedding.2", DIM, DIM)
        lin(pfx + "time_projection.1", DIM, 6 * DIM)
        lin(pfx + "head.head", DIM, pout)
        put(pfx + "head.modulation", (1, 2, DIM), 0.1)
        for i in range(LAYERS):
            B = f"{pfx}blocks.{i}."
            for w in ("q", "k", "v", "o"):
                lin(B + "self_attn." + w, DIM, DIM)
            put(B + "self_attn.norm_q.weight", (DIM,), 0.1, 1.0)
            put(B + "self_attn.norm_k.weight", (DIM,), 0.1, 1.0)
            for w in ("q", "k", "v", "o"):
                lin(B + "cross_attn." + w, DIM, DIM)
            put(B + "cross_attn.norm_q.weight", (DIM,), 0.1, 1.0)
            put(B + "cross_attn.norm_k.weight", (DIM,), 0.1, 1.0)
            put(B + "norm3.weight", (DIM,), 0.1, 1.0)
            put(B + "norm3.bias", (DIM,), 0.02)
            lin(B + "ffn.0", DIM, FFN)
            lin(B + "ffn.2", FFN, DIM)
            put(B + "modulation.modulation", (1, 6, DIM), 0.1)
            if i in FUSION:
                lin(B + "cross_attn.k_fusion", DIM, DIM)
                lin(B + "cross_attn.v_fusion", DIM, DIM)
                put(B + "cross_attn.norm_k_fusion.weight", (DIM,), 0.1, 1.0)
                put(B + "cross_attn.pre_attn_norm_fusion.weight", (DIM,), 0.1, 1.0)
                put(B + "cross_attn.pre_attn_norm_fusion.bias", (DIM,), 0.02)
    return t


def _run(exe, pack, ind, outd, iters):
    os.makedirs(outd, exist_ok=True)
    print(f"[ref-forward] {os.path.basename(exe)} {os.path.basename(pack)}", flush=True)
    r = subprocess.run([exe, pack, ind, outd, str(iters)], capture_output=True, text=True,
                       timeout=600)
    if r.returncode != 0:
        raise AssertionError(f"{exe} rc={r.returncode}\n{r.stdout}\n{r.stderr}")
    ms = [float(line.split()[2]) for line in r.stdout.splitlines() if line.startswith("forward_ms")]
    int8 = [line for line in r.stdout.splitlines() if line.startswith("use_int8")]
    ov = np.fromfile(os.path.join(outd, "out_video.bin"), np.float32)
    oa = np.fromfile(os.path.join(outd, "out_audio.bin"), np.float32)
    return ov, oa, ms, int8[0].split()[1] == "1"


def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def test_reference_forward_through_drop_in(tmp_path, sdq_dev, oracle):
    cpu = os.path.join(REF_DIR, "ref_forward_cpu")
    gpu = os.path.join(REF_DIR, "ref_forward_gpu")
    if not (os.path.exists(cpu) and os.path.exists(gpu)):
        pytest.fail("oracle/_ref/ref_forward_{cpu,gpu} not built (make -f oracle/Makefile ref)")
    tensors = _tensors(oracle)
    p8, p32 = str(tmp_path / "int8.sdcpp"), str(tmp_path / "f32.sdcpp")
    written = oracle.write_sdcpp(p8, tensors)
    assert sum(code == 0 for code, _, _ in written.values()) > 40  # the Linears went int8
    oracle.write_sdcpp(p32, tensors, min_quant_numel=1 << 62)
    # inputs: video latents [48, F=2, H=8, W=8] (32 tokens), audio [24, 20],
    # text contexts of 20 rows (zero-padded to text_len 64 by embed_ctx)
    F, H, W, La, Lc, t = 2, 8, 8, 24, 20, 500.0
    ind = str(tmp_path / "in")
    os.makedirs(ind)
    with open(os.path.join(ind, "dims.txt"), "w") as f:
        f.write(f"{F} {H} {W} {La} {Lc} {t}\n")
    for name, n, seed in (("video", 48 * F * H * W, 1), ("audio", La * 20, 2),
                          ("vctx", Lc * TEXT_DIM, 3), ("actx", Lc * TEXT_DIM, 4)):
        oracle.randn(n, seed).tofile(os.path.join(ind, name + ".bin"))
    ov_c, oa_c, ms_c, q_c = _run(cpu, p8, ind, str(tmp_path / "cpu"), 2)
    ov_g, oa_g, ms_g, q_g = _run(gpu, p8, ind, str(tmp_path / "gpu"), 4)
    ov_f, oa_f, _, q_f = _run(cpu, p32, ind, str(tmp_path / "f32"), 1)
    assert q_c and q_g and not q_f
    print(f"  forward wall ms: reference qgemm {ms_c}, GPU sd::qgemm {ms_g} "
          f"(the first GPU call uploads every weight)", flush=True)
    assert ov_g.size == 48 * F * H * W and oa_g.size == La * 20
    assert_bitexact(ov_g, ov_c, "out_video: GPU sd::qgemm vs the reference's qgemm")
    assert_bitexact(oa_g, oa_c, "out_audio: GPU sd::qgemm vs the reference's qgemm")
    cv, ca = _cos(ov_g, ov_f), _cos(oa_g, oa_f)
    print(f"  int8 vs fp32 forward cosine: video {cv:.6f}, audio {ca:.6f}", flush=True)
    assert cv > 0.99 and ca > 0.99  # tests/test_ovit8.cpp:113-122
