"""Block loading from a .sdcpp pack: the checks and messages of
OviDit::load_impl (ovi_dit.cpp:383-415, 505-537) on both loading paths (the
pack index with sequential file reads, and load_sdcpp's mapping). Every
check runs before anything is uploaded, so these run on the CPU."""
import numpy as np
import pytest

from test_gpu_pack_blocks import _write_pack


def test_pack_blocks_errors(oracle, tmp_path):
    """load_impl's checks and messages on the pack (ovi_dit.cpp:383-415, 505-537)."""
    import sdq

    dim, ffn = 256, 512
    path = str(tmp_path / "b.sdcpp")
    written = _write_pack(oracle, path, "video_model.", 1, dim, ffn, False, 40)
    for file_reads in (True, False):
        with pytest.raises(sdq.SdqError, match="missing tensor video_model.blocks.1.self_attn.q"):
            sdq.DitBlock.from_pack(path, "video_model.", [1], dim, ffn, False, file_reads)
        with pytest.raises(sdq.SdqError, match="bad shape for video_model.blocks.0.self_attn.q"):
            sdq.DitBlock.from_pack(path, "video_model.", [0], 128, ffn, False, file_reads)
        with pytest.raises(sdq.SdqError, match="missing tensor video_model.blocks.0.cross_attn"):
            sdq.DitBlock.from_pack(path, "video_model.", [0], dim, ffn, True, file_reads)
        with pytest.raises(sdq.SdqError, match="cannot open"):
            sdq.DitBlock.from_pack(path + ".none", "video_model.", [0], dim, ffn, False,
                                   file_reads)
    # a modulation bias of the wrong shape
    bad = {}
    for k, (code, a, s) in written.items():
        bad[k] = (a.astype(np.float32) * s[:, None]) if code == 0 else a
    bad["video_model.blocks.0.modulation.modulation"] = np.zeros((1, 5, dim), np.float32)
    p2 = str(tmp_path / "bad.sdcpp")
    oracle.write_sdcpp(p2, bad)
    for file_reads in (True, False):
        with pytest.raises(sdq.SdqError, match="bad modulation video_model.blocks.0."):
            sdq.DitBlock.from_pack(p2, "video_model.", [0], dim, ffn, False, file_reads)
