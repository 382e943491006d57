"""Static checks of the gfx950 code for hazards that the compiler does not
always cover (inline asm operands, buffer stores with an SGPR soffset):

* a vector-memory store of more than 8 bytes reads its data VGPRs after
  issue, so a VALU write of any of them needs 2 wait states after it;
* a VALU write of an SGPR (v_readlane / v_readfirstlane, e.g. reloading a
  spilled SGPR) needs 5 wait states before a vector-memory instruction
  reads that SGPR (descriptor, soffset), and an M0 write needs 1 before an
  LDS-DMA load (buffer_load ... lds).

A missed case silently uses stale offsets or data (seen as misplaced or
nondeterministic outputs). The test compiles each HIP source to assembly
and scans the straight-line neighbourhood of every vector-memory
instruction."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "self-evolve-diffusion-cpp_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
NEED = 2  # wait states between a wide (12- or 16-byte) store and a VALU write of its data

_STORE = re.compile(r"^\s*(buffer|global|flat|scratch)_store_dwordx([34])\s+(\S+?),\s*(\S+?),")
_VREG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")


def _regs(tok):
    m = _VREG.match(tok.strip())
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def _scan(asm_text):
    lines = asm_text.split("\n")
    bad = []
    for i, line in enumerate(lines):
        m = _STORE.match(line)
        if not m:
            continue
        # buffer: vdata, vaddr, ...; global/flat/scratch: vaddr, vdata, ...
        data = _regs(m.group(3) if m.group(1) == "buffer" else m.group(4))
        waits = 0
        for nxt in lines[i + 1:i + 40]:
            t = nxt.strip()
            if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
                continue
            op = t.split()[0]
            if op == "s_nop":
                waits += int(t.split()[1], 0) + 1
            elif op.startswith("v_"):
                dst = t.split()[1].rstrip(",") if len(t.split()) > 1 else ""
                if waits < NEED and _regs(dst) & data:
                    bad.append(f"{line.strip()}  ->  {t}")
                    break
                waits += 1
            elif op in ("s_branch", "s_endpgm", "s_setpc_b64") or op.startswith("s_cbranch"):
                break
            else:
                waits += 1
            if waits >= NEED:
                break
    return bad


_VMEM = re.compile(r"^\s*(buffer|global|flat|scratch)_(load|store|atomic)\S*\s+(.*)$")
_SREG = re.compile(r"^s(\d+)$|^s\[(\d+):(\d+)\]$")
SGPR_NEED = 5


def _sregs(tok):
    m = _SREG.match(tok.strip().rstrip(","))
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def _scan_sgpr(asm_text):
    """VALU SGPR write -> vector-memory SGPR read, and M0 write -> LDS-DMA."""
    lines = asm_text.split("\n")
    bad = []
    for i, line in enumerate(lines):
        m = _VMEM.match(line)
        if not m:
            continue
        ops = [t.strip() for t in m.group(3).split(",")]
        used = set()
        for t in ops:
            for tok in t.split():
                used |= _sregs(tok)
        lds_dma = m.group(2) == "load" and re.search(r"\blds\b", line) is not None
        waits = 0
        for prev in reversed(lines[max(0, i - 40):i]):
            t = prev.strip()
            if not t or t.startswith(";") or t.startswith("."):
                continue
            if t.endswith(":"):
                break
            op = t.split()[0]
            if op in ("s_branch", "s_endpgm", "s_setpc_b64") or op.startswith("s_cbranch"):
                break
            if op == "s_nop":
                waits += int(t.split()[1], 0) + 1
                if waits >= SGPR_NEED:
                    break
                continue
            dst = t.split()[1].rstrip(",") if len(t.split()) > 1 else ""
            if op.startswith("v_") and waits < SGPR_NEED and _sregs(dst) & used:
                bad.append(f"{t}  ->  {line.strip()}")
                break
            if lds_dma and dst == "m0" and waits < 1:
                bad.append(f"{t}  ->  {line.strip()}")
                break
            waits += 1
            if waits >= SGPR_NEED:
                break
    return bad


@pytest.mark.slow
@pytest.mark.parametrize("src", ["sdq_gemm.hip", "sdq_quant.hip", "sdq_repack.hip", "sdq_api.hip"])
def test_no_wide_store_data_hazard(tmp_path, src):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-fno-gpu-flush-denormals-to-zero", "-fhip-fp32-correctly-rounded-divide-sqrt",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(ROOT, "include"), "--cuda-device-only", "-S",
           os.path.join(CSRC, src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    bad = _scan(text)
    assert not bad, f"{len(bad)} wide stores followed too closely by a VALU write of their data:\n" + \
        "\n".join(bad[:10])
    bad = _scan_sgpr(text)
    assert not bad, f"{len(bad)} vector-memory instructions read an SGPR / M0 too soon after its write:\n" + \
        "\n".join(bad[:10])


def test_sgpr_scanner_flags_planted_hazards():
    asm = """
    v_readlane_b32 s12, v205, 4
    buffer_store_dwordx4 v[128:131], v133, s[56:59], s12 offen
"""
    assert _scan_sgpr(asm)
    assert not _scan_sgpr(asm.replace("v205, 4\n", "v205, 4\n    s_nop 4\n"))
    desc = """
    v_readfirstlane_b32 s57, v3
    s_mov_b32 s1, 0
    buffer_load_dwordx4 v161, s[56:59], s74 offen lds
"""
    assert _scan_sgpr(desc)
    m0 = """
    s_add_i32 m0, s80, 0x2000
    buffer_load_dwordx4 v161, s[56:59], s74 offen lds
"""
    assert _scan_sgpr(m0)
    assert not _scan_sgpr(m0.replace("0x2000\n", "0x2000\n    s_nop 0\n"))


def test_scanner_flags_a_planted_hazard():
    asm = """
    buffer_store_dwordx4 v[24:27], v28, s[60:63], s10 offen
    v_cndmask_b32_e32 v24, v204, v189, vcc
"""
    assert _scan(asm)
    ok = """
    buffer_store_dwordx4 v[24:27], v28, s[60:63], s10 offen
    s_nop 2
    v_cndmask_b32_e32 v24, v204, v189, vcc
"""
    assert not _scan(ok)
    flat = """
    global_store_dwordx4 v[0:1], v[4:7], off
    v_mov_b32_e32 v8, 0
    v_mov_b32_e32 v5, 0
"""
    assert _scan(flat)
    assert not _scan(flat.replace("v_mov_b32_e32 v8, 0", "v_mov_b32_e32 v8, 0\n    s_nop 0"))
    assert not _scan(flat.replace("v5, 0", "v0, 0"))
