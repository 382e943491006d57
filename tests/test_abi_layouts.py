"""Struct layouts across the C ABI (CPU: a small program compiled here).

The binding passes these structs by pointer through ctypes; a Structure whose
fields drifted from the C declaration (an added field, another order or
width) would hand the library shifted values with no error. For every struct
the binding mirrors, g++ compiles the C headers and prints sizeof and each
field's offsetof in declaration order; the ctypes class must match field by
field (by position: some ctypes names differ, e.g. `in_`).
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

from conftest import PKG, ROOT

HEADERS = [os.path.join(ROOT, "include", "sdq.h"), os.path.join(PKG, "host", "sd", "dit_block.h")]
# C struct -> ctypes class of the binding
PAIRS = {
    "sdq_epilogue": "Epilogue", "sdq_device_info": "DeviceInfo", "sdq_weight_src": "WeightSrc",
    "sdq_weight_fsrc": "WeightFileSrc", "sdq_group_item": "GroupItem", "sdq_ffn_item": "FfnItem",
    "sdq_rms_seg": "RmsSeg", "sdq_kernel_time": "KernelTime", "sdq_gemm_plan": "GemmPlan",
    "sd_dit_block_io": "BlockIO", "sd_linear": "Linear", "sd_dit_norms": "DitNorms",
    "sd_dit_block_step": "BlockStep",
}


def _c_fields():
    """struct name -> field names in declaration order, from the headers."""
    out = {}
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \1;", text, flags=re.S):
            names = []
            for decl in m.group(2).split(";"):
                decl = " ".join(decl.split())
                if not decl:
                    continue
                first, *more = [d.strip() for d in decl.split(",")]
                for d in [first] + more:
                    names.append(re.match(r".*?(\w+)\s*(\[.*)?$", d).group(1))
            out[m.group(1)] = names
    return out


@pytest.fixture(scope="module")
def c_layouts(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.fail("g++ is needed for the layout check")
    fields = _c_fields()
    missing = sorted(set(PAIRS) - set(fields))
    assert not missing, f"structs not found in the headers: {missing}"
    src = ['#include <cstddef>', '#include <cstdio>', '#include "sdq.h"', '#include "sd/dit_block.h"',
           "int main() {"]
    for s in PAIRS:
        offs = " ".join(f'printf(" %zu", offsetof({s}, {f}));' for f in fields[s])
        src.append(f'printf("{s} %zu", sizeof({s})); {offs} printf("\\n");')
    src.append("return 0; }")
    d = tmp_path_factory.mktemp("layouts")
    (d / "lay.cpp").write_text("\n".join(src))
    exe = d / "lay"
    subprocess.run([gxx, "-std=c++17", f"-I{ROOT}/include", f"-I{PKG}/host", str(d / "lay.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    lay = {}
    for line in out.splitlines():
        name, size, *offs = line.split()
        lay[name] = (int(size), [int(o) for o in offs])
    return fields, lay


@pytest.mark.parametrize("cstruct", sorted(PAIRS))
def test_ctypes_layout_matches_c(c_layouts, cstruct):
    import sdq

    fields, lay = c_layouts
    cls = getattr(sdq, PAIRS[cstruct])
    size, offs = lay[cstruct]
    ct = [(name, getattr(cls, name).offset) for name, *_ in cls._fields_]
    assert len(ct) == len(offs), (cstruct, fields[cstruct], [n for n, _ in ct])
    for (cname, coff), cf, off in zip(ct, fields[cstruct], offs):
        assert coff == off, f"{cstruct}.{cf} at {off}, binding's {cname} at {coff}"
    assert ctypes.sizeof(cls) == size, (cstruct, size, ctypes.sizeof(cls))
