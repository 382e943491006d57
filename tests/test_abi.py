"""C ABI surface (no GPU needed): the library loads, exports exactly what
include/sdq.h declares, links nothing from oracle/, and errors cleanly."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import PKG, ROOT

HEADER = os.path.join(ROOT, "include", "sdq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sdq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("sdq_init", "sdq_weight_upload", "sdq_qlinear", "sdq_qgemm",
                 "sdq_qlinear_host", "sdq_act_quant", "sdq_weight_free", "sdq_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import sdq

    lib = sdq.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(sdq.SIGNATURES), "binding out of sync with header"


def test_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", os.path.join(PKG, "lib", "libsdq.so")], capture_output=True,
                         text=True).stdout
    assert "oracle" not in out and "sdref" not in out
    nm = subprocess.run(["nm", "-D", "--defined-only", os.path.join(PKG, "lib", "libsdq.so")],
                        capture_output=True, text=True).stdout
    assert "orc_" not in nm and "sdref_" not in nm


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import sdq

    monkeypatch.setattr(sdq, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        sdq.load_library(str(tmp_path / "nope.so"))


def test_errors_without_device_are_codes_not_crashes():
    """Argument validation runs before any device work."""
    import sdq

    lib = sdq.load_library()
    out = ctypes.c_void_p()
    rc = lib.sdq_weight_upload(None, None, -1, 4, None, ctypes.byref(out))
    assert rc == sdq.ERR_INVALID
    assert b"negative" in lib.sdq_last_error()
    rc = lib.sdq_qgemm(None, None, 4, 4, None, None)
    assert rc == sdq.ERR_INVALID
    assert b"null weight" in lib.sdq_last_error()
    assert lib.sdq_weight_free(None) == 0
    assert lib.sdq_version().startswith(b"sdq")


def test_host_mirror_headers_compile_standalone(tmp_path):
    """The C++17 mirror of the reference interface builds with plain g++."""
    src = tmp_path / "use.cpp"
    src.write_text(
        '#include "sd/tensor.h"\n#include "sd/pack.h"\n#include "sd/qlinear.h"\n'
        "int main(){ sd::Tensor t({2,3}, sd::DType::F32); return (int)t.numel() - 6; }\n")
    exe = tmp_path / "use"
    r = subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-I",
                        os.path.join(PKG, "host"), str(src), "-o", str(exe), "-L",
                        os.path.join(PKG, "lib"), "-lsd_host", "-lsdq",
                        "-Wl,-rpath," + os.path.join(PKG, "lib")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert subprocess.run([str(exe)]).returncode == 0


def test_host_library_exports_its_c_shim():
    """libsd_host.so exports every C function of the host mirror's headers
    (the sd_dit_block_* shim, sd_rope_table_*), which the Python binding and
    non-C++ callers use."""
    import glob

    import sdq

    names = set()
    for h in glob.glob(os.path.join(PKG, "host", "sd", "*.h")):
        text = re.sub(r"/\*.*?\*/|//[^\n]*", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"^(?:int|double|size_t|const char\*|void)\s+(sd_[a-z0-9_]+)\s*\(",
                                text, flags=re.M))
    assert {"sd_dit_block_step_forward", "sd_rope_table_3d", "sd_dit_block_set_norms"} <= names
    lib = sdq.load_host_library()
    missing = sorted(n for n in names if not hasattr(lib, n))
    assert not missing, missing


def _prototypes(header=HEADER, prefix="sdq_"):
    """name -> (return type, [parameter types]) of every function named
    prefix* declared in `header`."""
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"#.*", "", text)
    protos = {}
    pat = r"([A-Za-z_][\w\s\*]*?)\b(" + prefix + r"[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;"
    for m in re.finditer(pat, text):
        ret, name, params = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        if params in ("", "void"):
            protos[name] = (ret, [])
            continue
        types = []
        for p in params.split(","):
            p = " ".join(p.split())
            # drop the parameter name (the last identifier), keep the type and its stars
            types.append(re.sub(r"\s*\b\w+$", "", p) if re.search(r"[\w\*]\s+\w+$", p) else p)
        protos[name] = (ret, types)
    return protos


def test_binding_signatures_match_the_header():
    """Every prototype's parameter count, scalar types and pointer-ness as
    the Python binding declares them: a drift would pass wrong arguments
    through ctypes without any error until a GPU run."""
    import sdq

    scalar = {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
              "float": ctypes.c_float, "double": ctypes.c_double}
    protos = _prototypes()
    assert set(protos) == set(sdq.SIGNATURES)
    for name, (ret, params) in protos.items():
        res, args = sdq.SIGNATURES[name]
        assert len(args) == len(params), (name, params, args)
        for p, a in zip(params, args):
            if "*" in p:
                assert a in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(a, ctypes._Pointer), \
                    (name, p, a)
            else:
                base = p.replace("const ", "").strip()
                assert scalar.get(base) is a, (name, p, a)
        if "*" in ret:
            assert res is ctypes.c_char_p, (name, ret)
        else:
            assert scalar[ret.replace("const ", "").strip()] is res, (name, ret, res)


def test_host_shim_signatures_match_its_headers():
    """The same for libsd_host.so's C shim (sd_dit_*, sd_rope_*), whose
    argument types the binding sets on the loaded library."""
    import sdq

    scalar = {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
              "float": ctypes.c_float, "double": ctypes.c_double}
    host = sdq.load_host_library()
    protos = {}
    for h in ("dit_block.h", "rope.h"):
        protos.update(_prototypes(os.path.join(PKG, "host", "sd", h), "sd_"))
    assert "sd_dit_block_forward" in protos and "sd_rope_table_3d" in protos
    unbound = []
    for name, (ret, params) in sorted(protos.items()):
        fn = getattr(host, name)
        if fn.argtypes is None:
            unbound.append(name)
            continue
        assert len(fn.argtypes) == len(params), (name, params, fn.argtypes)
        for p, a in zip(params, fn.argtypes):
            if "*" in p:
                assert a in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(a, ctypes._Pointer), \
                    (name, p, a)
            else:
                assert scalar.get(p.replace("const ", "").strip()) is a, (name, p, a)
        want = ctypes.c_char_p if "*" in ret else scalar[ret.replace("const ", "").strip()]
        assert fn.restype is want, (name, ret, fn.restype)
    assert not unbound, f"declared but not bound by the binding: {unbound}"
