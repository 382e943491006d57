"""The C++17 host mirror of the reference interface (sd::load_sdcpp,
sd::qgemm, sd::gpu::QLinear), driven through lib/test_host.

CPU tests: the .sdcpp v1 reader against our numpy writer (a restatement of
tools/quantize/pack_sdcpp.py) and against the reference's own compiled
loader, plus the error cases of tests/test_sdcpp.cpp:130-143.
GPU tests: sd::qgemm and QLinear (built from a .sdcpp pack, as
OviDit::load_impl does) bit-exact against the oracle."""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import PKG, assert_bitexact

BIN = os.path.join(PKG, "lib", "test_host")


def run(*args, check=True):
    r = subprocess.run([BIN, *map(str, args)], capture_output=True, text=True, timeout=300)
    if check and r.returncode != 0:
        raise AssertionError(f"test_host {args[0]} rc={r.returncode}\n{r.stdout}\n{r.stderr}")
    return r


def listing(path):
    out = {}
    for line in run("sdcpp", path).stdout.splitlines():
        f = line.split()
        name, code, nd = f[0], int(f[1]), int(f[2])
        out[name] = dict(code=code, dims=[int(x) for x in f[3:3 + nd]], off=int(f[3 + nd]))
    return out


def make_pack(path, oracle):
    rng = np.random.default_rng(0)
    tensors = {
        "blocks.0.ffn.0.weight": (rng.standard_normal((96, 700)) * 0.02).astype(np.float32),
        "blocks.0.ffn.0.bias": (rng.standard_normal(96) * 0.01).astype(np.float32),
        "tiny": rng.standard_normal(17).astype(np.float32),
        "f32t": rng.standard_normal((5, 7)).astype(np.float32),
        "blocks.0.self_attn.o.weight": (rng.standard_normal((200, 331)) * 0.02).astype(np.float32),
        "blocks.0.self_attn.o.bias": (rng.standard_normal(200) * 0.01).astype(np.float32),
    }
    written = oracle.write_sdcpp(path, tensors)
    return tensors, written


def test_sdcpp_listing_matches_format(tmp_path, oracle):
    p = str(tmp_path / "a.sdcpp")
    tensors, written = make_pack(p, oracle)
    got = listing(p)
    # 2 quantized (+2 scale views) and 4 raw
    assert set(got) == set(tensors) | {"blocks.0.ffn.0.weight.scale",
                                       "blocks.0.self_attn.o.weight.scale"}
    raw = open(p, "rb").read()
    for name, (code, a, s) in written.items():
        e = got[name]
        assert e["dims"] == list(tensors[name].shape)
        if code == 0:
            assert e["code"] == 2  # DType::I8
            n = a.size
            assert raw[e["off"]:e["off"] + n] == a.tobytes()
            sc = got[name + ".scale"]
            assert sc["off"] == e["off"] + n          # scales right after the int8 blob
            assert raw[sc["off"]:sc["off"] + 4 * s.size] == s.tobytes()
        else:
            assert e["code"] == 0  # DType::F32
            assert raw[e["off"]:e["off"] + a.nbytes] == a.tobytes()


def test_sdcpp_reader_agrees_with_reference_loader(tmp_path, oracle, ref):
    p = str(tmp_path / "b.sdcpp")
    tensors, _ = make_pack(p, oracle)
    got = listing(p)
    for name in tensors:
        r = ref.sdcpp_lookup(p, name)
        assert r["dims"] == got[name]["dims"]
        assert r["data_off"] == got[name]["off"]
        assert r["dtype"] == got[name]["code"]
        if r["scale_off"] >= 0:
            assert r["scale_off"] == got[name + ".scale"]["off"]
        assert r["count"] == len(got)


def _raw_pack(path, entries):
    """A .sdcpp v1 file from (name, code, array) in table order, repeated
    names allowed (the format does not forbid them): code 0 = int8 rows
    followed by one f32 scale per row, code 1 = f32."""
    blobs, table, off = [], [], 0
    for name, code, a in entries:
        if code == 0:
            rows = int(np.prod(a.shape[:-1]))
            blob = a.astype(np.int8).tobytes() + np.arange(1, rows + 1, dtype=np.float32).tobytes()
        else:
            blob = a.astype(np.float32).tobytes()
        nb = name.encode()
        table.append(struct.pack("<I", len(nb)) + nb + struct.pack("<BI", code, a.ndim) +
                     b"".join(struct.pack("<q", d) for d in a.shape) + struct.pack("<Q", off))
        blobs.append(blob)
        off += len(blob)
    with open(path, "wb") as f:
        f.write(b"SDCP" + struct.pack("<II", 1, len(entries)) + b"".join(table) + b"".join(blobs))


def test_sdcpp_repeated_names_follow_reference_loader(tmp_path, ref):
    """Repeated names: the reference's loader emplaces each entry's view and,
    for int8 entries, its ".scale" view in table order, the first view of a
    name winning (src/serde/sdcpp.cpp:107-131). The mirror's load_sdcpp and
    PackIndex::f32_view must give the same view for every name."""
    i8 = lambda *sh: (np.arange(int(np.prod(sh))) % 200 - 100).astype(np.int8).reshape(sh)  # noqa
    f32 = lambda *sh: np.linspace(-1, 1, int(np.prod(sh)), dtype=np.float32).reshape(sh)  # noqa
    entries = [
        ("X", 1, f32(4)), ("X", 0, i8(3, 8)),              # X: the f32; X.scale: the int8's scales
        ("Y.scale", 1, f32(2)), ("Y", 0, i8(2, 8)),        # Y.scale: the raw f32 (first)
        ("Z", 0, i8(2, 8)), ("Z.scale", 1, f32(2)), ("Z", 1, f32(5)),  # Z: int8; Z.scale: scales
        ("W.scale", 0, i8(2, 8)), ("W", 0, i8(2, 8)),      # W.scale: an int8 tensor
        ("V", 0, i8(4, 8)), ("V", 0, i8(5, 8)),            # V and V.scale: the first int8
    ]
    p = str(tmp_path / "rep.sdcpp")
    _raw_pack(p, entries)
    got = listing(p)
    names = sorted(got)
    assert ref.sdcpp_lookup(p, "X")["count"] == len(got)
    for name in names:
        r = ref.sdcpp_lookup(p, name)
        assert r is not None, name
        assert (r["dtype"], r["dims"], r["data_off"]) == (
            got[name]["code"], got[name]["dims"], got[name]["off"]), name
        v = run("f32view", p, name).stdout.split()
        if r["dtype"] == 0:  # DType::F32: the same bytes, raw or an int8 entry's scales
            assert v[0] in ("f32", "scales") and int(v[1]) == r["data_off"], (name, v, r)
        else:
            assert v == ["none"], (name, v)
    assert run("f32view", p, "nothing").stdout.split() == ["none"]


def _corrupt(tmp_path, oracle, fn, tag):
    p = str(tmp_path / "c.sdcpp")
    make_pack(p, oracle)
    data = bytearray(open(p, "rb").read())
    data = fn(data)
    q = str(tmp_path / f"{tag}.sdcpp")
    open(q, "wb").write(bytes(data))
    return q


@pytest.mark.parametrize("tag,fn,msg", [
    ("trunc", lambda d: d[:-64], "data out of bounds"),
    ("magic", lambda d: bytearray(b"X") + d[1:], "bad magic"),
    ("version", lambda d: d[:4] + struct.pack("<I", 2) + d[8:], "unsupported version"),
    ("short", lambda d: d[:15], "truncated"),
    ("hdr", lambda d: d[:40], "truncated"),
])
def test_sdcpp_errors(tmp_path, oracle, tag, fn, msg):
    q = _corrupt(tmp_path, oracle, fn, tag)
    r = run("sdcpp_err", q, check=False)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("sdcpp: ") and msg in r.stdout


def test_sdcpp_missing_file(tmp_path):
    r = run("sdcpp_err", tmp_path / "nope.sdcpp", check=False)
    assert r.returncode == 0 and "cannot open" in r.stdout


def test_sdcpp_bad_dtype_code(tmp_path, oracle):
    p = str(tmp_path / "d.sdcpp")
    oracle.write_sdcpp(p, {"x": np.zeros(4, np.float32)})
    data = bytearray(open(p, "rb").read())
    # header: magic(4) ver(4) count(4) name_len(4) name(1) code(1)
    data[17] = 7
    open(p, "wb").write(bytes(data))
    r = run("sdcpp_err", p, check=False)
    assert r.returncode == 0 and "bad dtype code" in r.stdout


def test_linear_from_pack_checks(tmp_path, oracle):
    p = str(tmp_path / "e.sdcpp")
    make_pack(p, oracle)
    r = run("linear_err", p, "blocks.0.ffn.0", 700, 95, check=False)
    assert r.returncode == 0 and "bad shape" in r.stdout
    r = run("linear_err", p, "blocks.9.ffn.0", 700, 96, check=False)
    assert r.returncode == 0 and "missing tensor" in r.stdout
    # a raw f32 weight (small tensor) is not an int8 pack entry
    oracle.write_sdcpp(p, {"l.weight": np.zeros((4, 8), np.float32),
                           "l.bias": np.zeros(4, np.float32)})
    r = run("linear_err", p, "l", 8, 4, check=False)
    assert r.returncode == 0 and "not an int8" in r.stdout


def test_linear_any_from_pack_checks(tmp_path, oracle):
    """lin()'s checks for either dtype (ovi_dit.cpp:397-415): shapes, a
    missing bias; no GPU call is made before they pass."""
    p = str(tmp_path / "h.sdcpp")
    oracle.write_sdcpp(p, {"head.weight": np.zeros((20, 300), np.float32),
                           "head.bias": np.zeros(20, np.float32),
                           "nob.weight": np.zeros((4, 8), np.float32)})
    r = run("mlin_any_err", p, "head", 300, 21, check=False)
    assert r.returncode == 0 and "bad shape for head.weight" in r.stdout
    r = run("mlin_any_err", p, "nob", 8, 4, check=False)
    assert r.returncode == 0 and "missing tensor nob.bias" in r.stdout


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_linear_any_from_pack_both_dtypes(tmp_path, sdq_dev, oracle):
    """mlin's dispatch (ovi_dit.cpp:66-84) through sd::gpu::linear_from_pack:
    an F32 pack entry (the audio head's [20, 3072] shape: fewer than 65536
    values, so the packer keeps it fp32) runs the fp32 matmul, an I8 one the
    int8 path; each bit-exact with the reference's branch."""
    p = str(tmp_path / "m.sdcpp")
    W = (oracle.randn(20 * 3072, 11) * np.float32(0.02)).reshape(20, 3072)
    b = oracle.randn(20, 12)
    W8 = (oracle.randn(160 * 512, 13) * np.float32(0.02)).reshape(160, 512)  # >= 65536: int8
    b8 = oracle.randn(160, 14)
    written = oracle.write_sdcpp(p, {"head.weight": W, "head.bias": b,
                                     "proj.weight": W8, "proj.bias": b8})
    M = 157
    x = oracle.randn(M * 3072, 15).reshape(M, 3072)
    x.tofile(tmp_path / "x.bin")
    r = run("mlin_any", p, "head", 3072, 20, M, tmp_path / "x.bin", tmp_path / "o.bin")
    assert "int8 0" in r.stdout
    got = np.fromfile(tmp_path / "o.bin", np.float32).reshape(M, 20)
    assert_bitexact(got, oracle.linear_f32(x, np.ascontiguousarray(W.T), b), "F32 head")
    x8 = oracle.randn(M * 512, 16).reshape(M, 512)
    x8.tofile(tmp_path / "x8.bin")
    r = run("mlin_any", p, "proj", 512, 160, M, tmp_path / "x8.bin", tmp_path / "o8.bin")
    assert "int8 1" in r.stdout
    _, q, s = written["proj.weight"]
    got = np.fromfile(tmp_path / "o8.bin", np.float32).reshape(M, 160)
    assert_bitexact(got, oracle.linear(x8, q, s, bias=b8), "I8 proj")
@pytest.mark.gpu
def test_sd_qgemm_host_tensor_api(tmp_path, sdq_dev, oracle):
    M, K, N = 77, 1000, 300
    A = oracle.randn(M * K, 1).reshape(M, K)
    W = oracle.randn(N * K, 2).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    for nm, arr in (("A", A), ("q", q), ("s", s)):
        arr.tofile(tmp_path / f"{nm}.bin")
    r = run("qgemm", M, K, N, tmp_path / "A.bin", tmp_path / "q.bin", tmp_path / "s.bin",
            tmp_path / "o.bin")
    assert "cache entries 1" in r.stdout
    got = np.fromfile(tmp_path / "o.bin", np.float32).reshape(M, N)
    assert_bitexact(got, oracle.qgemm(A, q, s), "sd::qgemm")
    # the driver then rewrote Bq (negated) and bs (doubled) in place: the
    # cache must notice and upload the new contents
    assert "cache entries after rewrite 1" in r.stdout
    got2 = np.fromfile(tmp_path / "o.bin.rewritten", np.float32).reshape(M, N)
    assert_bitexact(got2, oracle.qgemm(A, (-q.astype(np.int16)).astype(np.int8),
                                       (np.float32(2) * s).astype(np.float32)),
                    "sd::qgemm after the weights changed in place")


@pytest.mark.gpu
def test_sd_qgemm_cache_under_threads(tmp_path, sdq_dev, oracle):
    """Four threads call sd::qgemm on the same weights while a fifth keeps
    clearing the weight cache: a device copy dropped from the cache while a
    call uses it must stay valid until that call returns, and every result
    stays bit-exact."""
    M, K, N = 96, 768, 512
    A = oracle.randn(M * K, 5).reshape(M, K)
    W = oracle.randn(N * K, 6).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    for nm, arr in (("A", A), ("q", q), ("s", s)):
        arr.tofile(tmp_path / f"{nm}.bin")
    r = run("qgemm_threads", M, K, N, tmp_path / "A.bin", tmp_path / "q.bin",
            tmp_path / "s.bin", tmp_path / "o.bin", 4, 25)
    assert "calls 100 mismatches 0" in r.stdout, r.stdout
    assert r.stdout.rstrip().endswith("cache entries 0"), r.stdout
    got = np.fromfile(tmp_path / "o.bin", np.float32).reshape(M, N)
    assert_bitexact(got, oracle.qgemm(A, q, s), "sd::qgemm under threads")


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["mlin", "gelu", "gated", "add"])
def test_qlinear_from_pack(tmp_path, sdq_dev, oracle, mode):
    p = str(tmp_path / "f.sdcpp")
    tensors, written = make_pack(p, oracle)
    base, K, N = "blocks.0.self_attn.o", 331, 200
    _, q, s = written[base + ".weight"]
    bias = tensors[base + ".bias"]
    M = 45
    x = oracle.randn(M * K, 3).reshape(M, K)
    g = oracle.randn(N, 4)
    res = oracle.randn(M * N, 5).reshape(M, N)
    x.tofile(tmp_path / "x.bin")
    g.tofile(tmp_path / "g.bin")
    res.tofile(tmp_path / "r.bin")
    run("linear", p, base, K, N, M, mode, tmp_path / "x.bin", tmp_path / "g.bin",
        tmp_path / "r.bin", tmp_path / "o.bin")
    got = np.fromfile(tmp_path / "o.bin", np.float32).reshape(M, N)
    if mode == "mlin":
        assert_bitexact(got, oracle.linear(x, q, s, bias=bias), mode)
    elif mode == "gated":
        assert_bitexact(got, oracle.linear(x, q, s, bias=bias, epilogue="gated", gate=g,
                                           resid=res), mode)
    elif mode == "add":
        assert_bitexact(got, oracle.linear(x, q, s, bias=bias, epilogue="resid", resid=res), mode)
    else:
        want = oracle.linear(x, q, s, bias=bias, epilogue="gelu")
        assert np.all(np.abs(got - want) <= 1e-6 * (1 + np.abs(want)))


@pytest.mark.parametrize("grid", [(1, 1, 1), (3, 4, 5), (31, 45, 80)])
def test_rope_table_3d_matches_oracle(oracle, grid):
    """The host library's RoPE (cos, sin) table equals cosf/sinf of the
    oracle's rope_freqs_3d angles (both pinned to the reference build's
    rope_freqs_3d and apply_rope), bit for bit; 31x45x80 is the 720p/121-frame
    token grid."""
    import sdq

    T, H, W = grid
    cs = sdq.rope_table_3d(T, H, W)
    want = oracle.rope_cs(oracle.rope_freqs_3d(T, H, W, 128, 10000.0))
    assert cs.shape == (T * H * W, 64, 2)
    assert np.array_equal(cs.view(np.uint32), want.reshape(cs.shape).view(np.uint32))


@pytest.mark.parametrize("L,scaling", [(157, 0.19676), (1000, 1.0)])
def test_rope_table_1d_matches_oracle(oracle, L, scaling):
    import sdq

    cs = sdq.rope_table_1d(L, 128, 10000.0, scaling)
    want = oracle.rope_cs(oracle.rope_freqs_1d(L, 128, 10000.0, scaling))
    assert cs.shape == (L, 22, 2)
    assert np.array_equal(cs.view(np.uint32), want.reshape(cs.shape).view(np.uint32))
    with pytest.raises(ValueError):
        sdq.rope_table_1d(L, 127)


REF_CALLER = os.path.join(os.path.dirname(PKG), "oracle", "_ref", "ref_caller")


def _read_ref_caller(path):
    raw = open(path, "rb").read()
    M, K, N = struct.unpack_from("<3q", raw, 0)
    o = 24
    def take(dtype, count, shape):
        nonlocal o
        a = (np.frombuffer(raw, dtype, count, o) if count else np.zeros(0, dtype)).reshape(shape)
        o += a.nbytes
        return a

    A = take(np.float32, M * K, (M, K))
    Wq = take(np.int8, N * K, (N, K))
    sc = take(np.float32, N, (N,))
    out = take(np.float32, M * N, (M, N))
    assert o == len(raw)
    return A, Wq, sc, out


def test_ref_caller_links_without_a_second_tensor():
    """The drop-in link (CPU): libsd_qgemm.so defines sd::qgemm and leaves
    every sd::Tensor member undefined, and the reference-shaped caller built
    with the reference's tensor.cpp loads it and not libsd_host.so."""
    lib = os.path.join(PKG, "lib", "libsd_qgemm.so")
    syms = subprocess.run(["nm", "-DC", lib], capture_output=True, text=True, check=True).stdout
    defined = [ln for ln in syms.splitlines() if " T " in ln or " W " in ln]
    assert any("sd::qgemm(sd::Tensor const&" in ln for ln in defined)
    assert not any("sd::Tensor::" in ln for ln in defined), "libsd_qgemm defines Tensor members"
    assert any(" U sd::Tensor::Tensor(" in ln for ln in syms.splitlines())
    if not os.path.exists(REF_CALLER):
        pytest.skip("oracle/_ref/ref_caller not built (reference sources absent)")
    ldd = subprocess.run(["ldd", REF_CALLER], capture_output=True, text=True, check=True).stdout
    assert "libsd_qgemm.so" in ldd and "libsdq.so" in ldd and "libsd_host" not in ldd
    own = subprocess.run(["nm", "-C", REF_CALLER], capture_output=True, text=True,
                         check=True).stdout
    # the Tensor members are the reference's own (tensor.cpp), defined once, in the
    # program (the destructor's complete and base-object symbols share one address)
    addrs = {ln.split()[0] for ln in own.splitlines() if " T sd::Tensor::~Tensor()" in ln}
    assert len(addrs) == 1


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(17, 31, 13), (64, 1024, 512), (300, 3072, 1000),
                                   (2100, 640, 384), (0, 64, 32), (5, 0, 7), (5, 64, 0)])
def test_ref_caller_bitexact(tmp_path, oracle, M, K, N):
    """A program written against the reference's src/core/tensor.h, linked with
    the reference's tensor.cpp and libsd_qgemm.so, gets the reference's qgemm
    output bit for bit (test_core.cpp's seeds: randu 7+M for A, 13+N for W),
    including the empty shapes for which the reference returns its zero-filled
    output (qgemm.cpp:74-76)."""
    if not os.path.exists(REF_CALLER):
        pytest.skip("oracle/_ref/ref_caller not built (reference sources absent)")
    out = tmp_path / "o.bin"
    r = subprocess.run([REF_CALLER] + [str(v) for v in (M, K, N, 7 + M, 13 + N, out)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    A, Wq, sc, got = _read_ref_caller(out)
    assert_bitexact(got, oracle.qgemm(A, Wq, sc), f"ref_caller {M}x{K}x{N}")
    import pyoracle
    if pyoracle.Ref.available():
        assert_bitexact(got, pyoracle.Ref().qgemm(A, Wq, sc), "reference build")
