"""sdq_qlinear_group: several independent Linears in one call (one segmented
quantizer launch, one persistent GEMM launch per set of items with the same
K and epilogue form, the other items as separate calls) gives the same bits
as one sdq_qlinear per item, and the oracle's results."""
import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _weight(sdq, oracle, N, K, seed):
    W = (oracle.randn(N * K, seed) * np.float32(0.03)).reshape(N, K)
    q, s = oracle.quant_rows(W)
    return sdq.Weight.from_host(q, s), q, s


def _items(sdq, torch, oracle, dev, specs, seed0):
    """specs: (M, K, N, kind, bias?) -> item dicts with inputs on the GPU."""
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa: E731
    items, host = [], []
    for i, (M, K, N, kind, has_bias) in enumerate(specs):
        sd = seed0 + 10 * i
        w, q, s = _weight(sdq, oracle, N, K, sd)
        A = oracle.randn(M * K, sd + 1).reshape(M, K)
        b = oracle.randn(N, sd + 2) if has_bias else None
        g = oracle.randn(N, sd + 3)
        r = oracle.randn(M * N, sd + 4).reshape(M, N)
        fma = kind != "gated_nofma"
        kind = "gated" if kind == "gated_nofma" else kind
        it = dict(w=w, A=t(A), out=torch.full((M, N), float("nan"), device=dev), kind=kind,
                  bias=None if b is None else t(b), gate_fma=fma)
        if kind == "gated":
            it.update(gate=t(g), resid=it["out"])
            it["out"].copy_(t(r))
        elif kind == "resid":
            it.update(resid=it["out"])
            it["out"].copy_(t(r))
        items.append(it)
        host.append(dict(A=A, q=q, s=s, b=b, g=g, r=r, kind=kind, fma=fma))
    return items, host


def _separate(sdq, torch, items, host):
    outs = []
    for it, h in zip(items, host):
        y = torch.from_numpy(h["r"]).to(it["out"].device).contiguous() if h["kind"] in (
            "gated", "resid") else torch.empty_like(it["out"])
        sdq.qlinear(it["w"], it["A"], y, kind=h["kind"], bias=it["bias"], gate=it.get("gate"),
                    resid=y if h["kind"] in ("gated", "resid") else None, gate_fma=h["fma"])
        outs.append(y)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def _oracle(oracle, h):
    kw = dict(bias=h["b"])
    if h["kind"] == "gated":
        kw.update(epilogue="gated", gate=h["g"], resid=h["r"], use_fma=h["fma"])
    elif h["kind"] == "resid":
        kw.update(epilogue="resid", resid=h["r"])
    return oracle.linear(h["A"], h["q"], h["s"], **kw)


@pytest.mark.parametrize("case", ["one_set", "mixed", "mixed_forms"])
def test_group_equals_separate_calls(sdq_dev, oracle, case):
    import torch

    import sdq

    if case == "one_set":
        specs = [(100, 512, 384, "none", True), (157, 512, 256, "none", True),
                 (300, 512, 640, "none", True), (65, 512, 128, "none", True)]
    elif case == "mixed_forms":
        # one launch whose problems differ in epilogue kind, bias and gate form
        # (a block's q|k|v beside its gated output projection)
        specs = [(768, 1024, 768, "none", True), (768, 1024, 256, "gated", True),
                 (157, 1024, 256, "gated_nofma", False), (300, 1024, 384, "resid", False),
                 (129, 1024, 512, "gelu", True), (90, 1024, 128, "none", False)]
    else:
        specs = [(120, 512, 256, "gated", True), (90, 512, 512, "resid", True),
                 (77, 512, 256, "gelu", True), (20, 512, 256, "none", True),   # skinny: alone
                 (200, 512, 96, "none", False), (150, 1024, 256, "none", True),
                 (133, 512, 384, "none", True), (0, 512, 128, "none", True),
                 (2100, 512, 1024, "none", True), (129, 1024, 384, "none", True)]
    print(f"[group] {case}: {len(specs)} items", flush=True)
    items, host = _items(sdq, torch, oracle, sdq_dev, specs, 100)
    sdq.qlinear_group(items)
    torch.cuda.synchronize()
    got = [it["out"].cpu().numpy() for it in items]
    want = _separate(sdq, torch, items, host)
    for i, (g, w, h) in enumerate(zip(got, want, host)):
        assert_bitexact(g, w, f"item {i} ({specs[i]}) vs its own sdq_qlinear")
        if h["kind"] != "gelu" and specs[i][0] > 0:
            assert_bitexact(g, _oracle(oracle, h), f"item {i} vs the oracle")
    for it in items:
        it["w"].free()


def test_group_repeated_growing_and_shrinking(sdq_dev, oracle):
    """Consecutive calls of different sizes on one stream (the group scratch
    grows, then is reused by a smaller call)."""
    import torch

    import sdq

    for rnd, specs in enumerate(([(70, 512, 128, "none", True), (80, 512, 256, "none", True)],
                                 [(700, 1024, 1024, "none", True), (300, 1024, 512, "none", True),
                                  (257, 1024, 768, "none", True)],
                                 [(66, 512, 128, "resid", True), (99, 512, 256, "resid", True)])):
        print(f"[group] round {rnd}", flush=True)
        items, host = _items(sdq, torch, oracle, sdq_dev, specs, 500 + 50 * rnd)
        sdq.qlinear_group(items)
        torch.cuda.synchronize()
        for i, (it, h) in enumerate(zip(items, host)):
            assert_bitexact(it["out"].cpu().numpy(), _oracle(oracle, h), f"round {rnd} item {i}")
            it["w"].free()


def test_group_raw_abi_errors(sdq_dev, oracle):
    import ctypes

    import sdq

    lib = sdq.load_library()
    assert lib.sdq_qlinear_group(None, -1, None) == sdq.ERR_INVALID
    assert lib.sdq_qlinear_group(None, 17, None) == sdq.ERR_INVALID
    assert lib.sdq_qlinear_group(None, 0, None) == 0
    arr = (sdq.GroupItem * 1)()
    assert lib.sdq_qlinear_group(arr, 1, None) == sdq.ERR_INVALID  # null weight
    w, _, _ = _weight(sdq, oracle, 128, 512, 9)
    arr[0].w = w.h
    arr[0].M = 5
    assert lib.sdq_qlinear_group(arr, 1, None) == sdq.ERR_INVALID  # null A / Y
    assert b"null A or Y" in lib.sdq_last_error()
    arr[0].epi.kind = 2  # gated without gate / resid
    arr[0].A = arr[0].Y = ctypes.c_void_p(16)
    assert lib.sdq_qlinear_group(arr, 1, None) == sdq.ERR_INVALID
    w.free()


def test_group_rejects_overlapping_items(sdq_dev, oracle):
    """One item's output over another item's input, residual or output is
    refused before anything runs (the items run in any order); an item's own
    residual may be its own output."""
    import torch

    import sdq

    specs = [(96, 512, 512, "none", True), (96, 512, 256, "resid", True)]
    items, host = _items(sdq, torch, oracle, sdq_dev, specs, 900)
    before = [it["out"].clone() for it in items]
    buf = torch.zeros((96, 512), device=sdq_dev)
    # item 0 writes the buffer that item 1 reads as its input
    items[0]["out"] = buf
    items[1]["A"] = buf
    with pytest.raises(sdq.SdqError) as ei:
        sdq.qlinear_group(items)
    assert "overlaps" in str(ei.value)
    # item 1 writes into item 0's output (a view of the same storage)
    items[0]["out"] = before[0].clone()
    items[1]["A"] = torch.from_numpy(host[1]["A"]).to(sdq_dev)
    items[1]["out"] = items[1]["resid"] = items[0]["out"].view(-1)[: 96 * 256].view(96, 256)
    with pytest.raises(sdq.SdqError) as ei:
        sdq.qlinear_group(items)
    assert "overlaps" in str(ei.value)
    torch.cuda.synchronize()
    for it in items:
        it["w"].free()


def _stack_case(sdq, torch, oracle, dev, specs, seq_specs, ffn_shape, seed, chain=None):
    """items: grouped `specs` then `seq_specs` (M, K, N, kind, bias); with
    `chain` = i, the later items of a residual kind and the FFN update grouped
    item i's output in place after it (as a block's cross o and FFN follow its
    o, all on x); plus an FFN (M, D, F) or None. Returns (stack results,
    separate-call results)."""
    items, _ = _items(sdq, torch, oracle, dev, specs + seq_specs, seed)
    ng = len(specs)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa
    ffn = None
    if ffn_shape is not None:
        M, D, F = ffn_shape
        w1, _, _ = _weight(sdq, oracle, F, D, seed + 900)
        w2, _, _ = _weight(sdq, oracle, D, F, seed + 910)
        ffn = dict(fc1=w1, fc2=w2, b1=t(oracle.randn(F, seed + 920) * np.float32(0.01)),
                   b2=t(oracle.randn(D, seed + 921) * np.float32(0.01)),
                   h=t(oracle.randn(M * D, seed + 922).reshape(M, D)),
                   gate=t(oracle.randn(D, seed + 923)), hid=torch.empty((M, F), device=dev),
                   x=t(oracle.randn(M * D, seed + 924).reshape(M, D)))

    def link(its, f):
        if chain is None:
            return
        x = its[chain]["out"]
        for it in its[ng:]:
            if it["kind"] in ("gated", "resid"):
                it["out"] = it["resid"] = x
        if f is not None:
            f["x"] = x

    # the separate calls, on copies of every output
    ref = [dict(it, out=it["out"].clone()) for it in items]
    for it in ref:
        if it["kind"] in ("gated", "resid"):
            it["resid"] = it["out"]
    rffn = None if ffn is None else dict(ffn, hid=ffn["hid"].clone(), x=ffn["x"].clone())
    link(items, ffn)
    link(ref, rffn)
    sdq.qlinear_group(ref[:ng])
    for it in ref[ng:]:
        sdq.qlinear(it["w"], it["A"], it["out"], kind=it["kind"], bias=it["bias"],
                    gate=it.get("gate"), resid=it.get("resid"), gate_fma=it["gate_fma"])
    if rffn is not None:
        sdq.ffn(rffn["fc1"], rffn["b1"], rffn["fc2"], rffn["b2"], rffn["h"], rffn["gate"],
                rffn["hid"], rffn["x"])
    sdq.qlinear_stack(items, ng, ffn)
    torch.cuda.synchronize()
    got = [it["out"].cpu().numpy() for it in items]
    want = [it["out"].cpu().numpy() for it in ref]
    if ffn is not None:
        got += [ffn["hid"].cpu().numpy(), ffn["x"].cpu().numpy()]
        want += [rffn["hid"].cpu().numpy(), rffn["x"].cpu().numpy()]
    for it in items:
        it["w"].free()
    if ffn is not None:
        ffn["fc1"].free()
        ffn["fc2"].free()
    return got, want


@pytest.mark.parametrize("case", ["block768", "block157", "no_ffn", "fallback_skinny", "big_rows"])
def test_stack_equals_separate_calls(sdq_dev, oracle, case):
    """sdq_qlinear_stack against qlinear_group + qlinear per later item +
    ffn, bit for bit: a block's shapes at small widths (every input through
    the shared quantizer launch), a stack without FFN, one whose item takes
    another path (few rows: the whole stack runs as the separate calls), and
    256x256 tiles for the sequential item and fc1."""
    import torch

    import sdq

    D = 512
    if case == "block768":
        specs = [(768, D, 3 * D, "none", True), (768, D, D, "gated", True),
                 (768, D, D, "none", True), (96, D, 2 * D, "none", True), (157, D, 2 * D, "none", True)]
        seq, ffn = [(768, D, D, "resid", True)], (768, D, 4 * D)
    elif case == "block157":
        specs = [(157, D, 3 * D, "none", True), (157, D, D, "gated", True),
                 (157, D, D, "none", True), (96, D, 2 * D, "none", True), (768, D, 2 * D, "none", True)]
        seq, ffn = [(157, D, D, "resid", True)], (157, D, 4 * D)
    elif case == "no_ffn":
        specs = [(300, D, 256, "none", True), (300, D, 384, "gelu", False)]
        seq, ffn = [(300, D, 256, "resid", False), (200, D, 512, "none", True)], None
    elif case == "fallback_skinny":
        specs = [(300, D, 256, "none", True), (40, D, 128, "none", True)]
        seq, ffn = [(300, D, 256, "gated", True)], (130, D, 2 * D)
    else:  # 256x256 tiles for the later item and fc1 (>= 2 rounds of them)
        specs = [(256, D, 512, "none", True), (256, D, 256, "gated", True)]
        seq, ffn = [(8192, D, 4096, "none", True)], (8192, D, 4096)
    print(f"[stack] {case}", flush=True)
    chain = 1 if case.startswith("block") else None
    got, want = _stack_case(sdq, torch, oracle, sdq_dev, specs, seq, ffn, 700, chain)
    for i, (g, w) in enumerate(zip(got, want)):
        assert_bitexact(g, w, f"{case}: output {i} vs the separate calls")


def test_stack_rejects_overlaps(sdq_dev, oracle):
    """An output over an input that the stack quantizes up front (here a later
    item writing the first item's input), or two grouped items writing the
    same buffer, is refused before anything runs."""
    import torch

    import sdq

    specs = [(96, 512, 512, "none", True), (96, 512, 512, "none", True)]
    items, _ = _items(sdq, torch, oracle, sdq_dev, specs, 950)
    items[1]["out"] = items[0]["A"]
    with pytest.raises(sdq.SdqError) as ei:
        sdq.qlinear_stack(items, 1)
    assert "overlaps the input" in str(ei.value)
    items[1]["out"] = items[0]["out"]
    with pytest.raises(sdq.SdqError) as ei:
        sdq.qlinear_stack(items, 2)
    assert "writes the output" in str(ei.value)
    torch.cuda.synchronize()
    for it in items:
        it["w"].free()


def _random_stack(i):
    """Draws 0-6: shapes that the stack's shared quantizer launch takes (more
    than 64 rows, N a multiple of 4); draws 7-9 also few rows or a ragged N,
    so that the stack falls back to the separate calls."""
    r = np.random.default_rng(6600 + i)
    Ks = [256, 512, 1024, 1536]
    kinds = ["none", "gelu", "gated", "gated_nofma", "resid"]
    odd = 0.25 if i >= 7 else 0.0

    def spec(k_choices):
        M = int(r.integers(1, 65)) if r.random() < odd else int(r.integers(65, 900))
        N = int(r.integers(1, 1400)) if r.random() < odd else 4 * int(r.integers(16, 350))
        return (M, int(r.choice(k_choices)), N, str(r.choice(kinds)), bool(r.random() < 0.7))

    group = [spec(Ks) for _ in range(int(r.integers(1, 7)))]
    seq = [spec(Ks) for _ in range(int(r.integers(0, 4)))]
    ffn = None
    if r.random() < 0.6:
        D = int(r.choice(Ks))
        ffn = (int(r.integers(65, 900)), D, D * int(r.choice([2, 4])))
    return group, seq, ffn


@pytest.mark.parametrize("i", range(10))
def test_stack_random_sets(sdq_dev, oracle, i):
    """Seeded random stacks (1-6 grouped items, 0-3 later items, an FFN or
    not; mixed rows, K, N, epilogue forms and bias) against qlinear_group, then
    qlinear per later item, then ffn: bit for bit, on the shared quantizer
    launch and on the fallback path."""
    import torch

    import sdq

    group, seq, ffn = _random_stack(i)
    print(f"[stack-random] {i} group={group} seq={seq} ffn={ffn}", flush=True)
    got, want = _stack_case(sdq, torch, oracle, sdq_dev, group, seq, ffn, 1300 + 50 * i)
    for j, (g, w) in enumerate(zip(got, want)):
        assert_bitexact(g, w, f"random stack {i}: output {j}")


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("s_kind", ["gated", "gated_nofma", "resid"])
@pytest.mark.parametrize("g_kind", ["gated", "gated_nofma", "resid"])
def test_stack_folded_residual_pair(sdq_dev, oracle, monkeypatch, g_kind, s_kind, fold):
    """The first later item adds into the output a grouped item adds into
    (every pair of residual forms, with and without bias): the stack runs it
    in the grouped launch, both plain outputs to scratch and one elementwise
    pass applying the two residual steps in order. A second later item and
    the FFN then add into the same output after it. Bit for bit against the
    separate calls, with the fold and with it switched off
    (SDQ_NO_STACK_FOLD)."""
    import torch

    import sdq

    if not fold:
        monkeypatch.setenv("SDQ_NO_STACK_FOLD", "1")
    D = 512
    specs = [(300, D, 3 * D, "none", True), (300, D, D, g_kind, s_kind != "resid"),
             (200, D, 2 * D, "none", False)]
    seq = [(300, D, D, s_kind, g_kind == "resid"), (300, D, D, "resid", True)]
    print(f"[stack-fold] {g_kind} then {s_kind} fold={fold}", flush=True)
    got, want = _stack_case(sdq, torch, oracle, sdq_dev, specs, seq, (300, D, 2 * D), 4100, chain=1)
    for j, (g, w) in enumerate(zip(got, want)):
        assert_bitexact(g, w, f"fold {g_kind}+{s_kind} ({fold}): output {j}")


def _random_chain(i):
    """A group with one residual-form item (the target), later items of which
    those with a residual form add into the target after it (the first of them
    always, with the target's shape), and an FFN adding into it last or none."""
    r = np.random.default_rng(7700 + i)
    K = int(r.choice([256, 512, 1024]))
    M = int(r.integers(65, 900))
    N = 4 * int(r.integers(16, 300))
    res = ["gated", "gated_nofma", "resid"]
    others = ["none", "gelu"] + res
    target = (M, K, N, str(r.choice(res)), bool(r.random() < 0.7))
    group = [(int(r.integers(65, 900)), K, 4 * int(r.integers(16, 300)), "none",
              bool(r.random() < 0.7)) for _ in range(int(r.integers(0, 4)))]
    t = int(r.integers(0, len(group) + 1))
    group.insert(t, target)
    seq = [(M, int(r.choice([K, 2 * K])), N, str(r.choice(res)), bool(r.random() < 0.7))]
    for _ in range(int(r.integers(0, 3))):
        kind = str(r.choice(others))
        seq.append((M, K, N, kind, bool(r.random() < 0.7)) if kind in res else
                   (int(r.integers(65, 900)), K, 4 * int(r.integers(16, 300)), kind, True))
    ffn = (M, N, N * int(r.choice([2, 4]))) if r.random() < 0.6 else None
    return group, seq, ffn, t


@pytest.mark.parametrize("i", range(8))
def test_stack_random_chained(sdq_dev, oracle, i):
    """Seeded random stacks whose later residual items (and FFN) add into a
    grouped item's output, as a block's cross output projection and FFN add
    into x after its self-attention output: bit for bit against qlinear_group,
    then qlinear per later item, then ffn. The first later item takes the
    folded path when it shares the target's K (same k-fragments), the
    separate one otherwise."""
    import torch

    import sdq

    group, seq, ffn, t = _random_chain(i)
    print(f"[stack-chain] {i} group={group} target={t} seq={seq} ffn={ffn}", flush=True)
    got, want = _stack_case(sdq, torch, oracle, sdq_dev, group, seq, ffn, 5200 + 50 * i, chain=t)
    for j, (g, w) in enumerate(zip(got, want)):
        assert_bitexact(g, w, f"chained stack {i}: output {j}")
