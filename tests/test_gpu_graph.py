"""HIP-graph capture of the qGEMM entry points (GPU, through the binding).

sdq_qlinear keeps a workspace per stream, grown by a call larger than any
before it on that stream. Growing drains the stream and allocates, which a
capturing stream cannot do, so such a call is refused with an error and the
capture stays usable. After one eager call on the capture stream the same
call captures; sdq_qlinear_noalloc captures without that warm-up.

Each graph is replayed three times with new inputs written eagerly between
the replays. Every replay must equal the eager call on the same inputs bit
for bit (the eager path is pinned against the oracle elsewhere). The shapes
cover every launch form a captured call can contain: the quantizer, 128x128
tiles with a gated epilogue, split-K partials and their reduction, the
skinny kernels (one of them quantizing its few rows itself), and 256x256
tiles followed by the 128x128 tail.
"""
import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu

# (M, K, N, kind): 128x128 tiles + gated; split-K + gated reduction; the
# skinny kernel; a few rows quantized inside the GEMM; 256x256 + 128x128 tail
SHAPES = [(300, 3072, 1000, "gated"), (157, 14336, 3072, "gated"), (64, 14336, 1024, "none"),
          (2, 3072, 512, "none"), (8592, 256, 4096, "none")]


def _setup(sdq_dev, oracle, M, K, N, kind, seed):
    import torch

    import sdq

    W = oracle.randn(N * K, seed).reshape(N, K) * np.float32(0.02)
    q, s = oracle.quant_rows(W)
    w = sdq.Weight.from_host(q, s)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(sdq_dev)  # noqa: E731
    b = t(oracle.randn(N, seed + 1) * np.float32(0.01))
    g = t(oracle.randn(N, seed + 2)) if kind == "gated" else None
    A = torch.empty((M, K), device=sdq_dev)
    X = torch.empty((M, N), device=sdq_dev)
    return w, b, g, A, X


def _call(sdq, fn, w, A, Y, kind, b, g, X):
    fn(w, A, Y, kind=kind, bias=b, gate=g, resid=X if kind == "gated" else None)


def _replays(sdq_dev, oracle, fn, M, K, N, kind, seed, warm):
    import torch

    import sdq

    print(f"[graph] {fn.__name__} M={M} K={K} N={N} {kind} warm={warm}", flush=True)
    w, b, g, A, X = _setup(sdq_dev, oracle, M, K, N, kind, seed)
    print(f"[graph] plan {sdq.qlinear_plan(w, M, kind)}", flush=True)
    Yg = torch.zeros((M, N), device=sdq_dev)
    Ye = torch.zeros((M, N), device=sdq_dev)
    A.copy_(torch.randn((M, K), device=sdq_dev))
    X.copy_(torch.randn((M, N), device=sdq_dev))
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    if warm:
        with torch.cuda.stream(s):
            _call(sdq, fn, w, A, Yg, kind, b, g, X)
        s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        _call(sdq, fn, w, A, Yg, kind, b, g, X)
    for rep in range(3):
        A.copy_(torch.randn((M, K), device=sdq_dev))
        X.copy_(torch.randn((M, N), device=sdq_dev))
        Yg.fill_(-1.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _call(sdq, sdq.qlinear, w, A, Ye, kind, b, g, X)
        torch.cuda.synchronize()
        assert_bitexact(Yg.cpu().numpy(), Ye.cpu().numpy(),
                        f"{fn.__name__} replay {rep} M={M} K={K} N={N} {kind}")
    del graph
    w.free()


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s[:3])) + "_" + s[3])
def test_qlinear_captures_after_one_eager_call(sdq_dev, oracle, shape):
    import sdq

    M, K, N, kind = shape
    _replays(sdq_dev, oracle, sdq.qlinear, M, K, N, kind, 100, warm=True)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s[:3])) + "_" + s[3])
def test_noalloc_captures_without_warmup(sdq_dev, oracle, shape):
    import sdq

    M, K, N, kind = shape
    _replays(sdq_dev, oracle, sdq.qlinear_noalloc, M, K, N, kind, 200, warm=False)


def test_growth_under_capture_is_refused(sdq_dev, oracle):
    """A call with more rows than any call before it on the stream (torch
    hands out pooled streams, so the row count, not the stream, makes it new)
    would grow the stream's workspace: under capture it raises before anything
    is queued, the capture still ends normally, and the stream captures the
    call once it has run eagerly."""
    import torch

    import sdq

    M, K, N = 200000, 256, 64
    print(f"[graph] growth refused M={M} K={K} N={N}", flush=True)
    w, b, _, A, _ = _setup(sdq_dev, oracle, M, K, N, "none", 300)
    A.copy_(torch.randn((M, K), device=sdq_dev))
    Y = torch.zeros((M, N), device=sdq_dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(sdq.SdqError, match="captures a graph"):
        with torch.cuda.graph(graph, stream=s):
            sdq.qlinear(w, A, Y, bias=b)
    del graph
    _replays(sdq_dev, oracle, sdq.qlinear, M, K, N, "none", 300, warm=True)
    w.free()

_BLOCK_NAMES = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "kf", "vf", "fc1", "fc2")


def _block_weights(oracle, dim, ffn, seed):
    lin = {}
    for i, n in enumerate(_BLOCK_NAMES):
        out, inp = (ffn, dim) if n == "fc1" else ((dim, ffn) if n == "fc2" else (dim, dim))
        W = oracle.randn(out * inp, seed + 10 * i).reshape(out, inp) * np.float32(0.02)
        q, s = oracle.quant_rows(W)
        lin[n] = (q, s, oracle.randn(out, seed + 10 * i + 1) * np.float32(0.01))
    return lin


def test_pair_pass_captures_and_replays(sdq_dev, oracle):
    """HIP-graph capture of the twin pair pass (DitBlock.forward_pair over two
    streams), two fusion layers at small widths: after one eager pass on the
    capture stream and the second stream (their workspaces then large enough),
    the pass is captured, joined back by the pair's own stream waits, and
    replayed three times with new inputs written eagerly between the replays.
    Every replay's outputs equal an eager pass on the same inputs, bit for bit
    (the eager pair pass is pinned against the oracle in test_gpu_block.py)."""
    import torch

    import sdq

    dim, ffn, Mv, Ma, Mc, layers = 512, 1408, 300, 90, 77, 2
    print(f"[graph-pair] dim={dim} Mv={Mv} Ma={Ma} Mc={Mc} layers={layers}", flush=True)
    blocks = [sdq.DitBlock(_block_weights(oracle, dim, ffn, 1000 + 100 * b), True)
              for b in range(2 * layers)]
    dev = sdq_dev

    def io(M, Mt):
        r = lambda rows: torch.empty((rows, dim), device=dev)  # noqa: E731
        return dict(M=M, Mc=Mc, Mt=Mt, h_sa=r(M), att=r(M), xq=r(M), ctx=r(Mc), tn=r(Mt),
                    xt=r(M), h_ffn=r(M), x=r(M), gate_sa=torch.empty(dim, device=dev),
                    gate_ffn=torch.empty(dim, device=dev),
                    qkv=torch.empty((M, 3 * dim), device=dev), cq=r(M),
                    ckv=torch.empty((Mc, 2 * dim), device=dev),
                    kvt=torch.empty((Mt, 2 * dim), device=dev),
                    hid=torch.empty((M, ffn), device=dev))

    iov, ioa = io(Mv, Ma), io(Ma, Mv)
    tensors = [(k, v) for d in (iov, ioa) for k, v in d.items() if torch.is_tensor(v)]

    def fill(seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        for _, t in tensors:
            t.copy_(torch.randn(t.shape, generator=g, device=dev))

    s, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def passes():
        for i in range(layers):
            blocks[2 * i].forward_pair(blocks[2 * i + 1], iov, ioa, stream2=s2)

    fill(1)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        passes()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        passes()
    torch.cuda.synchronize()
    for rep in range(3):
        fill(10 + rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {f"{which}.{k}": v.cpu().numpy() for which, d in (("v", iov), ("a", ioa))
               for k, v in d.items() if torch.is_tensor(v)}
        fill(10 + rep)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            passes()
        torch.cuda.synchronize()
        for name, a in got.items():
            which, k = name.split(".")
            b = (iov if which == "v" else ioa)[k].cpu().numpy()
            assert_bitexact(a, b, f"replay {rep}: {name}")
    del graph
    for b in blocks:
        b.free()
