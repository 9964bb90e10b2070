"""HIP graph capture of the hot path (bench.py times graph replays).

Each op is called eagerly first (workspaces, prepacked scales and the KV
ring exist before capture), captured once, then replayed three times with
eager calls of the same op on other inputs in between.  Every replay must
equal the eager result bit for bit: the kernels are deterministic, and the
split-K decode kernels leave their arrival counters zero after each call,
so a replay sees the same state as an eager call.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qtpytorch_amd
    return qtpytorch_amd


def _x(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _capture(fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g, out


def _same(a, b):
    if isinstance(a, (tuple, list)):
        return all(_same(u, v) for u, v in zip(a, b))
    a, b = a.detach(), b.detach()
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


def _replays(fn, other):
    """fn(): the op on the captured inputs; other(): the op on other inputs."""
    ref = fn()
    ref = tuple(t.clone() for t in ref) if isinstance(ref, tuple) else ref.clone()
    other_ref = other()
    other_ref = tuple(t.clone() for t in other_ref) if isinstance(other_ref, tuple) else other_ref.clone()
    torch.cuda.synchronize()
    g, out = _capture(fn)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert _same(out, ref), f"replay {rep} differs from the eager result"
        o2 = other()
        torch.cuda.synchronize()
        assert _same(o2, other_ref), f"eager call after replay {rep} differs"
    del g


def test_graph_decode_linear(qa):
    dev = torch.device("cuda:0")
    lin = torch.nn.Linear(8192, 4096, bias=False)
    with torch.no_grad():
        lin.weight.copy_(_x((4096, 8192), 1, 0.02))
    m = qa.mx_linear.from_linear(lin.to(dev), qa.get_mx_dtype("int4d"), 128)
    x1, x2 = _x((16, 8192), 2).to(dev), _x((5, 8192), 3).to(dev)
    _replays(lambda: m(x1), lambda: m(x2))


def test_graph_transposed_decode_linear(qa):
    dev = torch.device("cuda:0")
    lin = torch.nn.Linear(8192, 2048, bias=True)
    with torch.no_grad():
        lin.weight.copy_(_x((2048, 8192), 4, 0.02))
        lin.bias.copy_(_x((2048,), 5))
    m = qa.mx_dynamic_linear.from_linear(lin.to(dev), "int4d", "int8d")
    x1, x2 = _x((16, 8192), 6).to(dev), _x((3, 8192), 7).to(dev)
    _replays(lambda: m(x1), lambda: m(x2))


@pytest.mark.parametrize("name", ["int4d", "int8d", "float8d", "int4dh"])
def test_graph_quantize_dequantize(qa, name):
    dev = torch.device("cuda:0")
    dt = qa.get_mx_dtype(name)
    x1, x2 = _x((512, 128), 8).to(dev), _x((64, 128), 9).to(dev)

    def qd(x):
        p, s, n = qa.ops.quantize(x, dt, 128, seed=1534857261 if dt.is_hadamard else None)
        d = qa.ops._dequant(p, s, dt, n, 128, orig_shape=tuple(x.shape),
                            seed=1534857261 if dt.is_hadamard else None)
        return p, s, d

    _replays(lambda: qd(x1), lambda: qd(x2))


def test_graph_gemm_and_kv_append(qa):
    dev = torch.device("cuda:0")
    d8 = qa.get_mx_dtype("int8d")
    A, B = _x((256, 512), 10).to(dev), _x((512, 384), 11).to(dev)
    qa_, qb = qa.mx_tensor.quantize(A, d8, 128), qa.mx_tensor.quantize(B, d8, 128)
    A2 = _x((128, 512), 12).to(dev)
    qa2 = qa.mx_tensor.quantize(A2, d8, 128)

    def mm(a):
        r = qa.ops.qscale_gemm(a._mx_packed, a._mx_scales, qb._mx_packed, qb._mx_scales, a.shape[0], 512, 384, 8,
                               128, 16, want_c=True)
        return r["packed"], r["scales"], r["c"]

    _replays(lambda: mm(qa_), lambda: mm(qa2))

    k1, v1 = _x((8, 32, 1, 128), 13).half().to(dev), _x((8, 32, 1, 128), 14).half().to(dev)
    k2, v2 = _x((8, 32, 1, 128), 15).half().to(dev), _x((8, 32, 1, 128), 16).half().to(dev)
    cache = qa.kv_cache_quantizer(n_heads=32, head_dim=128, dtype="int8dv", max_seq_len=8)
    for _ in range(8):
        cache.append_kv(k2, v2)

    def step(k, v):
        cache.append_kv(k, v)
        return tuple(t.clone() for t in cache.get())

    # the ring is full: every append evicts the oldest step, and the newest
    # step is the last one get() returns
    _replays(lambda: step(k1, v1)[0][:, :, -1:], lambda: step(k2, v2)[0][:, :, -1:])


def test_two_graphs_one_stream_second_replayed_first(qa):
    """Two decode-linear graphs captured one after the other on one new
    stream share its split-K workspace, which the first capture creates in
    graph memory.  Replaying the second graph first (and eager calls on that
    stream before any replay of the first) must still see zeroed arrival
    counters: every capture records the counter clear until an eager call
    has made it."""
    dev = torch.device("cuda:0")
    lin = torch.nn.Linear(8192, 2048, bias=False)
    with torch.no_grad():
        lin.weight.copy_(_x((2048, 8192), 21, 0.02))
    m = qa.mx_linear.from_linear(lin.to(dev), qa.get_mx_dtype("int4d"), 128)
    x1, x2 = _x((16, 8192), 22).to(dev), _x((8, 8192), 23).to(dev)
    ref1, ref2 = m(x1).clone(), m(x2).clone()   # eager, on the default stream
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g1, stream=s):
            o1 = m(x1)
        with torch.cuda.graph(g2, stream=s):
            o2 = m(x2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep in range(3):
        g2.replay()
        torch.cuda.synchronize()
        assert _same(o2, ref2), f"second graph, replay {rep}"
        with torch.cuda.stream(s):
            e2 = m(x2)   # eager on the capture stream
        torch.cuda.synchronize()
        assert _same(e2, ref2), f"eager call on the capture stream, round {rep}"
        g1.replay()
        torch.cuda.synchronize()
        assert _same(o1, ref1), f"first graph, replay {rep}"
    del g1, g2
