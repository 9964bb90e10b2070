"""The split-K workspaces of the int4 decode linear (mx_linear.forward,
mxtorch.py:7454-7473).

The decode kernel splits K over workgroups, which publish partial sums and
count their arrival in a caller-owned workspace; the last to arrive adds the
partials in split order and leaves the counters zero.  Workspaces are per
(device, stream): decode linears on two streams at once must not disturb
each other."""
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

pytestmark = pytest.mark.gpu

RTOL = 1e-3


@pytest.fixture(scope="module")
def qa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qtpytorch_amd
    return qtpytorch_amd


def dev():
    return torch.device("cuda:0")


def _randn(shape, seed, outliers=0.0, scale=20.0):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        m = torch.rand(*shape, generator=g) < outliers
        x[m] *= scale
    return x


def _weights(qa, K, N, seed):
    W = _randn((N, K), seed, outliers=1e-3) * 0.02
    wp, ws, _ = orc.linear_from_weight(W, "int4d", 128)
    wpg, wsg = wp.to(dev()), ws.to(dev())
    return wp, ws, wpg, wsg, qa.ops.prepack_scales(wsg, K, N, 128)


def test_two_streams_concurrently(qa):
    """Two decode linears of different shapes issued alternately on two
    streams, many times without synchronizing in between: every result
    equals the one computed alone, bit for bit."""
    dt = qa.get_mx_dtype("int4d")
    cases = []
    for (M, K, N, seed) in ((16, 8192, 4096, 81), (7, 4096, 8192, 83)):
        wp, ws, wpg, wsg, st = _weights(qa, K, N, seed)
        x = _randn((M, K), seed + 1).to(dev())
        alone = qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st)
        torch.cuda.synchronize()
        y_ref = orc.linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128)
        assert (alone.cpu() - y_ref).abs().max().item() <= RTOL * y_ref.abs().max().item()
        cases.append((x, wpg, wsg, st, K, N, alone))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(20):
        for i, s in enumerate(streams):
            x, wpg, wsg, st, K, N, _ = cases[i]
            with torch.cuda.stream(s):
                outs[i].append(qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st))
    torch.cuda.synchronize()
    for i in range(2):
        ref = cases[i][6].cpu()
        for k, y in enumerate(outs[i]):
            assert G.bits_equal(y.cpu(), ref), f"stream {i}, call {k} differs from the call alone"


def test_workspace_per_stream(qa):
    """Each stream gets its own split-K workspace, kept for later calls."""
    dt = qa.get_mx_dtype("int4d")
    _, _, wpg, wsg, st = _weights(qa, 4096, 1024, 91)
    x = _randn((4, 4096), 93).to(dev())
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        with torch.cuda.stream(s):
            qa.ops.linear_wq(x, wpg, wsg, dt, 4096, 1024, 128, w_scales_t=st)
    torch.cuda.synchronize()
    keys = {k for k in qa.ops._ZEROED_WS if k[0] == str(dev())}
    assert (str(dev()), s1.cuda_stream) in keys and (str(dev()), s2.cuda_stream) in keys
    assert qa.ops._ZEROED_WS[(str(dev()), s1.cuda_stream)].data_ptr() != \
        qa.ops._ZEROED_WS[(str(dev()), s2.cuda_stream)].data_ptr()
