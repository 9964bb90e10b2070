"""mxk_linear_wq_noalloc: the decode linear (and the MFMA linear beyond 16
rows) with its workspace in the library's static device scratch (no
allocation by the call), against mxk_linear_wq with a caller-provided
workspace, bit for bit, on calls in a row with later ones smaller, for int4,
int8, FP4 and FP8 weights, and its refusal of shapes whose workspace
exceeds the scratch.  Called through the C ABI with ctypes."""
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qtpytorch_amd
    return qtpytorch_amd


def _randn(shape, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(*shape, generator=g)


def _noalloc(qa, x, wp, ws, st, K, N, dt=None):
    L = qa._lib
    dt = dt or qa.get_mx_dtype("int4d")
    kind = L.MXK_KIND_FLOAT if dt.is_float else L.MXK_KIND_INT
    out = torch.empty(x.shape[0], N, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = L.lib().mxk_linear_wq_noalloc(x.data_ptr(), L.elem_type(x.dtype), x.shape[0], K, wp.data_ptr(),
                                           ws.data_ptr(), L.ptr(st), N, kind, dt.bits, 128, 0,
                                           out.data_ptr(), L.stream_of(x))
    L.check(rc, "linear_wq_noalloc")
    return out


@pytest.mark.parametrize("name", ["int4d", "int8d", "int2d", "int1d", "float4d", "float8d"])
@pytest.mark.parametrize("prepacked", [True, False])
def test_noalloc_matches_workspace_entry(qa, prepacked, name):
    dev = torch.device("cuda:0")
    dt = qa.get_mx_dtype(name)
    # decode kernel at 16 and 5 rows (the second call smaller), then the
    # MFMA linear at 40 rows
    for (M, K, N, seed) in ((16, 8192, 8192, 5), (5, 4096, 2048, 7), (40, 2048, 1024, 9)):
        print(f"noalloc {name} M={M} K={K} N={N} prepacked={prepacked}", flush=True)
        W = _randn((N, K), seed) * 0.02
        wp, ws, _ = orc.linear_from_weight(W, name, 128)
        wpg, wsg = wp.to(dev), ws.to(dev)
        st = qa.ops.prepack_scales(wsg, K, N, 128) if prepacked else None
        x = _randn((M, K), seed + 1).to(dev)
        y_ref = qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st)
        y = _noalloc(qa, x, wpg, wsg, st, K, N, dt)
        y2 = _noalloc(qa, x, wpg, wsg, st, K, N, dt)
        torch.cuda.synchronize()
        assert G.bits_equal(y.cpu(), y_ref.cpu())
        assert G.bits_equal(y2.cpu(), y_ref.cpu())


def test_noalloc_refuses_oversized_workspace(qa):
    dev = torch.device("cuda:0")
    K, N = 8192, 16384   # 8 split partials of 128 blocks: 8 MiB + counters > the 8 MiB scratch
    x = torch.zeros(16, K, device=dev)
    wp = torch.zeros(K * N // 2, dtype=torch.int8, device=dev)
    ws = torch.ones(K * N // 128, dtype=torch.float32, device=dev)
    with pytest.raises(qa._lib.MXKError, match="static scratch"):
        _noalloc(qa, x, wp, ws, None, K, N)
