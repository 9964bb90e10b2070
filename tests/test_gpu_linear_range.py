"""mx_linear's int4 decode path at any input magnitude (mx_linear.forward,
mxtorch.py:7454-7473: y = x.float() @ dequant(quantize(W.t()))).

The decode kernel feeds x*s to f16 MFMAs as a hi + lo pair; these tests
check that its power-of-two range scaling keeps every output within 1e-3 of
the oracle, per output row, for activations and weights from 1e-6 to 1e6,
for rows of very different magnitudes in one call, and at the benchmark
configuration (x [16, 8192], W [8192, 8192] ~ N(0, 0.02) with 0.1% outliers
at 20x) in float32 and bfloat16.  The oracle is the reference's CPU path
restated (quantize W.t(), dequantize, fp32 F.linear)."""
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


def _rowwise_ok(y, y_ref):
    """max over each row of |y - y_ref| within RTOL of that row's max |y_ref|."""
    err = (y - y_ref).abs().amax(dim=1)
    lim = RTOL * y_ref.abs().amax(dim=1)
    return bool((err <= lim).all()), (err / lim.clamp_min(1e-300)).max().item()


def _run(qa, x, W, K, N):
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    wp, ws, _ = orc.linear_from_weight(W, "int4d", 128)
    assert G.bits_equal(m._mx_weight._mx_packed.cpu(), wp)
    assert G.bits_equal(m._mx_weight._mx_scales.cpu(), ws)
    y = m(x.to(dev())).cpu()
    y_ref = orc.linear_forward(x, wp, ws, "int4d", K, N, 128)
    return y, y_ref


MAGS = [1e-6, 1e-3, 1.0, 1e4, 1e6]


@pytest.mark.parametrize("wmag", MAGS)
@pytest.mark.parametrize("xmag", MAGS)
def test_decode_magnitudes(qa, xmag, wmag):
    M, K, N = 16, 2048, 512
    print(f"decode magnitudes x~{xmag:g} W~{wmag:g}", flush=True)
    W = _randn((N, K), 101, outliers=1e-3) * wmag
    x = _randn((M, K), 103) * xmag
    y, y_ref = _run(qa, x, W, K, N)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_mixed_row_magnitudes(qa, xdt):
    """Rows from 1e-4 to 1e3 (1e-7 to 1e7 for float32 and bfloat16) in one
    call, and a row of zeros: each row within the bar of its own magnitude."""
    M, K, N = 16, 4096, 1024
    W = _randn((N, K), 107, outliers=1e-3) * 0.02
    lo, hi = (-4, 3) if xdt == torch.float16 else (-7, 7)
    mags = torch.logspace(lo, hi, M - 1)
    x = _randn((M, K), 109)
    x[: M - 1] *= mags[:, None]
    x[M - 1] = 0.0
    x = x.to(xdt)
    y, y_ref = _run(qa, x, W, K, N)
    assert torch.equal(y[M - 1], torch.zeros(N))
    ok, worst = _rowwise_ok(y[: M - 1], y_ref[: M - 1])
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_decode_mixed_k_magnitudes(qa):
    """Magnitudes that change along K inside one row group of the kernel: x
    large where the weights are small and the other way round."""
    M, K, N = 8, 2048, 256
    W = _randn((N, K), 113) * 0.02
    W[:, ::2] *= 1e-5
    x = _randn((M, K), 117)
    x[:, ::2] *= 1e5
    y, y_ref = _run(qa, x, W, K, N)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_config2_outliers(qa, xdt):
    """The benchmark configuration at full size: x [16, 8192] (float32 and
    its bfloat16 copy), W [8192, 8192] ~ 0.02*N(0,1) with 0.1% of the
    weights at 20x."""
    M = K = N = 8192
    M = 16
    W = _randn((N, K), 3, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 2).to(xdt)
    y, y_ref = _run(qa, x, W, K, N)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"
