"""mx_linear's decode paths (at most 16 rows of x; int4, int8, int2, FP4 and
FP8 codes) at any input magnitude (mx_linear.forward, mxtorch.py:7454-7473:
y = x.float() @ dequant(quantize(W.t()))).

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


def _run(qa, x, W, K, N, dt="int4d"):
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype(dt), 128)
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    assert G.bits_equal(m._mx_weight._mx_packed.cpu(), wp)
    assert G.bits_equal(m._mx_weight._mx_scales.cpu(), ws)
    y = m(x.to(dev())).cpu()
    y_ref = orc.linear_forward(x, wp, ws, dt, K, N, 128)
    return y, y_ref


MAGS = [1e-6, 1e-3, 1.0, 1e4, 1e6]
DTS = ["int4d", "int8d", "int2d", "int1d", "float4d", "float8d"]


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("wmag", MAGS)
@pytest.mark.parametrize("xmag", MAGS)
def test_decode_magnitudes(qa, xmag, wmag, dt):
    M, K, N = 16, 2048, 512
    print(f"decode magnitudes {dt} x~{xmag:g} W~{wmag:g}", flush=True)
    W = _randn((N, K), 101, outliers=1e-3) * wmag
    x = _randn((M, K), 103) * xmag
    y, y_ref = _run(qa, x, W, K, N, dt)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_mixed_row_magnitudes(qa, xdt, dt):
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
    y, y_ref = _run(qa, x, W, K, N, dt)
    assert torch.equal(y[M - 1], torch.zeros(N))
    ok, worst = _rowwise_ok(y[: M - 1], y_ref[: M - 1])
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", DTS)
def test_decode_mixed_k_magnitudes(qa, dt):
    """Magnitudes that change along K inside one row group of the kernel: x
    large where the weights are small and the other way round."""
    M, K, N = 8, 2048, 256
    W = _randn((N, K), 113) * 0.02
    W[:, ::2] *= 1e-5
    x = _randn((M, K), 117)
    x[:, ::2] *= 1e5
    y, y_ref = _run(qa, x, W, K, N, dt)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_config2_outliers(qa, xdt, dt):
    """The benchmark configuration at full size: x [16, 8192] (float32 and
    its bfloat16 copy), W [8192, 8192] ~ 0.02*N(0,1) with 0.1% of the
    weights at 20x (int8d: the same layer with int8 codes)."""
    M = K = N = 8192
    M = 16
    W = _randn((N, K), 3, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 2).to(xdt)
    y, y_ref = _run(qa, x, W, K, N, dt)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("M,K,N", [(1, 8192, 8192), (5, 4096, 1024), (16, 96, 128), (9, 2080, 384), (16, 16384, 256),
                                   (3, 32, 128)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_int8_shapes(qa, M, K, N, xdt):
    """int8 codes through the decode kernel called directly (ops.linear_wq),
    with the scales as stored (the kernel's own transposed copy in the
    workspace) and block-major (prepack_scales): one to sixteen rows, K a
    multiple of 32 down to one step, single and many column blocks, one
    split and many; both results within the bar of the oracle and equal."""
    from qtpytorch_amd import ops
    print(f"int8 decode M={M} K={K} N={N} {xdt}", flush=True)
    W = _randn((N, K), 7 * K + N, outliers=1e-3) * 0.05
    x = _randn((M, K), 11 * M + K).to(xdt)
    wp, ws, _ = orc.linear_from_weight(W, "int8d", 128)
    y = ops.linear_wq(x.to(dev()), wp.to(dev()), ws.to(dev()), "int8d", K, N, 128).cpu()
    sT = ops.prepack_scales(ws.to(dev()), K, N, 128)
    y2 = ops.linear_wq(x.to(dev()), wp.to(dev()), ws.to(dev()), "int8d", K, N, 128, w_scales_t=sT).cpu()
    y_ref = orc.linear_forward(x, wp, ws, "int8d", K, N, 128)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"
    assert torch.equal(y, y2)


@pytest.mark.parametrize("dt", ["int4d", "int8d", "int2d", "int1d", "float4d", "float8d"])
def test_decode_every_code(qa, dt):
    """Every code of the format in every column and k position through the
    decode kernel: x is 16 rows of the identity at a time, so each output is
    one dequantized weight.  Codes (k + 3 n) mod 2^bits, scales 2^-6 .. 2^6
    around a power of two from 2^-20 to 2^20 that changes between column
    blocks.  Each output may differ from the oracle's RN(grid[c] * s) only
    by the hi + lo split of s (2^-22) and, for the float grids, the factor
    RN(1/6) or RN(1/480)."""
    from qtpytorch_amd import ops
    bits = {"int4d": 4, "int8d": 8, "int2d": 2, "int1d": 1, "float4d": 4, "float8d": 8}[dt]
    K, N = 384, 256
    k = torch.arange(K)[:, None]
    n = torch.arange(N)[None, :]
    codes = (k + 3 * n) % (1 << bits)
    if dt.startswith("int"):
        codes = codes - (1 << (bits - 1))
    g = torch.Generator()
    g.manual_seed(bits + 1)
    nsc = K * N // 128
    off = torch.tensor([-20.0, 20.0])
    scales = torch.exp2(torch.empty(nsc).uniform_(-6, 6, generator=g) + off[torch.arange(nsc) % (N // 128)])
    packed = orc.pack(codes.reshape(-1), bits)
    ref = orc.dequant(packed, scales, dt, K * N, 128).reshape(K, N)
    pk, sc = packed.to(dev()), scales.to(dev())
    eye = torch.eye(K)
    for r0 in range(0, K, 16):
        y = ops.linear_wq(eye[r0:r0 + 16].to(dev()), pk, sc, dt, K, N, 128).cpu()
        want = ref[r0:r0 + 16]
        bad = (y - want).abs() > 2.0 ** -20 * want.abs()
        assert not bad.any(), (f"{dt} rows {r0}..{r0 + 15}: {int(bad.sum())} outputs off, first "
                               f"{y[bad][0].item()!r} vs {want[bad][0].item()!r}")
