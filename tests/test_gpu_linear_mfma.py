"""The MFMA weight-only linear: every mx_linear call the int4 decode kernels
do not take (more than 16 rows of x, int8d weights at any row count), and the
[out, in]-weight product of mx_dynamic_linear and of the input gradients at
more than 16 rows.

mx_linear.forward (mxtorch.py:7454-7473) is y = x.float() @ dequant(W) with
W stored as quantize(weight.t()); mx_dynamic_linear.forward
(mxtorch.py:8945-8962) is x.float() @ dequant(W).t() + bias.  The kernel
runs both on f16 MFMAs with x * scale carried as an f16 hi + lo pair and the
codes as exact f16 operands; every output row must be within 1e-3 of that
row's largest |y| of the oracle (the reference's CPU path restated:
quantize, dequantize, fp32 product), for activations and weights from 1e-6
to 1e6, rows of very different magnitudes in one call, ragged K and
M in {17, 64, 512, 8192} at K = N = 8192.  int2d, float4d and float8d
weights run on the same kernel with their codes decoded to exact f16 values
(FP4 / FP8 grid values times 6 / 480, the factor taken back out of the
outputs); an all-codes test pins every decoded code."""
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

pytestmark = pytest.mark.gpu

RTOL = 1e-3
FMTS = ["int4d", "int8d", "int2d", "int1d", "float4d", "float8d"]


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


def _rowwise(y, y_ref):
    err = (y - y_ref).abs().amax(dim=1)
    lim = RTOL * y_ref.abs().amax(dim=1)
    return bool((err <= lim).all()), (err / lim.clamp_min(1e-300)).max().item()


def _module(qa, W, dt):
    N, K = W.shape
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    return qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype(dt), 128)


def _check_linear(qa, x, W, dt, rows=None):
    """mx_linear(x) against the oracle, on `rows` of x (all when None)."""
    N, K = W.shape
    m = _module(qa, W, dt)
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    assert G.bits_equal(m._mx_weight._mx_packed.cpu(), wp)
    assert G.bits_equal(m._mx_weight._mx_scales.cpu(), ws)
    y = m(x.to(dev())).cpu()
    xs = x if rows is None else x[rows]
    ys = y if rows is None else y[rows]
    y_ref = orc.linear_forward(xs, wp, ws, dt, K, N, 128)
    ok, worst = _rowwise(ys, y_ref)
    assert ok, f"{dt} M={x.shape[0]} K={K} N={N}: worst row error {worst:.3g} x the bar"
    return y


@pytest.fixture(scope="module")
def big_weights():
    """W [8192, 8192] ~ 0.02 N(0,1) with 0.1% outliers at 20x (the
    benchmark weight), its packed int4d and int8d forms from the oracle."""
    W = _randn((8192, 8192), 3, outliers=1e-3, scale=20.0) * 0.02
    return W


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("M", [17, 64, 512, 8192])
def test_mfma_linear_8192(qa, big_weights, dt, M):
    """x [M, 8192] in float32 and bfloat16 against W [8192, 8192]; at
    M = 8192 the oracle checks 96 sampled rows (each row's product is
    independent of the others).  int2d / float4d / float8d at M = 17 and 512."""
    if dt not in ("int4d", "int8d") and M in (64, 8192):
        pytest.skip("the other formats share the kernel; two sizes bound the test time")
    W = big_weights
    K = N = 8192
    m = _module(qa, W, dt)
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    assert G.bits_equal(m._mx_weight._mx_scales.cpu(), ws)
    for xdt in (torch.float32, torch.bfloat16):
        print(f"mfma linear {dt} M={M} x {xdt}", flush=True)
        x = _randn((M, K), 2 + M).to(xdt)
        y = m(x.to(dev())).cpu()
        if M > 512:
            g = torch.Generator()
            g.manual_seed(M)
            rows = torch.randperm(M, generator=g)[:96]
            rows[0], rows[1] = 0, M - 1
        else:
            rows = torch.arange(M)
        y_ref = orc.linear_forward(x[rows], wp, ws, dt, K, N, 128)
        ok, worst = _rowwise(y[rows], y_ref)
        assert ok, f"{dt} M={M} {xdt}: worst row error {worst:.3g} x the bar"


MAGS = [1e-6, 1e-3, 1.0, 1e4, 1e6]


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("wmag", MAGS)
@pytest.mark.parametrize("xmag", MAGS)
def test_mfma_magnitudes(qa, dt, xmag, wmag):
    M, K, N = 64, 2048, 512
    print(f"mfma magnitudes {dt} x~{xmag:g} W~{wmag:g}", flush=True)
    W = _randn((N, K), 101, outliers=1e-3) * wmag
    x = _randn((M, K), 103) * xmag
    _check_linear(qa, x, W, dt)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dt", FMTS)
def test_mfma_mixed_row_magnitudes(qa, dt, xdt):
    """Rows from 1e-4 to 1e3 (1e-7 to 1e7 for float32 and bfloat16) in one
    call, and a row of zeros, which must give exact zeros."""
    M, K, N = 40, 4096, 1024
    W = _randn((N, K), 107, outliers=1e-3) * 0.02
    lo, hi = (-4, 3) if xdt == torch.float16 else (-7, 7)
    mags = torch.logspace(lo, hi, M - 1)
    x = _randn((M, K), 109)
    x[: M - 1] *= mags[:, None]
    x[M - 1] = 0.0
    x = x.to(xdt)
    print(f"mfma mixed rows {dt} {xdt}", flush=True)
    m = _module(qa, W, dt)
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    y = m(x.to(dev())).cpu()
    y_ref = orc.linear_forward(x, wp, ws, dt, K, N, 128)
    assert torch.equal(y[M - 1], torch.zeros(N))
    ok, worst = _rowwise(y[: M - 1], y_ref[: M - 1])
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", FMTS)
def test_mfma_mixed_k_magnitudes(qa, dt):
    """Magnitudes that change along K inside one row: x large where the
    weights are small and the other way round."""
    M, K, N = 48, 2048, 256
    W = _randn((N, K), 113) * 0.02
    W[:, ::2] *= 1e-5
    x = _randn((M, K), 117)
    x[:, ::2] *= 1e5
    print(f"mfma mixed K {dt}", flush=True)
    _check_linear(qa, x, W, dt)


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("M,K,N", [(16, 1024, 256), (33, 100, 128), (200, 300, 384), (130, 1000, 640),
                                   (300, 2304, 1152), (1, 4096, 128)])
def test_mfma_ragged_shapes(qa, dt, M, K, N):
    """K not a multiple of the 256-row stage, odd M, single column blocks,
    and every format but int4d at M <= 16."""
    if dt == "int4d" and M <= 16:
        pytest.skip("int4d at M <= 16 takes the decode kernels")
    print(f"mfma ragged {dt} M={M} K={K} N={N}", flush=True)
    W = _randn((N, K), 7 * M + K, outliers=1e-3) * 0.05
    x = _randn((M, K), 11 * M + N)
    _check_linear(qa, x, W, dt)


@pytest.mark.parametrize("dt", FMTS)
def test_mfma_bias(qa, dt):
    """apply_bias adds the dequantized stored bias after the product."""
    M, K, N = 80, 1024, 384
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(_randn((N, K), 5) * 0.03)
        lin.bias.copy_(_randn((N,), 6))
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype(dt), 128)
    m.apply_bias = True
    x = _randn((M, K), 8)
    y = m(x.to(dev())).cpu()
    wp, ws, _ = orc.linear_from_weight(lin.weight.detach().cpu(), dt, 128)
    pb, sb, nb = orc.quantize(lin.bias.detach().cpu(), dt, 128)
    b = orc.dequant(pb, sb, dt, nb, 128)
    y_ref = orc.linear_forward(x, wp, ws, dt, K, N, 128) + b
    ok, worst = _rowwise(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("M,K,N", [(17, 8192, 8192), (64, 8192, 8192), (512, 8192, 8192), (40, 384, 256),
                                   (300, 1280, 640)])
def test_mfma_linear_nt(qa, dt, M, K, N):
    """[out, in] weights (mx_dynamic_linear.forward, mxtorch.py:8945-8962):
    x.float() @ dequant(W).t() + bias through ops.linear_wq_nt."""
    from qtpytorch_amd import ops
    if dt not in ("int4d", "int8d") and M == 64:
        pytest.skip("the other formats share the kernel; 17 and 512 rows bound the test time")
    print(f"mfma linear_nt {dt} M={M} K={K} N={N}", flush=True)
    W = _randn((N, K), 31 + M, outliers=1e-3) * 0.02
    x = _randn((M, K), 37 + N)
    bias = _randn((N,), 41)
    wp, ws, _ = orc.dynamic_linear_from_weight(W, dt, 128)
    y = ops.linear_wq_nt(x.to(dev()), wp.to(dev()), ws.to(dev()), dt, N, K, 128, bias=bias.to(dev())).cpu()
    y_ref = orc.dynamic_linear_forward(x, wp, ws, dt, K, N, 128, bias=bias)
    ok, worst = _rowwise(y - bias, y_ref - bias)
    assert ok, f"worst row error {worst:.3g} x the bar"
    # the K-block-major scales give the same result
    sT = ops.prepack_scales(ws.to(dev()), N, K, 128) if dt == "int4d" else None
    if sT is not None:
        y2 = ops.linear_wq_nt(x.to(dev()), wp.to(dev()), ws.to(dev()), dt, N, K, 128, bias=bias.to(dev()),
                              w_scales_t=sT).cpu()
        assert torch.equal(y2, y)


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("xmag,wmag", [(1e-6, 1e6), (1e6, 1e-6), (1e-3, 1e-3), (1e4, 1e4)])
def test_mfma_linear_nt_magnitudes(qa, dt, xmag, wmag):
    from qtpytorch_amd import ops
    M, K, N = 48, 1024, 256
    print(f"mfma linear_nt magnitudes {dt} x~{xmag:g} W~{wmag:g}", flush=True)
    W = _randn((N, K), 43, outliers=1e-3) * wmag
    x = _randn((M, K), 47) * xmag
    wp, ws, _ = orc.dynamic_linear_from_weight(W, dt, 128)
    y = ops.linear_wq_nt(x.to(dev()), wp.to(dev()), ws.to(dev()), dt, N, K, 128).cpu()
    y_ref = orc.dynamic_linear_forward(x, wp, ws, dt, K, N, 128)
    ok, worst = _rowwise(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


@pytest.mark.parametrize("dt", FMTS)
def test_mfma_input_gradient(qa, dt):
    """mx_linear's input gradient at batch 96: grad @ dequant(W)^T
    (F.linear(x, W_dq) of mxtorch.py:7473 differentiated), against float64."""
    M, K, N = 96, 1024, 768
    W = _randn((N, K), 51, outliers=1e-3) * 0.02
    m = _module(qa, W, dt)
    x = _randn((M, K), 53).to(dev()).requires_grad_(True)
    g = _randn((M, N), 57)
    y = m(x)
    y.backward(g.to(dev()))
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    w_dq = orc.dequant(wp, ws, dt, K * N, 128).reshape(K, N).double()
    gi_ref = (g.double() @ w_dq.t()).float()
    ok, worst = _rowwise(x.grad.cpu(), gi_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_mfma_dynamic_linear_batch(qa):
    """mx_dynamic_linear at 64 tokens (more than the decode kernels take)."""
    K, N = 2048, 1024
    lin = torch.nn.Linear(K, N)
    with torch.no_grad():
        lin.weight.copy_(_randn((N, K), 61) * 0.02)
        lin.bias.copy_(_randn((N,), 62) * 0.1)
    b = lin.bias.detach().clone()
    m = qa.mx_dynamic_linear.from_linear(lin.to(dev()), "int8d", "int8d")
    x = _randn((4, 16, K), 63)
    y = m(x.to(dev())).cpu()
    wp, ws, _ = orc.dynamic_linear_from_weight(lin.weight.detach().cpu(), "int8d", 128)
    y_ref = orc.dynamic_linear_forward(x, wp, ws, "int8d", K, N, 128, bias=b)
    ok, worst = _rowwise((y - b).reshape(-1, N), (y_ref - b).reshape(-1, N))
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_mfma_repeat_bitwise(qa):
    """Deterministic: two calls give the same bits (fixed reduction orders),
    also at a shape that splits K across workgroups."""
    for M in (20, 700):
        W = _randn((1024, 4096), 71) * 0.02
        m = _module(qa, W, "int4d")
        x = _randn((M, 4096), 73).to(dev())
        assert torch.equal(m(x), m(x))


@pytest.mark.parametrize("dt", ["int1d", "int2d", "int4d", "int8d", "float4d", "float8d"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_mfma_every_code(qa, dt, layout):
    """Every code of the format in every column and k position: codes
    (k + 3 n) mod 2^bits, scales 2^-6 .. 2^6 around a power of two from
    2^-20 to 2^20 that changes between column blocks (the [K][N] kernel
    keeps a block's terms relative to its largest scale), x the identity
    (M = K = 384 rows, more than the decode kernels take), so that y is the
    dequantized weight itself, one product term per output.  Each output may
    differ from the oracle's RN(grid[c] * s) only by the hi + lo split of
    s (2^-22) and, for the float grids, the factor RN(1/6) or RN(1/480):
    a code decoded to any other grid value fails by far more."""
    from qtpytorch_amd import ops
    bits = {"int1d": 1, "int2d": 2, "int4d": 4, "int8d": 8, "float4d": 4, "float8d": 8}[dt]
    K, N = 384, 256
    k = torch.arange(K)[:, None]
    n = torch.arange(N)[None, :]
    codes = (k + 3 * n) % (1 << bits)
    if dt.startswith("int"):
        codes = codes - (1 << (bits - 1))  # signed codes, every one of them
    g = torch.Generator()
    g.manual_seed(bits)
    x = torch.eye(K)
    nsc = K * N // 128
    off = torch.tensor([-20.0, 20.0, 0.0, 7.0])
    if layout == "kn":
        # block (k, nb) at k * N/128 + nb
        scales = torch.exp2(torch.empty(nsc).uniform_(-6, 6, generator=g) + off[torch.arange(nsc) % (N // 128)])
        packed = orc.pack(codes.reshape(-1), bits)
        y = ops.linear_wq(x.to(dev()), packed.to(dev()), scales.to(dev()), dt, K, N, 128).cpu()
        ref = orc.dequant(packed, scales, dt, K * N, 128).reshape(K, N)
    else:
        codes_nk = codes.t().contiguous()  # [N][K]: blocks along K, block (n, kb) at n * K/128 + kb
        scales = torch.exp2(torch.empty(nsc).uniform_(-6, 6, generator=g) + off[torch.arange(nsc) % 4])
        packed = orc.pack(codes_nk.reshape(-1), bits)
        y = ops.linear_wq_nt(x.to(dev()), packed.to(dev()), scales.to(dev()), dt, N, K, 128).cpu()
        ref = orc.dequant(packed, scales, dt, K * N, 128).reshape(N, K).t()
    print(f"mfma every code {dt} {layout}", flush=True)
    assert torch.isfinite(y).all()
    err = (y - ref).abs()
    lim = 2.0 ** -20 * ref.abs()
    bad = err > lim
    assert not bad.any(), (f"{int(bad.sum())} outputs off, first at {bad.nonzero()[0].tolist()}: "
                           f"{y[bad][0].item()!r} vs {ref[bad][0].item()!r}")


@pytest.mark.parametrize("dt", ["int4dh", "int8dh", "float4dh", "int8dv"])
def test_mx_linear_rotated_and_vector_weights(qa, dt):
    """'h' and 'v' weights, which no kernel decodes in registers: the
    reference's own dequantize-then-F.linear (mxtorch.py:7470-7473).  The
    dequantize undoes the rotation as ops.HADAMARD_DEQUANT_MODE says: the
    rows quantize rotated (the default), or the reference's whole-tensor
    unrotation (mxtorch.py:1582-1595)."""
    from qtpytorch_amd import ops
    M, K, N = 24, 512, 256
    W = _randn((N, K), 131, outliers=1e-3) * 0.05
    x = _randn((M, K), 137)
    m = _module(qa, W, dt)
    wp, ws, _ = orc.linear_from_weight(W, dt, 128)
    assert G.bits_equal(m._mx_weight._mx_packed.cpu(), wp)
    assert G.bits_equal(m._mx_weight._mx_scales.cpu(), ws)
    for mode in ("rows", "reference"):
        print(f"mx_linear {dt} unrotation {mode}", flush=True)
        old = ops.HADAMARD_DEQUANT_MODE
        ops.HADAMARD_DEQUANT_MODE = mode
        try:
            y = m(x.to(dev())).cpu()
        finally:
            ops.HADAMARD_DEQUANT_MODE = old
        w_f = orc.dequant(wp, ws, dt, K * N, 128, orig_shape=(K, N), hadamard_mode=mode).reshape(K, N)
        ok, worst = _rowwise(y, x @ w_f)
        assert ok, f"{dt} ({mode}): worst row error {worst:.3g} x the bar"
