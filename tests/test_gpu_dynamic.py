"""GPU parity of dynamic activations and the int8 x int8 / transposed-weight
linears (mxtorch.py:2665-2731, 3910-3960, 8870-8968, 6693-6752) against the
CPU oracle on the same seeded inputs.

Bar:
  * dynamic_quantize codes and scales, and _MXLinearAutograd's forward
    (quantize -> packed GEMM -> dequantize -> + bias): bitwise equal;
  * float outputs of fused_int8_linear, mx_dynamic_linear and the input
    gradients (an fp32 sgemm in the reference, summation order
    library-defined): max|y - y_ref| <= 1e-3 * max|y_ref|.
"""
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


def _x(shape, seed=0, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _close(y, ref, rtol=RTOL):
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, (y.shape, ref.shape)
    err = (y - ref).abs().max().item()
    assert err <= rtol * max(ref.abs().max().item(), 1e-30), f"max err {err}, max|ref| {ref.abs().max().item()}"


# ---------------------------------------------------------------- dynamic_quantize
@pytest.mark.parametrize("gran", ["per_token", "per_channel", "per_tensor"])
@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d", "float8d"])
@pytest.mark.parametrize("shape", [(16, 4096), (5, 3, 100), (7, 130), (1, 7), (300, 64)])
@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
def test_dynamic_quantize_matches_oracle(qa, gran, name, shape, src):
    x = _x(shape, 1, 2.0)
    x[..., 0] *= 30.0
    x = {"f32": x, "f16": x.half(), "bf16": x.bfloat16()}[src]
    q = qa.dynamic_quantize(x.to(dev()), name, gran)
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, gran)
    assert tuple(q.shape) == sh and q._mx_n == n and q._mx_block == blk
    assert q._mx_dtype.name == name
    assert G.bits_equal(q._mx_packed.cpu(), p), "packed codes differ"
    assert G.bits_equal(q._mx_scales.cpu(), s), "scales differ"


@pytest.mark.parametrize("gran", ["per_channel", "per_tensor"])
@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d"])
@pytest.mark.parametrize("shape", [(64, 3072), (33, 5120), (8, 1024, 2), (2048, 1024)])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_dynamic_quantize_vector_paths(qa, gran, name, shape, src):
    """The vectorised kernels (16-byte loads, per channel when a row is a
    multiple of 1024 columns, with the fixed-column grid for 3, 5 and 1 x
    1024 columns and several grid steps): codes and scales bit for bit,
    with values below 2^-96 and columns of zeros mixed in (the exact-divide
    branch of the encode)."""
    x = _x(shape, 5, 3.0)
    flat = x.view(-1)
    flat[::97] *= 1e-33
    x.view(x.shape[0], -1)[:, 5] = 0.0
    x = {"f32": x, "bf16": x.bfloat16()}[src]
    q = qa.dynamic_quantize(x.to(dev()), name, gran)
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, gran)
    assert tuple(q.shape) == sh and q._mx_n == n and q._mx_block == blk
    assert G.bits_equal(q._mx_packed.cpu(), p), "packed codes differ"
    assert G.bits_equal(q._mx_scales.cpu(), s), "scales differ"


@pytest.mark.parametrize("name", ["int3d", "int16d"])
def test_dynamic_quantize_per_token_word_widths(qa, name):
    x = _x((9, 200), 2)
    q = qa.dynamic_quantize(x.to(dev()), name, "per_token")
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, "per_token")
    assert G.bits_equal(q._mx_packed.cpu(), p) and G.bits_equal(q._mx_scales.cpu(), s)


def test_dynamic_quantize_zeros_and_per_block(qa):
    x = torch.zeros(4, 64)
    q = qa.dynamic_quantize(x.to(dev()), "int8d", "per_token")
    p, s, _, _, _ = orc.dynamic_quantize(x, "int8d", "per_token")
    assert G.bits_equal(q._mx_packed.cpu(), p) and G.bits_equal(q._mx_scales.cpu(), s)
    y = _x((3, 100), 3)
    q = qa.dynamic_quantize(y.to(dev()), "int4d", "per_block", 64)
    p, s, n = orc.quantize(y, "int4d", 64)
    assert G.bits_equal(q._mx_packed.cpu(), p) and G.bits_equal(q._mx_scales.cpu(), s)


def test_dynamic_quantize_full_size_row_sample(qa):
    """Config-2-sized activations [4096, 8192]: every row's scale and a sample of rows' codes."""
    x = _x((4096, 8192), 4)
    q = qa.dynamic_quantize(x.to(dev()), "int8d", "per_token")
    s_ref = x.abs().amax(dim=1).clamp(min=1e-12) / 127.0
    assert G.bits_equal(q._mx_scales.cpu(), s_ref)
    codes = q._mx_packed.cpu().view(4096, 8192)
    for r in (0, 1, 777, 4095):
        p, s, _, _, _ = orc.dynamic_quantize(x[r:r + 1], "int8d", "per_token")
        assert torch.equal(codes[r], p)


# ---------------------------------------------------------------- fused_int8_linear
def _fused_ref(xq, wq, bias):
    return orc.fused_int8_linear(xq._mx_packed.cpu(), xq._mx_scales.cpu(), xq._mx_dtype.name, tuple(xq.shape),
                                 xq._mx_n, xq._mx_block, wq._mx_packed.cpu(), wq._mx_scales.cpu(),
                                 wq._mx_dtype.name, tuple(wq.shape), wq._mx_n, wq._mx_block,
                                 None if bias is None else bias.cpu())


@pytest.mark.parametrize("M,K,N", [(8, 64, 32), (1, 128, 64), (16, 1024, 200), (100, 512, 384), (300, 256, 130)])
@pytest.mark.parametrize("xg", ["per_token", "per_block"])
@pytest.mark.parametrize("wname", ["int8d", "int4d", "int2d"])
@pytest.mark.parametrize("has_bias", [False, True])
def test_fused_int8_linear_mfma_path(qa, M, K, N, xg, wname, has_bias):
    x, w = _x((M, K), 5), _x((N, K), 6, 0.05)
    b = _x((N,), 7) if has_bias else None
    xq = qa.dynamic_quantize(x.to(dev()), "int8d", xg, 64)
    wq = qa.mx_tensor.quantize(w.to(dev()), qa.get_mx_dtype(wname), 128)
    assert qa.ops.linear_i8_eligible(xq._mx_dtype, wq._mx_dtype, K, xq._mx_block, wq._mx_block)
    y = qa.fused_int8_linear(xq, wq, None if b is None else b.to(dev()))
    _close(y, _fused_ref(xq, wq, b))


def test_fused_int8_linear_large_v3(qa):
    """A prefill-sized product (256x128 tiles fill the chip: the 3-stage kernel)."""
    M, K, N = 2048, 4096, 4096
    x, w = _x((M, K), 8), _x((N, K), 9, 0.02)
    xq = qa.dynamic_quantize(x.to(dev()), "int8d", "per_token")
    wq = qa.mx_tensor.quantize(w.to(dev()), qa.get_mx_dtype("int8d"), 128)
    b = _x((N,), 10)
    y = qa.fused_int8_linear(xq, wq, b.to(dev()))
    _close(y, _fused_ref(xq, wq, b))


@pytest.mark.parametrize("wname", ["float8d", "float4d", "int4dh", "int8d"])
def test_fused_int8_linear_other_paths(qa, wname):
    """Weights outside the MFMA path (float grids, 'h') and x blocks that straddle K chunks."""
    x, w = _x((12, 96), 11), _x((40, 96), 12, 0.1)
    xq = qa.mx_tensor.quantize(x.to(dev()), qa.get_mx_dtype("int8d"), 48)
    wq = qa.mx_tensor.quantize(w.to(dev()), qa.get_mx_dtype(wname), 32)
    b = _x((40,), 13)
    y = qa.fused_int8_linear(xq, wq, b.to(dev()))
    if wname == "int4dh":
        # 'h' weights dequantize through the inverse rotation of their rows
        w_f = wq.dequantize().cpu()
        ref = torch.nn.functional.linear(xq.dequantize().cpu(), w_f, b)
    else:
        ref = _fused_ref(xq, wq, b)
    _close(y, ref)


def test_fused_int8_linear_float_and_method(qa):
    x, w, b = _x((8, 64), 14), _x((128, 64), 15), _x((128,), 16)
    y = qa.fused_int8_linear(x.to(dev()), w.to(dev()), b.to(dev()))
    _close(y, torch.nn.functional.linear(x, w, b), 1e-4)
    xq = qa.mx_tensor.quantize(_x((4, 32), 17).to(dev()), qa.get_mx_dtype("int8d"))
    wq = qa.mx_tensor.quantize(_x((16, 32), 18).to(dev()), qa.get_mx_dtype("int8d"))
    y1 = xq.fused_int8_linear(wq)
    y2 = qa.mx_fused_ops.fused_int8_linear(xq, wq)
    assert y1.shape == (4, 16)
    assert torch.equal(y1, y2)
    _close(y1, _fused_ref(xq, wq, None))


# ---------------------------------------------------------------- mx_dynamic_linear
@pytest.mark.parametrize("wname", ["int4d", "int8d", "int2d", "float4d", "float8d"])
@pytest.mark.parametrize("shape", [(4, 64), (2, 3, 256), (16, 512)])
@pytest.mark.parametrize("has_bias", [False, True])
def test_mx_dynamic_linear_forward(qa, wname, shape, has_bias):
    K = shape[-1]
    lin = torch.nn.Linear(K, 96, bias=has_bias)
    with torch.no_grad():
        lin.weight.copy_(_x((96, K), 19, 0.05))
        if has_bias:
            lin.bias.copy_(_x((96,), 20))
    m = qa.mx_dynamic_linear.from_linear(lin.to(dev()), wname, "int8d")
    x = _x(shape, 21)
    y = m(x.to(dev()))
    wp, ws, _ = orc.dynamic_linear_from_weight(lin.weight.data.cpu(), wname, 128)
    assert G.bits_equal(m.weight._mx_packed.cpu(), wp) and G.bits_equal(m.weight._mx_scales.cpu(), ws)
    ref = orc.dynamic_linear_forward(x, wp, ws, wname, K, 96, 128, lin.bias.data.cpu() if has_bias else None)
    _close(y, ref)
    # the activation quantization the reference builds
    xq = m.quantize_activation(x.to(dev()))
    p, s, _, _, _ = orc.dynamic_quantize(x, "int8d", "per_token")
    assert G.bits_equal(xq._mx_packed.cpu(), p) and G.bits_equal(xq._mx_scales.cpu(), s)


def test_mx_dynamic_linear_decode_shape_and_grad(qa):
    K, N = 8192, 1024
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(_x((N, K), 22, 0.02))
        lin.bias.copy_(_x((N,), 23))
    m = qa.mx_dynamic_linear.from_linear(lin.to(dev()), "int4d", "int8d")
    x = _x((16, K), 24)
    xg = x.to(dev()).requires_grad_(True)
    y = m(xg)
    wp, ws, _ = orc.dynamic_linear_from_weight(lin.weight.data.cpu(), "int4d", 128)
    ref = orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128, lin.bias.data.cpu())
    _close(y, ref)
    g = _x((16, N), 25)
    y.backward(g.to(dev()))
    wd = orc.dequant(wp, ws, "int4d", N * K, 128).reshape(N, K)
    _close(xg.grad, g @ wd)


# ---------------------------------------------------------------- mx_linear gradients, _MXLinearAutograd
@pytest.mark.parametrize("wname", ["int4d", "int8d", "float4d"])
@pytest.mark.parametrize("shape", [(16, 512), (3, 5, 256)])
def test_mx_linear_input_gradient(qa, wname, shape):
    K, N = shape[-1], 384
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(_x((N, K), 26, 0.05))
    m = qa.mx_linear.from_linear(lin.to(dev()), wname, 128)
    x = _x(shape, 27)
    xg = x.to(dev()).requires_grad_(True)
    y = m(xg)
    wp, ws, _ = orc.linear_from_weight(lin.weight.data.cpu(), wname, 128)
    _close(y, orc.linear_forward(x, wp, ws, wname, K, N, 128))
    g = _x(tuple(y.shape), 28)
    y.backward(g.to(dev()))
    ref = orc.mx_linear_autograd_backward(g, wp, ws, wname, K, N, 128, x.shape)
    _close(xg.grad, ref)


@pytest.mark.parametrize("xname,wname", [("int8d", "int8d"), ("int4d", "int4d")])
@pytest.mark.parametrize("shape", [(16, 256), (2, 3, 128)])
@pytest.mark.parametrize("has_bias", [False, True])
def test_mx_linear_autograd_function(qa, xname, wname, shape, has_bias):
    K, N = shape[-1], 256
    w = _x((N, K), 29, 0.05)
    wp, ws, _ = orc.linear_from_weight(w, wname, 128)
    w_mx = qa.mx_tensor.quantize(w.t().contiguous().to(dev()), qa.get_mx_dtype(wname), 128)
    assert G.bits_equal(w_mx._mx_packed.cpu(), wp)
    bq = bp = bs = None
    if has_bias:
        bvec = _x((N,), 30)
        bq = qa.mx_tensor.quantize(bvec.to(dev()), qa.get_mx_dtype(wname), 128)
        bp, bs, _ = orc.quantize(bvec, wname, 128)
    x = _x(shape, 31)
    xg = x.to(dev()).requires_grad_(True)
    y = qa._mx_linear_forward(xg, w_mx, bq, qa.get_mx_dtype(xname), 128, K, N)
    ref = orc.mx_linear_autograd_forward(x, wp, ws, wname, xname, K, N, 128, bp, bs)
    assert G.bits_equal(y.detach().cpu(), ref), "forward differs from the oracle"
    g = _x(tuple(y.shape), 32)
    y.backward(g.to(dev()))
    _close(xg.grad, orc.mx_linear_autograd_backward(g, wp, ws, wname, K, N, 128, x.shape))


# ---------------------------------------------------------------- int4 decode with [N][K] weights
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("K,N", [(128, 16), (1024, 272), (1152, 1024), (8192, 4096)])
@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
def test_linear_wq_nt_decode_path(qa, M, K, N, src):
    w = _x((N, K), 33, 0.02)
    w[torch.rand(N, K, generator=torch.Generator().manual_seed(34)) < 1e-3] *= 20
    wp, ws, _ = orc.dynamic_linear_from_weight(w, "int4d", 128)
    x = _x((M, K), 35)
    x = {"f32": x, "f16": x.half(), "bf16": x.bfloat16()}[src]
    b = _x((N,), 36)
    y = qa.ops.linear_wq_nt(x.to(dev()), wp.to(dev()), ws.to(dev()), "int4d", N, K, 128, bias=b.to(dev()))
    _close(y, orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128, b))


@pytest.mark.parametrize("mag", [1e6, 1e-6])
def test_linear_wq_nt_decode_extreme_activations(qa, mag):
    """Activations past the f16 range (staged with a power-of-two rescale) and tiny ones."""
    K, N = 2048, 512
    w = _x((N, K), 37, 0.02)
    wp, ws, _ = orc.dynamic_linear_from_weight(w, "int4d", 128)
    x = _x((16, K), 38) * mag
    y = qa.ops.linear_wq_nt(x.to(dev()), wp.to(dev()), ws.to(dev()), "int4d", N, K, 128)
    _close(y, orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128))
