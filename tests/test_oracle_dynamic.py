"""CPU pins of the oracle's dynamic-activation and int8 x int8 linear
restatements (mxtorch.py:2665-2731, 3910-3960, 8870-8968, 6693-6752).

What pins each function:
  * dynamic_quantize per_token: equal, bit for bit, to the golden-pinned
    'v' quantizer (quant_vector, checked against the reference's own
    vectors in test_oracle_golden.py) with block = row length, for int
    dtypes (there max_val = max_int); per_tensor equals per_token of the
    flattened tensor as one row; per_channel equals per_token of the
    transpose, transposed back; float dtypes use max_int of the width, not
    the format maximum (the reference's formula, mxtorch.py:2705);
  * fused_int8_linear: brute force in float64 over the dequantized codes
    on tiny shapes, with a non-square weight so a transposed operand fails;
  * dynamic_linear_forward: brute force in float64, [out, in] weight layout;
  * mx_linear_autograd_backward: torch autograd of the float product;
    mx_linear_autograd_forward: the composition of golden-pinned quantize,
    dispatch_qgemm and dequant.
"""
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G


def _x(shape, seed=0, dtype=torch.float32):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d", "int16d"])
@pytest.mark.parametrize("shape", [(4, 64), (3, 5, 100), (1, 7)])
def test_per_token_equals_vector_rule(name, shape):
    x = _x(shape, 1) * 3
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, "per_token")
    vp, vs, vn = orc.quant_vector(x, name + "v", shape[-1])
    assert sh == tuple(shape) and n == x.numel() and blk == shape[-1]
    assert G.bits_equal(p, vp)
    assert G.bits_equal(s, vs)


@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d"])
def test_per_tensor_is_one_row(name):
    x = _x((6, 50), 2)
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, "per_tensor")
    tp, ts, _, _, _ = orc.dynamic_quantize(x.reshape(1, -1), name, "per_token")
    assert G.bits_equal(p, tp) and G.bits_equal(s, ts)
    assert s.shape == (1,) and blk == x.numel() and sh == (6, 50)


@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d"])
@pytest.mark.parametrize("shape", [(8, 12), (5, 3, 4)])
def test_per_channel_is_token_of_transpose(name, shape):
    x = _x(shape, 3)
    bits = orc.parse_dtype(name)[1]
    p, s, sh, n, blk = orc.dynamic_quantize(x, name, "per_channel")
    x2 = x.reshape(shape[0], -1)
    tp, ts, _, _, _ = orc.dynamic_quantize(x2.t().contiguous(), name, "per_token")
    codes = orc.unpack_auto(p, bits, n).reshape(x2.shape)
    tcodes = orc.unpack_auto(tp, bits, n).reshape(x2.shape[1], x2.shape[0])
    assert torch.equal(codes, tcodes.t())
    assert G.bits_equal(s, ts)
    assert blk == shape[0]


def test_float_dtype_uses_width_max_int():
    x = _x((3, 16), 4)
    _, s, _, _, _ = orc.dynamic_quantize(x, "float8d", "per_token")
    a = x.abs().amax(dim=1)
    assert G.bits_equal(s, a / 127.0)   # not the E4M3 maximum


def test_per_block_is_quantize():
    x = _x((4, 100), 5)
    p, s, sh, n, blk = orc.dynamic_quantize(x, "int4d", "per_block", 64)
    qp, qs, qn = orc.quantize(x, "int4d", 64)
    assert G.bits_equal(p, qp) and G.bits_equal(s, qs) and n == qn and blk == 64


def _brute_linear(xd, wd, b):
    M, K = xd.shape
    N = wd.shape[0]
    out = torch.zeros(M, N, dtype=torch.float64)
    for m in range(M):
        for n in range(N):
            out[m, n] = sum(float(xd[m, k]) * float(wd[n, k]) for k in range(K))
    if b is not None:
        out += b.double()
    return out


@pytest.mark.parametrize("xg", ["per_token", "per_block"])
def test_fused_int8_linear_brute_force(xg):
    x, w, b = _x((3, 64), 6), _x((5, 64), 7), _x((5,), 8)
    xp, xs, xsh, xn, xb = orc.dynamic_quantize(x, "int8d", xg, 32)
    wp, ws, wn = orc.quantize(w, "int4d", 32)
    out = orc.fused_int8_linear(xp, xs, "int8d", xsh, xn, xb, wp, ws, "int4d", w.shape, wn, 32, b)
    xd = orc.dequant(xp, xs, "int8d", xn, xb).reshape(3, 64)
    wd = orc.dequant(wp, ws, "int4d", wn, 32).reshape(5, 64)
    ref = _brute_linear(xd, wd, b)
    assert out.shape == (3, 5)
    assert (out.double() - ref).abs().max() <= 1e-5 * ref.abs().max()


def test_dynamic_linear_forward_brute_force():
    w, b = _x((6, 32), 9) * 0.1, _x((6,), 10)
    x = _x((2, 3, 32), 11)
    wp, ws, wn = orc.dynamic_linear_from_weight(w, "int4d", 32)
    out = orc.dynamic_linear_forward(x, wp, ws, "int4d", 32, 6, 32, b)
    wd = orc.dequant(wp, ws, "int4d", wn, 32).reshape(6, 32)
    ref = _brute_linear(x.reshape(-1, 32), wd, b).reshape(2, 3, 6)
    assert out.shape == (2, 3, 6)
    assert (out.double() - ref).abs().max() <= 1e-5 * ref.abs().max()


def test_mx_linear_autograd_backward_is_autograd_of_product():
    K, N = 40, 24
    w = _x((N, K), 12) * 0.1
    wp, ws, wn = orc.linear_from_weight(w, "int8d", 16)        # [in, out] storage
    wd = orc.dequant(wp, ws, "int8d", wn, 16).reshape(K, N)
    x = _x((2, 5, K), 13).requires_grad_(True)
    y = x @ wd
    g = _x(tuple(y.shape), 14)
    y.backward(g)
    gi = orc.mx_linear_autograd_backward(g, wp, ws, "int8d", K, N, 16, x.shape)
    assert gi.shape == x.shape
    assert (gi - x.grad).abs().max() <= 1e-6 * x.grad.abs().max()


def test_mx_linear_autograd_forward_composition():
    K, N = 64, 32
    # every 32-element block of the stored [K, N] weight has absmax 1, so all
    # weight scales are equal and the GEMM's reading of B's flat scales as
    # [K/32, N] (mxtorch.py:1352-1355) gives the true scale of each element
    w = _x((N, K), 15).clamp(-0.9, 0.9)
    w[0::32, :] = 1.0
    wp, ws, wn = orc.linear_from_weight(w, "int8d", 32)
    bp, bs, bn = orc.quantize(_x((N,), 16), "int8d", 32)
    x = _x((2, 3, K), 17)
    out = orc.mx_linear_autograd_forward(x, wp, ws, "int8d", "int8d", K, N, 32, bp, bs)
    xp, xs, xn = orc.quantize(x.reshape(-1, K), "int8d", 32)
    pc, sc, name = orc.dispatch_qgemm(xp, xs, "int8d", (6, K), xn, wp, ws, "int8d", (K, N), K * N, 32)
    assert name == "int16d"
    ref = orc.dequant(pc, sc, name, 6 * N, 32).reshape(2, 3, N) + orc.dequant(bp, bs, "int8d", N, 32)
    assert G.bits_equal(out, ref)
    assert torch.unique(ws).numel() == 1
    # and it approximates the float product (int16 requantization, int8 operands)
    fl = x @ orc.dequant(wp, ws, "int8d", wn, 32).reshape(K, N) + orc.dequant(bp, bs, "int8d", N, 32)
    assert (out - fl).abs().max() <= 0.02 * fl.abs().max()
