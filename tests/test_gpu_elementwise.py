"""GPU parity of quantized element-wise arithmetic (qa + qb, qa - qb, qa * qb,
-qa; mxtorch.py:5321-5497, 1186-1296, 6177-6193) against the oracle
(oracle.dispatch_qelementwise / negate, pinned in
tests/test_oracle_elementwise.py): packed codes, scales and dtypes bitwise
equal."""
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


def dev():
    return torch.device("cuda:0")


def _bits_eq(a, b):
    return G.bits_equal(a.detach().cpu(), b.detach().cpu())


def _operands(shape, seed, block, a_name, b_name, mode):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if mode == "near":     # same block scales up to a few ulps: the integer path, with overflow
        y = x * 1.0000001 + 1e-3 * torch.randn(*shape, generator=g)
    elif mode == "far":    # scales 3-50x apart: the float path
        y = torch.randn(*shape, generator=g) * 40.0
    else:                  # mixed: both paths across blocks
        y = torch.randn(*shape, generator=g) * torch.rand(*shape, generator=g).pow(4) * 8.0
    pa, sa, n = orc.quantize(x, a_name, block)
    pb, sb, _ = orc.quantize(y, b_name, block)
    return (pa, sa), (pb, sb), n


def _mx(qa, p, s, name, shape, n, block):
    return qa.mx_tensor(p.to(dev()), s.to(dev()), qa.get_mx_dtype(name), torch.Size(shape), n, block)


CASES = [
    ("int8d", "int8d", 128, (16, 300), "near"),
    ("int8d", "int8d", 128, (16, 300), "far"),
    ("int8d", "int8d", 128, (16, 300), "mixed"),
    ("int4d", "int4d", 64, (7, 129), "mixed"),
    ("int4d", "int4d", 128, (3, 1000), "near"),
    ("int2d", "int2d", 32, (5, 77), "mixed"),
    ("int3d", "int3d", 128, (4, 333), "mixed"),
    ("int16d", "int16d", 256, (2, 700), "mixed"),
    ("float4d", "float4d", 128, (9, 200), "mixed"),
    ("float8d", "float8d", 96, (9, 200), "mixed"),
    ("int8dv", "int8dv", 128, (4, 512), "mixed"),
    ("int8d", "int4d", 128, (8, 256), "mixed"),       # b read with a's width
    ("int4d", "int8d", 128, (8, 256), "near"),
    ("int8d", "float4u", 128, (8, 256), "mixed"),     # output dtype float4u
    ("int5d", "int5d", 192, (3, 400), "far"),
    ("int7d", "int6d", 200, (3, 401), "mixed"),       # block not a multiple of 64: two-pass packing
]


@pytest.mark.parametrize("op", ["add", "sub", "mul"])
@pytest.mark.parametrize("a_name,b_name,block,shape,mode", CASES,
                         ids=[f"{c[0]}-{c[1]}-b{c[2]}-{c[4]}" for c in CASES])
def test_qelementwise_vs_oracle(qa, op, a_name, b_name, block, shape, mode):
    (pa, sa), (pb, sb), n = _operands(shape, 17 + block, block, a_name, b_name, mode)
    A = _mx(qa, pa, sa, a_name, shape, n, block)
    B = _mx(qa, pb, sb, b_name, shape, n, block)
    C = {"add": A + B, "sub": A - B, "mul": A * B}[op]
    rp, rs, rname = orc.dispatch_qelementwise(op, pa, sa, a_name, pb, sb, b_name, n, block)
    assert C._mx_dtype.name == rname
    assert C._mx_n == n and tuple(C._mx_orig_shape) == shape and C._mx_block == block
    assert _bits_eq(C._mx_scales, rs), "scales differ"
    assert _bits_eq(C._mx_packed, rp), "packed codes differ"


@pytest.mark.parametrize("op", ["add", "sub", "mul"])
@pytest.mark.parametrize("name", ["int2d", "int4d", "int8d"])
@pytest.mark.parametrize("mode", ["near", "far", "mixed"])
def test_qelementwise_tiny_and_zero_scales(qa, op, name, mode):
    """The fused kernel multiplies codes scaled by 2^(8 - bits) with scales
    scaled by 2^(bits - 8), exact for scales >= 2^-100; blocks whose scale
    is smaller (down to subnormal) or zero take the codes back to their
    values.  Operands with such scales in some blocks, against the oracle
    bitwise."""
    shape, block = (8, 512), 128
    (pa, sa), (pb, sb), n = _operands(shape, 23, block, name, name, mode)
    sa = sa.clone()
    sb = sb.clone()
    sa[::3] *= 2.0 ** -110
    sb[1::4] *= 2.0 ** -125
    sa[5] = 0.0
    sb[7] = 1e-44
    A = _mx(qa, pa, sa, name, shape, n, block)
    B = _mx(qa, pb, sb, name, shape, n, block)
    C = {"add": A + B, "sub": A - B, "mul": A * B}[op]
    rp, rs, rname = orc.dispatch_qelementwise(op, pa, sa, name, pb, sb, name, n, block)
    assert C._mx_dtype.name == rname
    assert _bits_eq(C._mx_scales, rs), "scales differ"
    assert _bits_eq(C._mx_packed, rp), "packed codes differ"


@pytest.mark.parametrize("name", ["int1d", "int2d", "int3d", "int4d", "int5d", "int8d", "int16d", "float4d",
                                  "float8d", "int4dh"])
def test_neg_vs_oracle(qa, name):
    shape, block = (5, 301), 128   # a padded last block
    x = torch.randn(*shape)
    p, s, n = orc.quantize(x, name, block)
    N = -_mx(qa, p, s, name, shape, n, block)
    rp, rs = orc.negate(p, s, name, n)
    assert N._mx_dtype.name == name
    assert _bits_eq(N._mx_packed, rp) and _bits_eq(N._mx_scales, rs)


def test_operator_routes(qa):
    """Routes of _binary_op (mxtorch.py:6450-6506, 6807-6819): a scalar
    operand requantizes the float result with the mx_tensor's dtype; torch.add
    on two mx_tensors takes the dequantize -> add -> requantize branch with
    _resolve_mixed's dtype; a shape mismatch fails as torch broadcasting does."""
    shape, block = (6, 256), 128
    (pa, sa), (pb, sb), n = _operands(shape, 5, block, "int8d", "int4d", "mixed")
    A = _mx(qa, pa, sa, "int8d", shape, n, block)
    B = _mx(qa, pb, sb, "int4d", shape, n, block)
    da = orc.dequant(pa, sa, "int8d", n, block).reshape(shape)
    db = orc.dequant(pb, sb, "int4d", n, block).reshape(shape)

    def same(mx, x, name):
        rp, rs, _ = orc.quantize(x, name, block)
        return mx._mx_dtype.name == name and _bits_eq(mx._mx_packed, rp) and _bits_eq(mx._mx_scales, rs)

    assert same(A + 2.5, da + 2.5, "int8d")
    assert same(A * 3.0, da * 3.0, "int8d")
    assert same(torch.add(A, B), da + db, "int4d")   # _resolve_mixed(int8d, int4d)
    assert same(A / 4.0, da / 4.0, "int8d")
    C = _mx(qa, pa[: 3 * 256].clone(), sa[:6].clone(), "int8d", (3, 256), 3 * 256, block)
    with pytest.raises(RuntimeError):
        _ = A + C                                      # broadcasting [6,256] + [3,256] fails, as in torch


def test_large_elementwise_roundtrip(qa):
    """A 2^24-element add on the GPU path against the oracle on a sampled
    set of blocks (blocks are independent)."""
    n, block = 1 << 24, 128
    g = torch.Generator()
    g.manual_seed(9)
    x = torch.randn(n, generator=g)
    y = torch.randn(n, generator=g) * torch.rand(n, generator=g).pow(3) * 4
    dt = qa.get_mx_dtype("int8d")
    A = qa.mx_tensor.quantize(x.to(dev()), dt, block)
    B = qa.mx_tensor.quantize(y.to(dev()), dt, block)
    C = A + B
    nb = n // block
    pick = torch.tensor(sorted({0, 1, 2, 777, nb // 2, nb - 2, nb - 1} | set(range(1000, nb, 9973))))
    idx = (pick[:, None] * block + torch.arange(block)[None, :]).reshape(-1)
    pa, sa, _ = orc.quantize(x[idx], "int8d", block)
    pb, sb, _ = orc.quantize(y[idx], "int8d", block)
    rp, rs, _ = orc.dispatch_qelementwise("add", pa, sa, "int8d", pb, sb, "int8d", idx.numel(), block)
    assert _bits_eq(C._mx_scales.cpu()[pick], rs)
    assert _bits_eq(C._mx_packed.cpu()[idx], rp)


@pytest.mark.parametrize("mkn", [(5, 128, 3), (7, 256, 9), (16, 128, 8)])
@pytest.mark.parametrize("name", ["int4d", "int8d"])
def test_elementwise_on_gemm_outputs(qa, mkn, name):
    """C + C, C - C and C * C where C = qa @ qb holds exactly M*N codes
    (mxtorch.py:5570), M*N not always a multiple of the block or of a lane's
    load: bitwise equal to the oracle applied to the oracle's C."""
    M, K, N = mkn
    g = torch.Generator()
    g.manual_seed(M * 1000 + N)
    A, B = torch.randn(M, K, generator=g), torch.randn(K, N, generator=g)
    dt = qa.get_mx_dtype(name)
    qc = qa.mx_tensor.quantize(A.to(dev()), dt, 128) @ qa.mx_tensor.quantize(B.to(dev()), dt, 128)
    pa, sa, na = orc.quantize(A, name, 128)
    pb, sb, nb = orc.quantize(B, name, 128)
    pc, sc, out_name = orc.dispatch_qgemm(pa, sa, name, (M, K), na, pb, sb, name, (K, N), nb, 128)
    assert _bits_eq(qc._mx_packed, pc) and _bits_eq(qc._mx_scales, sc)
    for op, r in (("add", qc + qc), ("sub", qc - qc), ("mul", qc * qc)):
        p_ref, s_ref, o_ref = orc.dispatch_qelementwise(op, pc, sc, out_name, pc, sc, out_name, M * N, 128)
        assert r._mx_dtype.name == o_ref, op
        assert _bits_eq(r._mx_packed, p_ref), op
        assert _bits_eq(r._mx_scales, s_ref), op


def test_hadamard_add_keeps_seed(qa):
    """add / sub of two 'h' tensors quantized with a non-default seed stay
    in the code domain and keep that seed, so the result dequantizes with the
    rotation its codes were made in; operands of different seeds go through
    dequantize -> add -> requantize."""
    dev = torch.device("cuda:0")
    g = torch.Generator()
    g.manual_seed(91)
    x = torch.randn(64, 128, generator=g)
    y = torch.randn(64, 128, generator=g) * 0.5
    dt = qa.get_mx_dtype("int4dh")
    a = qa.mx_tensor.quantize(x.to(dev), dt, 128, seed=777)
    b = qa.mx_tensor.quantize(y.to(dev), dt, 128, seed=777)
    for op, ref in (("add", x + y), ("sub", x - y)):
        c = a + b if op == "add" else a - b
        assert c._mx_seed == 777
        err = (c.dequantize().cpu() - ref).abs().max().item()
        assert err < 0.35 * ref.abs().max().item(), f"{op}: {err}"
        # the same codes read with the default seed are another rotation's
        wrong = qa.mx_tensor(c._mx_packed, c._mx_scales, dt, c._mx_orig_shape, c._mx_n, 128)
        assert wrong._mx_seed != 777
        err_wrong = (wrong.dequantize().cpu() - ref).abs().max().item()
        assert err_wrong > 2 * err, f"{op}: {err_wrong} vs {err}"
    b2 = qa.mx_tensor.quantize(y.to(dev), dt, 128, seed=778)
    c2 = a + b2
    err2 = (c2.dequantize().cpu() - (x + y)).abs().max().item()
    assert err2 < 0.35 * (x + y).abs().max().item()
