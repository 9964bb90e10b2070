"""Pins for the oracle's quantized element-wise arithmetic (oracle.qscale_add,
qscale_mul, dispatch_qelementwise, negate; mxtorch.py:1186-1296,
5321-5497, 6177-6193).  The reference's own tests check these loosely
(mxtorch_test.py:3303-3314: dequant(-q) = -dequant(q), dtype and scales
kept); the checks below fix them through independent routes:

  * equal scales, no overflow: codes are the exact integer sums a + b;
  * overflow: the scale doubles once and codes are rne(a/2) + rne(b/2);
  * scales more than 2:1 apart: the result is the 'v'-rule quantization
    (oracle.quant_vector, pinned by the golden int8dv fixtures) of the
    float32 sum RN(a*sa) + RN(b*sb), computed here with numpy float32;
  * mul: per element with numpy float32 (IEEE RN at every step);
  * sub(a, b) = add(a, -b) on int codes; neg twice is the identity;
  * the output-dtype rules on every pair of widths, from their definitions.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as orc


def _codes(n, bits, seed, lo=None):
    g = torch.Generator()
    g.manual_seed(seed)
    q = (1 << (bits - 1)) - 1
    return torch.randint(-q if lo is None else lo, q + 1, (n,), generator=g, dtype=torch.int32)


def test_add_equal_scales_is_integer_sum():
    bits, block, nb = 8, 64, 6
    a = _codes(nb * block, bits, 1, lo=-60)
    b = _codes(nb * block, bits, 2, lo=-60)
    a.clamp_(-60, 60)
    b.clamp_(-60, 60)
    s = torch.rand(nb) + 0.25
    c, cs = orc.qscale_add(a, s, b, s.clone(), bits, block)
    assert torch.equal(c, a + b)
    assert torch.equal(cs, s)


def test_add_overflow_doubles_scale_once():
    bits, block = 4, 32
    a = torch.full((block,), 7, dtype=torch.int32)
    b = torch.full((block,), 5, dtype=torch.int32)
    b[::2] = -3
    s = torch.tensor([0.5])
    c, cs = orc.qscale_add(a, s, b, s.clone(), bits, block)
    assert cs.item() == 1.0
    half = lambda v: np.rint(np.float32(v) * np.float32(0.5)).astype(np.int32)
    expect = half(a.numpy()) + half(b.numpy())
    assert np.array_equal(c.numpy(), np.clip(expect, -7, 7))


@pytest.mark.parametrize("bits", [2, 4, 8, 16])
def test_add_far_scales_is_v_rule_of_float_sum(bits):
    block, nb = 128, 5
    a = _codes(nb * block, bits, 3 + bits)
    b = _codes(nb * block, bits, 4 + bits)
    sa = torch.rand(nb) + 1.0
    sb = sa * torch.tensor([3.0, 0.1, 2.5, 100.0, 0.45])  # every ratio > 2
    c, cs = orc.qscale_add(a, sa, b, sb, bits, block)
    af = a.numpy().astype(np.float32).reshape(nb, block)
    bf = b.numpy().astype(np.float32).reshape(nb, block)
    s = af * sa.numpy()[:, None].astype(np.float32) + bf * sb.numpy()[:, None].astype(np.float32)
    vname = f"int{bits}dv"
    rp, rs, _ = orc.quant_vector(torch.from_numpy(s.reshape(-1)), vname, block)
    assert torch.equal(cs, rs)
    assert torch.equal(c, orc.unpack_auto(rp, bits, nb * block).to(torch.int32))


@pytest.mark.parametrize("bits", [2, 3, 4, 8, 16])
def test_mul_elementwise_float32(bits):
    block, nb = 64, 4
    a = _codes(nb * block, bits, 5 + bits)
    b = _codes(nb * block, bits, 6 + bits)
    sa, sb = torch.rand(nb) + 0.1, torch.rand(nb) * 3
    c, cs = orc.qscale_mul(a, sa, b, sb, bits, block)
    q = np.float32((1 << (bits - 1)) - 1)
    prod = a.numpy().astype(np.float32) * b.numpy().astype(np.float32)
    expect = np.rint(np.clip(prod / q, -q, q)).astype(np.int32)
    assert np.array_equal(c.numpy(), expect)
    assert np.array_equal(cs.numpy(), (sa.numpy().astype(np.float32) * sb.numpy().astype(np.float32)) * q)


def test_sub_is_add_of_negated_codes_and_neg_is_involution():
    x = torch.randn(3, 200)
    y = torch.randn(3, 200) * 0.7
    pa, sa, n = orc.quantize(x, "int4d", 32)
    pb, sb, _ = orc.quantize(y, "int4d", 32)
    nbp, nbs = orc.negate(pb, sb, "int4d", n)
    sub = orc.dispatch_qelementwise("sub", pa, sa, "int4d", pb, sb, "int4d", n, 32)
    add = orc.dispatch_qelementwise("add", pa, sa, "int4d", nbp, nbs, "int4d", n, 32)
    assert torch.equal(sub[0], add[0]) and torch.equal(sub[1], add[1])
    p2, s2 = orc.negate(*orc.negate(pa, sa, "int4d", n), "int4d", n)
    assert torch.equal(orc.unpack_auto(p2, 4, n), orc.unpack_auto(pa, 4, n)) and torch.equal(s2, sa)


def test_neg_matches_reference_test_conditions():
    """mxtorch_test.py:3303-3314."""
    w = torch.randn(64, 64)
    p, s, n = orc.quantize(w, "int8d", 32)
    np_, ns = orc.negate(p, s, "int8d", n)
    pos = orc.dequant(p, s, "int8d", n, 32)
    neg = orc.dequant(np_, ns, "int8d", n, 32)
    assert (pos + neg).abs().max().item() < 1e-5
    assert torch.equal(ns, s)
    # 8-bit codes are negated byte by byte with a clamp at +-127: -(-128) -> 127
    raw = torch.tensor([-128, -1, 0, 5, 127], dtype=torch.int8)
    assert orc.negate(raw, torch.ones(1), "float8d", 5)[0].tolist() == [127, 1, 0, -5, -127]


def test_output_dtype_rules():
    bits = (1, 2, 3, 4, 5, 6, 7, 8, 16)
    for a in bits:
        for b in bits:
            assert orc.resolve_mixed(f"int{a}d", f"float{b}u") == f"float{min(a, b)}u"
        assert orc.resolve_mixed(f"int{a}dv", f"int{a}dh") == f"int{a}dh"
    widened = {1: 2, 2: 4, 3: 6, 4: 8, 5: 8, 6: 16, 7: 16, 8: 16, 16: 16}
    for a, w in widened.items():
        assert orc.qmul_out_name(f"int{a}d") == f"int{w}d"
        assert orc.qmul_out_name(f"float{a}u") == f"float{w}d"
