"""The oracle's model-level restatements against vectors written by the
reference itself (tests/golden/gen_fixtures.py):

  * quantized element-wise add / sub / mul / neg for int8d, int4d and int2d,
    including blocks whose scales are more than 2:1 apart
    (_dispatch_qadd / _dispatch_qsub / _dispatch_qmul, mxtorch.py:5321-5497;
    __neg__ mxtorch.py:6177-6193);
  * to_mx on a model with Linear and LayerNorm layers (mxtorch.py:9744-9858)
    and its forward;
  * mx_multihead_attention.from_mha / forward (mxtorch.py:7800-7877);
  * mx_transformer_encoder_layer.from_encoder_layer / forward
    (mxtorch.py:9161-9278);
  * the checkpoint the reference's save_quantized writes for that model
    (mxtorch.py:9860-9898), loaded with torch.load(weights_only=True).
Packed codes and scales bitwise; float outputs within a few ulps where the
reference's fp32 sgemm order is library-defined."""
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import mx_oracle as orc
from tests import _golden as G

EW = G.cases("elementwise")


@pytest.mark.parametrize("case", EW, ids=[c["key"] for c in EW])
def test_elementwise_oracle_matches_reference(case):
    key, name = case["key"], case["dtype"]
    A, B = G.get(key + "/A"), G.get(key + "/B")
    pa, sa, na = orc.quantize(A, name, 128)
    pb, sb, nb = orc.quantize(B, name, 128)
    pw, sw, _ = orc.quantize(B * case["wide_factor"], name, 128)
    for op, (bp, bs) in (("add", (pb, sb)), ("sub", (pb, sb)), ("mul", (pb, sb)),
                         ("addw", (pw, sw)), ("subw", (pw, sw)), ("mulw", (pw, sw))):
        pc, sc, out = orc.dispatch_qelementwise(op.rstrip("w"), pa, sa, name, bp, bs, name, na, 128)
        assert out == case["out_dtype"][op]
        assert torch.equal(pc, G.get(f"{key}/{op}/packed")), op
        assert G.bits_equal(sc, G.get(f"{key}/{op}/scales")), op
        dq = orc.dequant(pc, sc, out, na, 128)
        assert G.bits_equal(dq, G.get(f"{key}/{op}/dequant").reshape(-1)), op
    pn, sn = orc.negate(pa, sa, name, na)
    assert torch.equal(pn, G.get(f"{key}/neg/packed")) and G.bits_equal(sn, G.get(f"{key}/neg/scales"))


def _tomx_params():
    return {n: G.get(f"tomx/param/{n}") for n in ("fc1.weight", "fc1.bias", "norm.weight", "norm.bias",
                                                 "fc2.weight", "fc2.bias")}


def test_to_mx_model_oracle_matches_reference():
    p = _tomx_params()
    x = G.get("tomx/x")
    for lin in ("fc1", "fc2"):
        wp, ws, _ = orc.linear_from_weight(p[f"{lin}.weight"], "int4d", 128)
        assert torch.equal(wp, G.get(f"tomx/{lin}/w_packed")) and G.bits_equal(ws, G.get(f"tomx/{lin}/w_scales"))
    nw, nb = orc.layer_norm_from(p["norm.weight"], p["norm.bias"], "int4d", 128)
    assert torch.equal(nw[0], G.get("tomx/norm/w_packed")) and torch.equal(nb[0], G.get("tomx/norm/b_packed"))
    w1p, w1s, _ = orc.linear_from_weight(p["fc1.weight"], "int4d", 128)
    h = orc.linear_forward(x, w1p, w1s, "int4d", 64, 128, 128, has_bias=True)
    n = orc.layer_norm_forward(F.relu(h), nw, nb, (128,), 1e-5, "int4d", 128)
    w2p, w2s, _ = orc.linear_from_weight(p["fc2.weight"], "int4d", 128)
    y = orc.linear_forward(orc._dq_entry(n, "int4d", 128), w2p, w2s, "int4d", 128, 32, 128, has_bias=True)
    y_ref = G.get("tomx/y")
    assert (y - y_ref).abs().max().item() <= 1e-5 * y_ref.abs().max().item()


def test_reference_checkpoint_format():
    """The reference's save_quantized file: the __mx_version__ marker and one
    entry per quantized "weight" / "bias" attribute (mx_linear's own packed
    weights are not among them, mxtorch.py:9867-9884), holding the same
    bytes the oracle's quantize produces."""
    ck = torch.load(os.path.join(G.HERE, "ref_checkpoint.pt"), map_location="cpu", weights_only=True)
    assert ck["__mx_version__"] == 2
    assert set(ck) == {"__mx_version__", "norm.weight", "norm.bias"}
    p = _tomx_params()
    for attr in ("weight", "bias"):
        e = ck[f"norm.{attr}"]
        pk, sc, n = orc.quantize(p[f"norm.{attr}"], "int4d", 128)
        assert e["dtype"] == "int4d" and e["shape"] == [128] and e["n"] == n and e["block"] == 128
        assert torch.equal(e["packed"], pk) and G.bits_equal(e["scales"], sc)


def test_mha_oracle_matches_reference():
    P = lambda n: G.get(f"mha/param/{n}")  # noqa: E731
    inp, outw, outb = orc.mha_from(P("in_proj_weight"), P("out_proj.weight"), P("out_proj.bias"), "int8d", 128)
    assert torch.equal(inp[0], G.get("mha/in_proj/packed")) and G.bits_equal(inp[1], G.get("mha/in_proj/scales"))
    assert torch.equal(outw[0], G.get("mha/out_proj/packed"))
    q = G.get("mha/q")
    (pk, sc, _), attn, _ = orc.mha_forward(q, q, q, 128, 4, inp, P("in_proj_bias"), outw, outb, "int8d", 128)
    assert torch.equal(pk, G.get("mha/out/packed")) and G.bits_equal(sc, G.get("mha/out/scales"))
    assert G.bits_equal(attn, G.get("mha/attn"))


def test_encoder_layer_oracle_matches_reference():
    case = G.cases("encoder_layer")[0]
    names = ["self_attn.in_proj_weight", "self_attn.in_proj_bias", "self_attn.out_proj.weight",
             "self_attn.out_proj.bias", "linear1.weight", "linear1.bias", "linear2.weight", "linear2.bias",
             "norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias"]
    params = {n: G.get(f"enc/param/{n}") for n in names}
    for lin in ("linear1", "linear2"):
        wp, _, _ = orc.linear_from_weight(params[f"{lin}.weight"], "int8d", 128)
        assert torch.equal(wp, G.get(f"enc/{lin}/w_packed"))
    y = orc.encoder_layer_forward(G.get("enc/src"), params, "int8d", 128, nhead=case["nhead"])
    y_ref = G.get("enc/y")
    assert G.bits_equal(y, y_ref) or (y - y_ref).abs().max().item() <= 1e-5 * y_ref.abs().max().item()


VQ = G.cases("vector_quantize")


@pytest.mark.parametrize("case", VQ, ids=[c["key"] for c in VQ])
def test_vector_quantize_oracle_matches_reference(case):
    codes, scales = orc.vector_quantize(G.get("vq/x"), case["dtype"], case["axis"])
    assert torch.equal(codes, G.get(case["key"] + "/codes"))
    assert G.bits_equal(scales, G.get(case["key"] + "/scales"))
    assert G.bits_equal(orc.vector_dequantize(codes, scales, case["axis"]), G.get(case["key"] + "/dequant"))


def test_vector_quantize_per_row_is_the_v_rule():
    """Per row, vector_quantize's int codes are the golden-pinned 'v'
    quantizer's (quant_vector) with the row length as block, for widths whose
    'v' codes pack into bytes."""
    x = G.get("vq/x")
    for name in ("int8d", "int4d", "int2d"):
        codes, scales = orc.vector_quantize(x, name, 1)
        p, s, n = orc.quantize(x, name.replace("d", "dv"), 300)
        assert G.bits_equal(scales, s)
        assert torch.equal(codes.reshape(-1), orc.unpack_auto(p, orc.parse_dtype(name)[1], n).to(torch.int32))
