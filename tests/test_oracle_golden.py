"""Pins the CPU oracle (oracle/mx_oracle.py) against the golden vectors that
tests/golden/gen_fixtures.py wrote by running the reference's CPU path
(mxtorch.py) on seeded, ragged, tie, zero, tiny and outlier inputs, and
against the reference's own pack KATs (mxtorch_test.py:86-112, 204-209).

Bar: packed bytes/words, scales and dequantized floats are bitwise equal
(sign of zero included); GEMM outputs (packed codes, scales) bitwise equal.
"""
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

QCASES = G.cases("quantize")


@pytest.mark.parametrize("case", QCASES, ids=[c["key"] for c in QCASES])
def test_quantize_matches_reference(case):
    x = G.input_tensor(case["input"])
    seed = None
    if case["dtype"].endswith("h"):
        seed = G.index()["hash_seed"][case["dtype"]]
    packed, scales, n = orc.quantize(x, case["dtype"], case["block"], seed=seed)
    assert n == case["n"]
    assert G.bits_equal(packed, G.get(case["key"] + "/packed"))
    assert G.bits_equal(scales, G.get(case["key"] + "/scales"))
    dq = orc.dequant(packed, scales, case["dtype"], n, case["block"], seed=seed,
                     orig_shape=tuple(case["shape"]), hadamard_mode="reference")
    assert G.bits_equal(dq.reshape(case["shape"]), G.get(case["key"] + "/dequant"))


NFCASES = G.cases("quantize_nonfinite")


@pytest.mark.parametrize("case", NFCASES, ids=[c["key"] for c in NFCASES])
def test_quantize_nonfinite_matches_reference(case):
    """Blocks holding NaN or +-inf (mxtorch.py:1456-1460, 1497-1524): the
    reference's amax gives NaN or inf scales, and its codes come from NaN
    and zero quotients.  Codes and scales bitwise (the reference's NaN
    scales are 0x7FC00000); dequantized values with any NaN for a NaN."""
    x = G.input_tensor(case["input"])
    seed = G.index()["hash_seed"][case["dtype"]] if case["dtype"].endswith("h") else None
    packed, scales, n = orc.quantize(x, case["dtype"], case["block"], seed=seed)
    assert G.bits_equal(packed, G.get(case["key"] + "/packed"))
    assert G.bits_equal(scales, G.get(case["key"] + "/scales"))
    assert torch.isnan(scales).any() and torch.isinf(scales).any()
    dq = orc.dequant(packed, scales, case["dtype"], n, case["block"], seed=seed,
                     orig_shape=tuple(case["shape"]), hadamard_mode="reference")
    assert G.nan_aware_equal(dq.reshape(case["shape"]), G.get(case["key"] + "/dequant"))


MCASES = G.cases("matmul")


@pytest.mark.parametrize("case", MCASES, ids=[c["key"] for c in MCASES])
def test_qgemm_matches_reference(case):
    A, B = G.get(case["key"] + "/A"), G.get(case["key"] + "/B")
    name = case["dtype"]
    pa, sa, na = orc.quantize(A, name, 128)
    pb, sb, nb = orc.quantize(B, name, 128)
    pc, sc, out_name = orc.dispatch_qgemm(pa, sa, name, A.shape, na, pb, sb, name, B.shape, nb, 128)
    assert out_name == case["out_dtype"]
    assert G.bits_equal(pc, G.get(case["key"] + "/packed"))
    assert G.bits_equal(sc, G.get(case["key"] + "/scales"))
    M, N = case["M"], case["N"]
    dq = orc.dequant(pc, sc, out_name, M * N, 128).reshape(M, N)
    assert G.bits_equal(dq, G.get(case["key"] + "/dequant"))
    ste = orc.qgemm_ste_forward(A, B, name, 128)
    assert G.bits_equal(ste, G.get(case["key"] + "/ste"))


LCASES = G.cases("linear")


@pytest.mark.parametrize("case", LCASES, ids=[c["key"] for c in LCASES])
def test_linear_matches_reference(case):
    W = G.get(case["key"] + "/W")
    x = G.get(case["key"] + "/x")
    wp, ws, _ = orc.linear_from_weight(W, case["dtype"], 128)
    assert G.bits_equal(wp, G.get(case["key"] + "/w_packed"))
    assert G.bits_equal(ws, G.get(case["key"] + "/w_scales"))
    y = orc.linear_forward(x, wp, ws, case["dtype"], case["in"], case["out"], 128,
                           has_bias=case["bias"])
    # F.linear is an fp32 sgemm: same library, same shapes, same order here.
    assert G.bits_equal(y, G.get(case["key"] + "/y"))


KCASES = G.cases("kv")


@pytest.mark.parametrize("case", KCASES, ids=[c["key"] for c in KCASES])
def test_kv_cache_matches_reference(case):
    key = case["key"]
    ks, vs = G.get(key + "/k"), G.get(key + "/v")
    steps = [orc.kv_append(ks[t], vs[t], case["dtype"], case["D"]) for t in range(case["T"])]
    for t, (kq, vq, _) in enumerate(steps):
        assert G.bits_equal(kq[0], G.get(f"{key}/kq{t}/packed"))
        assert G.bits_equal(kq[1], G.get(f"{key}/kq{t}/scales"))
        assert G.bits_equal(vq[0], G.get(f"{key}/vq{t}/packed"))
        assert G.bits_equal(vq[1], G.get(f"{key}/vq{t}/scales"))
    K, V = orc.kv_get(steps, case["dtype"], case["D"], case["H"])
    assert G.bits_equal(K, G.get(key + "/K"))
    assert G.bits_equal(V, G.get(key + "/V"))


def test_pack_kats_from_reference_tests():
    """mxtorch_test.py:86-112: int4/int1/int2 byte counts and exact int4/int2
    round trips; 3-bit pack_arb yields int32 words."""
    vals = torch.tensor([3, -2, 7, -8, 0, 1, -1, 4], dtype=torch.int8)
    p4 = orc.pack(vals, 4)
    assert p4.dtype == torch.int8 and p4.numel() == 4
    assert torch.equal(orc.unpack(p4, 4, 8), vals.float())
    assert G.bits_equal(p4, G.get("kat/pack4"))
    # LSB-first: byte0 = lo(3) | lo(-2)<<4 = 0x03 | 0xE0
    assert p4.tolist()[0] == torch.tensor(0xE3, dtype=torch.uint8).view(torch.int8).item()
    p1 = orc.pack(torch.tensor([0, 1, 0, 1, 1, 0, 1, 0], dtype=torch.int8), 1)
    assert p1.numel() == 1 and G.bits_equal(p1, G.get("kat/pack1"))
    v2 = torch.tensor([1, -2, 0, -1, 1, -2, 0, 1], dtype=torch.int8)
    p2 = orc.pack(v2, 2)
    assert p2.numel() == 2 and torch.equal(orc.unpack(p2, 2, 8), v2.float())
    assert G.bits_equal(p2, G.get("kat/pack2"))
    p3 = orc.pack_arb(torch.tensor([3, -4, 2, -3, 0, 1, -1, 3], dtype=torch.int32), 3)
    assert p3.dtype == torch.int32 and G.bits_equal(p3, G.get("kat/pack3"))
    p16 = orc.pack_arb(torch.tensor([32767, -32767, 5, -1, 0], dtype=torch.int32), 16)
    assert G.bits_equal(p16, G.get("kat/pack16"))
    assert torch.equal(orc.unpack_arb(p16, 16, 5), torch.tensor([32767., -32767., 5., -1., 0.]))


def test_int4_masks():
    """mxtorch_test.py:204-209: int4 fields sit under masks 0xF and 0xF0."""
    p = orc.pack(torch.tensor([5, 0, 0, 6], dtype=torch.int8), 4)
    assert (p[0].item() & 0xF) == 5 and (p[0].item() & 0xF0) == 0
    assert ((p[1].item() & 0xF0) >> 4) == 6


def test_grids_match_reference():
    assert G.bits_equal(orc.float_grid(4), G.get("grid/4"))
    assert G.bits_equal(orc.float_grid(8), G.get("grid/8"))
