"""GPU parity: the HIP path (libmxk.so through qtpytorch_amd) against the
reference's golden vectors and the CPU oracle on the same seeded inputs.

Bar (from the north star):
  * packed codes, scales, dequantized floats, int32 GEMM accumulators and
    the fp32 GEMM accumulator C: bitwise equal;
  * fp32 outputs of mx_linear (an fp32 sgemm in the reference, whose
    summation order is library-defined): max|y - y_ref| <= 1e-3 * max|y_ref|.
"""
import math

import numpy as np
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

pytestmark = pytest.mark.gpu

LINEAR_RTOL = 1e-3


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


# ---------------------------------------------------------------- golden vectors
QCASES = G.cases("quantize")


@pytest.mark.parametrize("case", QCASES, ids=[c["key"] for c in QCASES])
def test_quantize_golden(qa, case):
    x = G.input_tensor(case["input"]).to(dev())
    dt = qa.get_mx_dtype(case["dtype"])
    seed = G.index()["hash_seed"].get(case["dtype"]) if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x, dt, case["block"], seed=seed)
    assert n == case["n"]
    assert _bits_eq(packed, G.get(case["key"] + "/packed")), "packed codes differ"
    assert _bits_eq(scales, G.get(case["key"] + "/scales")), "scales differ"
    dq = qa.ops._dequant(packed, scales, dt, n, case["block"], orig_shape=tuple(case["shape"]), seed=seed,
                         hadamard_mode="reference")
    assert _bits_eq(dq.reshape(case["shape"]), G.get(case["key"] + "/dequant")), "dequantized values differ"


NFCASES = G.cases("quantize_nonfinite")


@pytest.mark.parametrize("case", NFCASES, ids=[c["key"] for c in NFCASES])
def test_quantize_nonfinite_golden(qa, case):
    """Blocks holding NaN or +-inf, against the reference-written codes and
    scales (bitwise: NaN scales 0x7FC00000, infinite scales +inf, codes of
    NaN quotients 0, float codes of NaN the last index); dequantized values
    with any NaN for a NaN."""
    x = G.input_tensor(case["input"]).to(dev())
    dt = qa.get_mx_dtype(case["dtype"])
    seed = G.index()["hash_seed"].get(case["dtype"]) if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x, dt, case["block"], seed=seed)
    assert _bits_eq(packed, G.get(case["key"] + "/packed")), "packed codes differ"
    assert _bits_eq(scales, G.get(case["key"] + "/scales")), "scales differ"
    dq = qa.ops._dequant(packed, scales, dt, n, case["block"], orig_shape=tuple(case["shape"]), seed=seed,
                         hadamard_mode="reference")
    assert G.nan_aware_equal(dq.reshape(case["shape"]).cpu(), G.get(case["key"] + "/dequant"))


@pytest.mark.parametrize("name", ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int8dv", "int4dh",
                                  "float8dh"])
@pytest.mark.parametrize("src", ["f32", "f16", "long", "generic"])
def test_quantize_nonfinite_kernels(qa, name, src):
    """NaN and +-inf through every quantize kernel (the fused kernel from
    fp32 and from fp16, the one-workgroup-per-block kernel for blocks above
    512, the generic two-pass kernel for other block sizes) against the
    oracle, which restates the reference's torch ops: codes and scales
    bitwise."""
    dt = qa.get_mx_dtype(name)
    if dt.is_hadamard and src in ("long", "generic"):
        pytest.skip("'h' rotates rows of the last dimension; covered at 128")
    block = {"long": 1024, "generic": 96}.get(src, 128)
    g = torch.Generator()
    g.manual_seed(77)
    x = torch.randn(24, 1024, generator=g)
    flat = x.view(-1)
    flat[5] = float("nan")
    flat[1500] = float("inf")
    flat[3000] = float("-inf")
    flat[3001] = float("nan")
    flat[9000] = float("inf")
    flat[9001] = float("-inf")
    flat[20000] = float("-nan")
    if src == "f16":
        x = x.half()
    if dt.is_hadamard:
        x = x.reshape(-1, 128)
    seed = 1534857261 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, block, seed=seed)
    rp, rs, rn = orc.quantize(x, name, block, seed=seed) if seed is not None else orc.quantize(x, name, block)
    assert n == rn
    assert _bits_eq(packed, rp), "packed codes differ"
    assert _bits_eq(scales, rs), "scales differ"


MCASES = G.cases("matmul")


@pytest.mark.parametrize("case", MCASES, ids=[c["key"] for c in MCASES])
def test_qgemm_golden(qa, case):
    A = G.get(case["key"] + "/A").to(dev())
    B = G.get(case["key"] + "/B").to(dev())
    dt = qa.get_mx_dtype(case["dtype"])
    qa_ = qa.mx_tensor.quantize(A, dt, 128)
    qb_ = qa.mx_tensor.quantize(B, dt, 128)
    qc = qa_ @ qb_
    assert isinstance(qc, qa.mx_tensor)
    assert qc._mx_dtype.name == case["out_dtype"]
    assert _bits_eq(qc._mx_packed, G.get(case["key"] + "/packed"))
    assert _bits_eq(qc._mx_scales, G.get(case["key"] + "/scales"))
    if qc._mx_dtype.is_int:
        assert _bits_eq(qc.dequantize(), G.get(case["key"] + "/dequant"))
        ste = qa._QGemmSTE.apply(A, B, dt, 128)
        assert _bits_eq(ste, G.get(case["key"] + "/ste"))


LCASES = G.cases("linear")


@pytest.mark.parametrize("case", LCASES, ids=[c["key"] for c in LCASES])
def test_linear_golden(qa, case):
    W = G.get(case["key"] + "/W")
    lin = torch.nn.Linear(case["in"], case["out"], bias=case["bias"])
    with torch.no_grad():
        lin.weight.copy_(W)
        if case["bias"]:
            lin.bias.copy_(G.get(case["key"] + "/bias"))
    lin = lin.to(dev())
    m = qa.mx_linear.from_linear(lin, qa.get_mx_dtype(case["dtype"]), 128)
    assert _bits_eq(m._mx_weight._mx_packed, G.get(case["key"] + "/w_packed"))
    assert _bits_eq(m._mx_weight._mx_scales, G.get(case["key"] + "/w_scales"))
    y = m(G.get(case["key"] + "/x").to(dev())).cpu()
    y_ref = G.get(case["key"] + "/y")
    assert (y - y_ref).abs().max().item() <= LINEAR_RTOL * y_ref.abs().max().item()


KCASES = G.cases("kv")


@pytest.mark.parametrize("case", KCASES, ids=[c["key"] for c in KCASES])
def test_kv_cache_golden(qa, case):
    key = case["key"]
    cache = qa.kv_cache_quantizer(n_heads=case["H"], head_dim=case["D"], dtype=case["dtype"])
    ks, vs = G.get(key + "/k"), G.get(key + "/v")
    for t in range(case["T"]):
        cache.append_kv(ks[t].to(dev()), vs[t].to(dev()))
    kq, vq = cache.get_quantized()
    for t in range(case["T"]):
        assert _bits_eq(kq[t]._mx_packed, G.get(f"{key}/kq{t}/packed"))
        assert _bits_eq(kq[t]._mx_scales, G.get(f"{key}/kq{t}/scales"))
        assert _bits_eq(vq[t]._mx_packed, G.get(f"{key}/vq{t}/packed"))
        assert _bits_eq(vq[t]._mx_scales, G.get(f"{key}/vq{t}/scales"))
    K, V = cache.get()
    assert _bits_eq(K, G.get(key + "/K"))
    assert _bits_eq(V, G.get(key + "/V"))


# ---------------------------------------------------------------- seeded vs oracle
def _randn(shape, seed, outliers=0.0, scale=50.0):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        m = torch.rand(*shape, generator=g) < outliers
        x[m] *= scale
    return x


QDTYPES = ["int8d", "int4d", "int2d", "int1d", "int3d", "int5d", "int7d", "float4d", "float8d", "int8dv",
           "int4dv", "int16d", "int4dh", "int8dh", "float8dh", "int1dh"]


@pytest.mark.parametrize("dtype", QDTYPES)
@pytest.mark.parametrize("block", [128, 64, 32, 256, 96])
def test_quantize_seeded_vs_oracle(qa, dtype, block):
    seed = 1000 + QDTYPES.index(dtype) * 7 + block
    x = _randn((37, 1024 + 3 * 128), seed, outliers=1e-3)
    if dtype.endswith("h"):
        x = x[:, :512].contiguous()
    dt = qa.get_mx_dtype(dtype)
    hseed = 12345 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, block, seed=hseed)
    rp, rs, rn = orc.quantize(x, dtype, block, seed=hseed)
    assert n == rn
    assert _bits_eq(packed, rp), f"{dtype}/{block}: packed codes differ"
    assert _bits_eq(scales, rs), f"{dtype}/{block}: scales differ"
    dq = qa.ops._dequant(packed, scales, dt, n, block, orig_shape=tuple(x.shape), seed=hseed,
                         hadamard_mode="rows")
    rdq = orc.dequant(rp, rs, dtype, rn, block, seed=hseed, orig_shape=tuple(x.shape), hadamard_mode="rows")
    assert _bits_eq(dq, rdq), f"{dtype}/{block}: dequantized values differ"


@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d"])
@pytest.mark.parametrize("block", [4, 12, 20, 36, 100, 132, 252, 1000, 4096])
def test_dequantize_block_sizes(qa, dtype, block):
    """The 4-output-slot dequantizer finds each slot's block by a
    multiplicative division by block / 4 (an invariant divisor, Granlund and
    Montgomery): blocks that are not powers of two, ragged n, against the
    oracle bit for bit."""
    n = 9 * block * 37 + 4 * (block // 4 // 2 + 1) + 3
    x = _randn((n,), 4000 + block, outliers=1e-3)
    dt = qa.get_mx_dtype(dtype)
    packed, scales, nn = qa.ops.quantize(x.to(dev()), dt, block)
    rp, rs, rn = orc.quantize(x, dtype, block)
    assert nn == rn and _bits_eq(packed, rp) and _bits_eq(scales, rs)
    dq = qa.ops._dequant(packed, scales, dt, nn, block, orig_shape=(n,))
    rdq = orc.dequant(rp, rs, dtype, rn, block, orig_shape=(n,))
    assert _bits_eq(dq, rdq), f"{dtype}/{block}: dequantized values differ"


@pytest.mark.parametrize("dtype", ["float4d", "float8d", "float4dh", "float8dh"])
def test_float_codes_of_subnormals(qa, dtype):
    """Float codes of subnormal values k * 2^-149 in blocks whose scale lies
    within 3 ulps of 2k, where RN(x / s) turns zero: Markstein's correction
    alone rounds some of these to 0 where IEEE division gives 2^-149 (its
    residual falls on the subnormal grid), so the quantizers divide by the
    hardware sequence when a wave holds a subnormal.  Blocks of 128: element 0
    is the scale, the rest subnormals of both signs near k * 2^-149.  Codes
    and scales bit-exact against the oracle (782 of the values change their
    zero-ness under the correction alone)."""
    g = np.random.default_rng(5)
    rows = []
    for r in range(256):
        k = int(g.integers(1, 1 << 22))
        s = np.float32(2 * k)
        for _ in range(abs(r % 7 - 3)):
            s = np.nextafter(s, np.float32(np.inf if r % 7 > 3 else 0.0), dtype=np.float32)
        ks = np.clip(k + g.integers(-2, 3, 127), 1, (1 << 23) - 1)
        sub = (ks.astype(np.float64) * 2.0 ** -149).astype(np.float32) * np.where(g.random(127) < 0.5, -1, 1)
        rows.append(np.concatenate([[s], sub.astype(np.float32)]))
    x = torch.from_numpy(np.stack(rows).astype(np.float32))
    # (the 'h' quantizers rotate first, which keeps only part of the values
    # subnormal; they run the same rows for coverage of their vote)
    dt = qa.get_mx_dtype(dtype)
    hseed = 4321 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=hseed)
    rp, rs, rn = orc.quantize(x, dtype, 128, seed=hseed)
    assert n == rn
    assert _bits_eq(scales, rs), f"{dtype}: scales differ"
    assert _bits_eq(packed, rp), f"{dtype}: packed codes differ"


@pytest.mark.parametrize("dtype", ["int4dh", "int8dh", "int2dh", "int1dh", "float4dh", "float8dh"])
def test_quantize_had_tiny_values(qa, dtype):
    """'h' quantize of rows holding values below 2^-96 (subnormals, 2^-100,
    1e-35, zeros of both signs) next to normal ones, and rows of tiny values
    only.  The integer widths of 2+ bits divide by sqrt(128) without the
    small-value vote (their codes of such values are 0 on either path, the
    scale comes from the maximum before the division); int1dh and the float
    widths keep it.  Codes and scales bit-exact against the oracle."""
    g = torch.Generator()
    g.manual_seed(91)
    rows = []
    tiny = torch.tensor([1e-45, -1e-45, 3e-45, 2.0 ** -100, -(2.0 ** -100), 1e-35, -1e-38, 0.0, -0.0, 2.0 ** -126])
    for r in range(64):
        v = torch.randn(128, generator=g)
        if r % 4 == 0:
            v = tiny[torch.randint(0, tiny.numel(), (128,), generator=g)]
        elif r % 4 == 1:
            m = torch.rand(128, generator=g) < 0.5
            v[m] = tiny[torch.randint(0, tiny.numel(), (int(m.sum()),), generator=g)]
        elif r % 4 == 2:
            v = v * 1e-30
        rows.append(v)
    x = torch.stack(rows)
    dt = qa.get_mx_dtype(dtype)
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=777)
    rp, rs, rn = orc.quantize(x, dtype, 128, seed=777)
    assert n == rn
    assert _bits_eq(scales, rs), f"{dtype}: scales differ"
    assert _bits_eq(packed, rp), f"{dtype}: packed codes differ"


@pytest.mark.parametrize("src", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int8dv", "float8d", "int4dh", "int1d"])
def test_quantize_half_inputs(qa, src, dtype):
    x = _randn((64, 256), 77, outliers=1e-2, scale=20.0).to(src)
    dt = qa.get_mx_dtype(dtype)
    hseed = 99 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=hseed)
    rp, rs, _ = orc.quantize(x, dtype, 128, seed=hseed)
    assert _bits_eq(packed, rp) and _bits_eq(scales, rs)


@pytest.mark.parametrize("n", [1, 5, 127, 129, 1000, 4097])
@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int8dv"])
def test_ragged_lengths(qa, n, dtype):
    x = _randn((n,), 5 + n)
    packed, scales, m = qa.ops.quantize(x.to(dev()), qa.get_mx_dtype(dtype), 128)
    rp, rs, _ = orc.quantize(x, dtype, 128)
    assert _bits_eq(packed, rp) and _bits_eq(scales, rs)
    dq = qa.ops._dequant(packed, scales, qa.get_mx_dtype(dtype), m, 128)
    assert _bits_eq(dq, orc.dequant(rp, rs, dtype, m, 128))


def test_misaligned_input_takes_generic_path(qa):
    base = _randn((1025,), 3).to(dev())
    x = base[1:]  # 4-byte offset: not 16-byte aligned
    for dtype in ("int4d", "float8d", "int8dv"):
        packed, scales, _ = qa.ops.quantize(x, qa.get_mx_dtype(dtype), 128)
        rp, rs, _ = orc.quantize(x.cpu(), dtype, 128)
        assert _bits_eq(packed, rp) and _bits_eq(scales, rs)


def test_hadamard_large_rotation(qa):
    """1-D input: one whole-tensor rotation of next_pow2(n) = 16384 points
    (global butterfly pass + LDS tail)."""
    x = _randn((12000,), 8)
    dt = qa.get_mx_dtype("int4dh")
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=7)
    rp, rs, _ = orc.quantize(x, "int4dh", 128, seed=7)
    assert _bits_eq(packed, rp) and _bits_eq(scales, rs)
    dq = qa.ops._dequant(packed, scales, dt, n, 128, seed=7, hadamard_mode="reference")
    assert _bits_eq(dq, orc.dequant(rp, rs, "int4dh", n, 128, seed=7))


@pytest.mark.parametrize("dtype", ["int4dh", "int8dh", "int2dh", "int1dh", "float4dh", "float8dh"])
def test_hadamard_rows128_dequant(qa, dtype):
    """Rows of 128 = blocks of 128: the fused dequantize + inverse rotation
    kernel, bit-exact against the oracle's row-wise unrotation, with a row
    count that leaves the last workgroup partly idle."""
    x = _randn((1000, 128), 61, outliers=1e-3)
    dt = qa.get_mx_dtype(dtype)
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=4242)
    rp, rs, rn = orc.quantize(x, dtype, 128, seed=4242)
    assert _bits_eq(packed, rp) and _bits_eq(scales, rs)
    dq = qa.ops._dequant(packed, scales, dt, n, 128, orig_shape=(1000, 128), seed=4242, hadamard_mode="rows")
    rdq = orc.dequant(rp, rs, dtype, rn, 128, seed=4242, orig_shape=(1000, 128), hadamard_mode="rows")
    assert _bits_eq(dq, rdq)


@pytest.mark.parametrize("dtype", ["float8d", "float4d", "int8d", "int4d", "int2d", "int1d", "float8dh", "int8dh",
                                   "int4dh"])
def test_dequant_every_code(qa, dtype):
    """Every byte value 0..255 (so every code of every width, and every pair
    of 4-bit codes) in every position of a slot, against the oracle's grid
    lookup; scales from 1e-30 to 1e30 and both signs of zero in the output."""
    g = torch.Generator()
    g.manual_seed(17)
    perm = torch.cat([torch.randperm(256, generator=g) for _ in range(16)])
    packed = perm.to(torch.uint8).view(torch.int8)
    dt = qa.get_mx_dtype(dtype)
    n = packed.numel() * 8 // dt.bits
    nb = n // 128
    scales = torch.logspace(-30, 30, nb, dtype=torch.float32)
    hseed = 5 if dt.is_hadamard else None
    shape = (n // 128, 128)
    dq = qa.ops._dequant(packed.to(dev()), scales.to(dev()), dt, n, 128, orig_shape=shape, seed=hseed,
                         hadamard_mode="rows")
    rdq = orc.dequant(packed, scales, dtype, n, 128, seed=hseed, orig_shape=shape, hadamard_mode="rows")
    assert _bits_eq(dq, rdq)


@pytest.mark.parametrize("dtype", ["int4dh", "float8dh"])
def test_hadamard_rows128_tiny_values(qa, dtype):
    """Rotated values below 2^-96 take the exactly rounded division path of
    the fused kernels (one wave-wide vote per row group): rows scaled by
    1e-33, all-zero rows and rows mixing both, bit-exact against the oracle."""
    x = _randn((384, 128), 62)
    x[::3] *= 1e-33
    x[1::7] = 0.0
    x[2::5, :64] *= 1e-36
    dt = qa.get_mx_dtype(dtype)
    packed, scales, n = qa.ops.quantize(x.to(dev()), dt, 128, seed=99)
    rp, rs, rn = orc.quantize(x, dtype, 128, seed=99)
    assert _bits_eq(packed, rp) and _bits_eq(scales, rs)
    dq = qa.ops._dequant(packed, scales, dt, n, 128, orig_shape=(384, 128), seed=99, hadamard_mode="rows")
    rdq = orc.dequant(rp, rs, dtype, rn, 128, seed=99, orig_shape=(384, 128), hadamard_mode="rows")
    assert _bits_eq(dq, rdq)
    # quantized scales never go below 1e-12, so caller-supplied tiny scales
    # drive the dequantize side below 2^-96 (every third row of normal codes)
    ts = rs.clone()
    ts[1::3] *= 1e-30
    dq = qa.ops._dequant(packed, ts.to(dev()), dt, n, 128, orig_shape=(384, 128), seed=99, hadamard_mode="rows")
    rdq = orc.dequant(rp, ts, dtype, rn, 128, seed=99, orig_shape=(384, 128), hadamard_mode="rows")
    assert _bits_eq(dq, rdq)
    assert 0 < rdq[rdq != 0].abs().min() < 2.0 ** -96


GEMM_SHAPES = [(512, 512, 512), (256, 384, 200), (100, 256, 130), (33, 128, 17), (8, 640, 1024)]


@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int2d", "int1d"])
@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_qgemm_seeded_vs_oracle(qa, dtype, shape):
    M, K, N = shape
    A = _randn((M, K), 31 + M)
    B = _randn((K, N), 37 + N)
    dt = qa.get_mx_dtype(dtype)
    pa, sa, na = qa.ops.quantize(A.to(dev()), dt, 128)
    pb, sb, nb = qa.ops.quantize(B.to(dev()), dt, 128)
    out_dt = qa.matmul_output_dtype(dt, dt)
    res = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, out_dt.bits, want_c=True, want_acc=True)
    rpa, rsa, _ = orc.quantize(A, dtype, 128)
    rpb, rsb, _ = orc.quantize(B, dtype, 128)
    ac = orc.unpack_auto(rpa, dt.bits, M * K).to(torch.int32)
    bc = orc.unpack_auto(rpb, dt.bits, K * N).to(torch.int32)
    codes, scales, C = orc.qscale_matmul(ac, rsa, bc, rsb, M, K, N, dt.bits, 128, out_dt.bits, return_c=True)
    acc = orc.int_accumulators(ac, bc, M, K, N, 128)
    assert torch.equal(res["acc"].cpu(), acc), "int32 accumulators differ"
    assert _bits_eq(res["c"], C), "fp32 accumulator C differs"
    assert _bits_eq(res["packed"], orc.pack_auto(codes, out_dt.bits))
    assert _bits_eq(res["scales"], scales)


def _large_gemm_vs_oracle(qa, dtype, M, K, N, pa, sa, pb, sb, rows):
    """C and the int32 accumulators of qscale_gemm on the GPU (all three
    kernel variants: C and accumulators, C only, accumulators only) against
    the oracle on a sample of A's rows (output rows are independent).
    Scale arrays whose counts do not match M*KB / KB*N stand for ones, as in
    the reference."""
    bits = qa.get_mx_dtype(dtype).bits
    res = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, bits, 128, 16, want_packed=False, want_c=True, want_acc=True)
    c_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, bits, 128, 16, want_packed=False, want_c=True)
    acc_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, bits, 128, 16, want_packed=False, want_acc=True)
    assert _bits_eq(res["c"], c_only["c"])
    assert torch.equal(res["acc"], acc_only["acc"])
    KB = -(-K // 128)
    ac = orc.unpack_auto(pa.cpu(), bits, M * K).to(torch.int32).reshape(M, K)[rows].reshape(-1)
    bc = orc.unpack_auto(pb.cpu(), bits, K * N).to(torch.int32)
    sa_rows = sa.cpu().reshape(M, KB)[rows].reshape(-1) if sa.numel() == M * KB else sa.cpu()[:1]
    _, _, C = orc.qscale_matmul(ac, sa_rows, bc, sb.cpu(), len(rows), K, N, bits, 128, 16, return_c=True)
    assert _bits_eq(res["c"].cpu()[rows], C.reshape(len(rows), N))
    acc = orc.int_accumulators(ac, bc, len(rows), K, N, 128)
    assert torch.equal(res["acc"].cpu()[:, rows], acc)
    return res


LARGE_GEMM_SHAPES = [(4096, 384, 2048), (4100, 640, 2050), (4100, 640, 2080), (4096, 256, 4096), (4096, 128, 2048),
                     (4096, 1152, 2048)]


@pytest.mark.parametrize("dtype", ["int8d", "int4d"])
@pytest.mark.parametrize("shape", LARGE_GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_qgemm_large_tiles_sampled_rows(qa, dtype, shape):
    """Shapes large enough for the 256x128-tile pipelined kernel (grouped and
    row-major tile orders, one and two K blocks, K blocks past the 3-stage
    ring, ragged M/N).  N % 16 == 0 (int8) or N % 32 == 0 (int4) takes the
    loop that reads both operands as stored (int4 unpacked in its load
    stage); 2050 takes the unpacking pre-pass.  Bitwise against the oracle
    on sampled rows of C and of the int32 accumulators."""
    M, K, N = shape
    dt = qa.get_mx_dtype(dtype)
    A = _randn((M, K), 101 + K)
    B = _randn((K, N), 103 + N)
    pa, sa, _ = qa.ops.quantize(A.to(dev()), dt, 128)
    pb, sb, _ = qa.ops.quantize(B.to(dev()), dt, 128)
    rows = sorted({0, 1, 15, 16, 17, 127, 128, 255, 256, 1000, M // 2, M - 2, M - 1})
    _large_gemm_vs_oracle(qa, dtype, M, K, N, pa, sa, pb, sb, rows)


@pytest.mark.parametrize("dtype", ["int8d", "int4d"])
@pytest.mark.parametrize("shape", [(4096, 384, 2048), (4100, 640, 2048), (4096, 1152, 4096), (4100, 256, 2176)],
                         ids=lambda s: "x".join(map(str, s)))
def test_qgemm_fused_requant(qa, dtype, shape):
    """N a multiple of 128: qa @ qb's int16d (int8d for int4 operands)
    codes and scales come from the GEMM's epilogue (mxtorch.py:1372-1385 on
    each row segment of 128).  They equal the two-pass result (fp32 C, then
    the requantization kernel) bit for bit, with and without the fp32 C
    asked for as well, and the oracle's on sampled rows."""
    M, K, N = shape
    dt = qa.get_mx_dtype(dtype)
    ob = qa.matmul_output_dtype(dt, dt).bits
    pa, sa, _ = qa.ops.quantize(_randn((M, K), 301 + K).to(dev()), dt, 128)
    pb, sb, _ = qa.ops.quantize(_randn((K, N), 303 + N).to(dev()), dt, 128)
    fused = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, ob)
    fused_c = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, ob, want_c=True, want_acc=True)
    # the two-pass path: fp32 C, then the requantization kernel over it
    c_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, ob, want_packed=False, want_c=True)
    pk2, sc2, _ = qa.ops.quantize(c_only["c"], qa.get_mx_dtype(f"int{ob}dv"), 128)
    for r in (fused, fused_c):
        assert _bits_eq(r["packed"], pk2), "packed codes differ from the two-pass result"
        assert _bits_eq(r["scales"], sc2), "scales differ from the two-pass result"
    assert _bits_eq(fused_c["c"], c_only["c"])
    rows = sorted({0, 1, 127, 128, 255, 256, M // 2, M - 1})
    bits = dt.bits
    KB = K // 128
    ac = orc.unpack_auto(pa.cpu(), bits, M * K).to(torch.int32).reshape(M, K)[rows].reshape(-1)
    bc = orc.unpack_auto(pb.cpu(), bits, K * N).to(torch.int32)
    sa_rows = sa.cpu().reshape(M, KB)[rows].reshape(-1)
    codes, scales = orc.qscale_matmul(ac, sa_rows, bc, sb.cpu(), len(rows), K, N, bits, 128, ob)
    got = orc.unpack_auto(fused["packed"].cpu(), ob, M * N).reshape(M, N)[rows]
    assert torch.equal(got.to(torch.int32), codes.reshape(len(rows), N)), "codes differ from the oracle"
    assert _bits_eq(fused["scales"].cpu().reshape(M, N // 128)[rows], scales.reshape(len(rows), N // 128))


@pytest.mark.parametrize("dtype", ["int8d", "int4d"])
def test_qgemm_large_tiles_scale_counts(qa, dtype):
    """Scale arrays of the wrong length mean ones (mxtorch.py:1352-1355) on
    the as-stored loop as well: A's, B's, and both."""
    M, K, N = 4096, 384, 2048
    dt = qa.get_mx_dtype(dtype)
    pa, sa, _ = qa.ops.quantize(_randn((M, K), 211).to(dev()), dt, 128)
    pb, sb, _ = qa.ops.quantize(_randn((K, N), 213).to(dev()), dt, 128)
    rows = [0, 5, 255, 256, 2047, 4095]
    for a_s, b_s in ((sa[:-1], sb), (sa, sb[:-1]), (sa[:-1], sb[:-1])):
        _large_gemm_vs_oracle(qa, dtype, M, K, N, pa, a_s, pb, b_s, rows)


SMALL_GEMM_SHAPES = [(40, 384, 48), (16, 1024, 16), (64, 1152, 96), (1, 128, 32), (72, 256, 4080), (300, 512, 208),
                     (40, 384, 256), (300, 1152, 384), (1, 128, 128)]


@pytest.mark.parametrize("block", [128, 64])
@pytest.mark.parametrize("shape", SMALL_GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_qgemm_small_tiles(qa, shape, block):
    """The one-launch int8 kernel for grids below the CU count, with K blocks
    of 128 and of 64 (the reference's benchmark block): 32x32 tiles,
    K blocks round-robin over 4 waves (9 blocks: a short last round), M and
    N tails inside a tile, N below the tile; C, the int32 accumulators (all
    three kernel variants) and the int16d requantization bitwise against the
    oracle (with and without C and the accumulators), then scale arrays of
    the wrong length as ones."""
    M, K, N = shape
    dt = qa.get_mx_dtype("int8d")
    A = _randn((M, K), 401 + M)
    B = _randn((K, N), 409 + N)
    pa, sa, _ = qa.ops.quantize(A.to(dev()), dt, block)
    pb, sb, _ = qa.ops.quantize(B.to(dev()), dt, block)
    res = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, 8, block, 16, want_c=True, want_acc=True)
    c_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, 8, block, 16, want_packed=False, want_c=True)
    acc_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, 8, block, 16, want_packed=False, want_acc=True)
    rpa, rsa, _ = orc.quantize(A, "int8d", block)
    rpb, rsb, _ = orc.quantize(B, "int8d", block)
    ac = orc.unpack_auto(rpa, 8, M * K).to(torch.int32)
    bc = orc.unpack_auto(rpb, 8, K * N).to(torch.int32)
    codes, scales, C = orc.qscale_matmul(ac, rsa, bc, rsb, M, K, N, 8, block, 16, return_c=True)
    acc = orc.int_accumulators(ac, bc, M, K, N, block)
    assert torch.equal(res["acc"].cpu(), acc), "int32 accumulators differ"
    assert torch.equal(acc_only["acc"].cpu(), acc)
    assert _bits_eq(res["c"], C), "fp32 accumulator C differs"
    assert _bits_eq(c_only["c"], C)
    assert _bits_eq(res["packed"], orc.pack_auto(codes, 16))
    assert _bits_eq(res["scales"], scales)
    pk_only = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, 8, block, 16)
    assert _bits_eq(pk_only["packed"], orc.pack_auto(codes, 16))
    assert _bits_eq(pk_only["scales"], scales)
    for a_s, b_s in ((sa[:-1], sb), (sa, sb[:-1]), (sa[:-1], sb[:-1])):
        got = qa.ops.qscale_gemm(pa, a_s, pb, b_s, M, K, N, 8, block, 16, want_packed=False, want_c=True)
        ra = rsa[:-1] if a_s.numel() < sa.numel() else rsa
        rb = rsb[:-1] if b_s.numel() < sb.numel() else rsb
        _, _, Cw = orc.qscale_matmul(ac, ra, bc, rb, M, K, N, 8, block, 16, return_c=True)
        assert _bits_eq(got["c"], Cw), "C with ones for a mis-sized scale array differs"


def _small_gemm_shapes(seed, count, block=128):
    g = np.random.default_rng(seed)
    kmax = 1536 // block + 1
    return [(int(g.integers(1, 300)), int(g.integers(1, kmax)) * block, int(g.integers(1, 41)) * 16, block)
            for _ in range(count)]


@pytest.mark.parametrize("shape", _small_gemm_shapes(4242, 10) + _small_gemm_shapes(4343, 10, 64),
                         ids=lambda s: "x".join(map(str, s)))
def test_qgemm_small_random_shapes(qa, shape):
    """Seeded random shapes through the one-launch int8 kernel (M 1..299, K a
    multiple of the block (128, or 64: odd multiples included) up to 1536, N
    a multiple of 16 up to 640): C, the int32 accumulators and the int16d
    codes bitwise against the oracle."""
    M, K, N, block = shape
    print(f"small gemm M={M} K={K} N={N} block={block}", flush=True)
    dt = qa.get_mx_dtype("int8d")
    A = _randn((M, K), 503 + M)
    B = _randn((K, N), 509 + N)
    pa, sa, _ = qa.ops.quantize(A.to(dev()), dt, block)
    pb, sb, _ = qa.ops.quantize(B.to(dev()), dt, block)
    res = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, 8, block, 16, want_c=True, want_acc=True)
    rpa, rsa, _ = orc.quantize(A, "int8d", block)
    rpb, rsb, _ = orc.quantize(B, "int8d", block)
    ac = orc.unpack_auto(rpa, 8, M * K).to(torch.int32)
    bc = orc.unpack_auto(rpb, 8, K * N).to(torch.int32)
    codes, scales, C = orc.qscale_matmul(ac, rsa, bc, rsb, M, K, N, 8, block, 16, return_c=True)
    assert torch.equal(res["acc"].cpu(), orc.int_accumulators(ac, bc, M, K, N, block))
    assert _bits_eq(res["c"], C)
    assert _bits_eq(res["packed"], orc.pack_auto(codes, 16))
    assert _bits_eq(res["scales"], scales)


def test_qgemm_int4_tiny_scales(qa):
    """The int4 loop folds the code unpacking's factor 256 into A's scales
    (SA * 2^-8) when that is exact; scales below 2^-118 whose low bits the
    shift would drop switch it to the exact epilogue.  Rows whose scales
    are scaled by 2^-124 and 2^-140 (subnormal), and normal rows, all
    bitwise against the oracle."""
    M, K, N = 4096, 512, 2048
    dt = qa.get_mx_dtype("int4d")
    pa, sa, _ = qa.ops.quantize(_randn((M, K), 221).to(dev()), dt, 128)
    pb, sb, _ = qa.ops.quantize(_randn((K, N), 223).to(dev()), dt, 128)
    ts = sa.clone().view(M, -1)
    ts[1::4] *= 2.0 ** -124
    ts[2::4] *= 2.0 ** -140
    ts = ts.reshape(-1)
    assert ((ts * 2.0 ** -8) * 2.0 ** 8 != ts).any(), "the test needs scales the 2^-8 fold cannot carry"
    rows = [0, 1, 2, 3, 5, 6, 1022, 1023, 4093, 4094]
    _large_gemm_vs_oracle(qa, "int4d", M, K, N, pa, ts, pb, sb, rows)


@pytest.mark.parametrize("dtype", ["int4d", "int8d", "int2d", "float4d", "float8d", "int1d"])
@pytest.mark.parametrize("shape", [(16, 1024, 768), (3, 300, 200), (64, 512, 256), (1, 128, 128)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_linear_vs_oracle(qa, dtype, shape, xdt):
    M, K, N = shape
    W = _randn((N, K), 11 + K, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 13 + M).to(xdt)
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype(dtype), 128)
    y = m(x.to(dev())).cpu()
    wp, ws, _ = orc.linear_from_weight(W, dtype, 128)
    assert _bits_eq(m._mx_weight._mx_packed, wp)
    y_ref = orc.linear_forward(x, wp, ws, dtype, K, N, 128)
    err = (y - y_ref).abs().max().item()
    assert err <= LINEAR_RTOL * y_ref.abs().max().item(), f"max err {err}"


@pytest.mark.parametrize("shape", [(16, 8192, 256), (5, 4096, 384), (16, 2048, 1024), (1, 8192, 128)])
def test_linear_decode_split_k(qa, shape):
    """Shapes whose K is split across workgroups (partials + last-workgroup
    reduction) on the int4 decode path, against the oracle."""
    M, K, N = shape
    W = _randn((N, K), 21 + K, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 23 + M)
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    wp, ws = m._mx_weight._mx_packed.cpu(), m._mx_weight._mx_scales.cpu()
    y_ref = orc.linear_forward(x, wp, ws, "int4d", K, N, 128)
    for _ in range(3):  # repeated calls reuse the self-resetting split-K counters
        y = m(x.to(dev())).cpu()
        err = (y - y_ref).abs().max().item()
        assert err <= LINEAR_RTOL * y_ref.abs().max().item(), f"max err {err}"


@pytest.mark.parametrize("shape,xdt", [
    ((16, 4096, 8192), torch.float32),   # two-block groups, 64-row waves, 8 splits
    ((9, 8192, 8064), torch.float16),    # odd block count: single-block groups, 64-row waves
    ((16, 8160, 8192), torch.float32),   # K not a multiple of the split: a partial last split
    ((4, 1024, 2176), torch.bfloat16),   # 17 blocks, 32-row waves
])
def test_linear_decode_plans(qa, shape, xdt):
    """Each work split of the decode kernel (column-group width, rows per
    wave, split count, partial last split) against the oracle; the fused
    bias equals the bias added afterwards, bit for bit."""
    M, K, N = shape
    W = _randn((N, K), 51 + N, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 53 + M).to(xdt)
    wp, ws, _ = orc.linear_from_weight(W, "int4d", 128)
    dt = qa.get_mx_dtype("int4d")
    wpg, wsg, xg = wp.to(dev()), ws.to(dev()), x.to(dev())
    st = qa.ops.prepack_scales(wsg, K, N, 128)
    y = qa.ops.linear_wq(xg, wpg, wsg, dt, K, N, 128, w_scales_t=st).cpu()
    y_ref = orc.linear_forward(x, wp, ws, "int4d", K, N, 128)
    assert (y - y_ref).abs().max().item() <= LINEAR_RTOL * y_ref.abs().max().item()
    b = _randn((N,), 57)
    yb = qa.ops.linear_wq(xg, wpg, wsg, dt, K, N, 128, bias=b.to(dev()), w_scales_t=st).cpu()
    assert _bits_eq(yb, y + b)


def test_linear_decode_config2_shape(qa):
    """The benchmark shape: x [16, 8192] @ int4d W [8192, 8192]."""
    x = _randn((16, 8192), 2)
    W = _randn((8192, 8192), 3) * 0.02
    lin = torch.nn.Linear(8192, 8192, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    y = m(x.to(dev())).cpu()
    y_ref = orc.linear_forward(x, m._mx_weight._mx_packed.cpu(), m._mx_weight._mx_scales.cpu(), "int4d",
                               8192, 8192, 128)
    assert (y - y_ref).abs().max().item() <= LINEAR_RTOL * y_ref.abs().max().item()


@pytest.mark.parametrize("shape", [(16, 4096, 1024), (7, 2048, 384)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_linear_decode_scale_layouts(qa, shape, xdt):
    """The decode kernel with block-major scales from prepack_scales and with
    the reference-layout scales transposed on the fly: same result, within
    tolerance of the oracle; the prepacked copy is the exact transpose."""
    M, K, N = shape
    W = _randn((N, K), 31 + K, outliers=1e-3, scale=20.0) * 0.02
    x = _randn((M, K), 33 + M).to(xdt)
    wp, ws, _ = orc.linear_from_weight(W, "int4d", 128)
    dt = qa.get_mx_dtype("int4d")
    wpg, wsg, xg = wp.to(dev()), ws.to(dev()), x.to(dev())
    st = qa.ops.prepack_scales(wsg, K, N, 128)
    assert torch.equal(st.cpu(), ws.reshape(K, N // 128).t().contiguous())
    y_pre = qa.ops.linear_wq(xg, wpg, wsg, dt, K, N, 128, w_scales_t=st).cpu()
    y_fly = qa.ops.linear_wq(xg, wpg, wsg, dt, K, N, 128).cpu()
    assert _bits_eq(y_pre, y_fly)
    y_ref = orc.linear_forward(x, wp, ws, "int4d", K, N, 128)
    assert (y_pre - y_ref).abs().max().item() <= LINEAR_RTOL * y_ref.abs().max().item()


def test_linear_prepacked_scales_follow_weight_updates(qa):
    """mx_linear rebuilds its block-major scale copy when the weight's scales
    change in place."""
    K, N = 1024, 256
    W = _randn((N, K), 41) * 0.02
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    x = _randn((4, K), 43).to(dev())
    y1 = m(x).cpu()
    m._mx_weight._mx_scales.mul_(2.0)
    y2 = m(x).cpu()
    assert (y2 - 2.0 * y1).abs().max().item() <= 1e-5 * y1.abs().max().item()


def test_kv_bulk_roundtrip(qa):
    """Config-5 layout at reduced size: fp16 K [B,H,S,D] -> int8dv / int4d per row of D."""
    k = _randn((2, 4, 256, 128), 55).half()
    for dtype in ("int8dv", "int4d"):
        rows = k.reshape(-1, 128)
        packed, scales, n = qa.ops.quantize(rows.to(dev()), qa.get_mx_dtype(dtype), 128)
        rp, rs, _ = orc.quantize(rows, dtype, 128)
        assert _bits_eq(packed, rp) and _bits_eq(scales, rs)
        dq = qa.ops._dequant(packed, scales, qa.get_mx_dtype(dtype), n, 128)
        assert _bits_eq(dq, orc.dequant(rp, rs, dtype, n, 128))


def test_mx_tensor_api(qa):
    x = _randn((64, 256), 1).to(dev())
    q = qa.mx_tensor.quantize(x, qa.get_mx_dtype("int4d"), 128)
    assert q.shape == torch.Size([64, 256]) and q.dim() == 2 and q.numel() == 64 * 256
    assert q.device == x.device and q.requires_grad is False and q.dtype == torch.float32
    assert q.compression_ratio > 7.0
    assert "int4d" in repr(q)
    q2 = q.to("int8d")
    assert q2._mx_dtype.name == "int8d"
    qc = q.cpu()
    assert qc._mx_packed.device.type == "cpu"
    assert _bits_eq(qc.cuda().dequantize(), q.dequantize())
    assert torch.matmul(q, q.t()).shape == torch.Size([64, 64])
    y = qa.mx_matmul(x, x.t().contiguous(), "int8d")
    assert isinstance(y, qa.mx_tensor) and y._mx_dtype.name == "int16d"


def test_to_mx_model(qa):
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.ReLU(), torch.nn.Linear(512, 128)).to(dev())
    x = torch.randn(4, 256, device=dev())
    model.to("int8d")
    assert isinstance(model[0], qa.mx_linear) and isinstance(model[2], qa.mx_linear)
    y = model(x)
    assert y.shape == (4, 128) and torch.isfinite(y).all()


# ---------------------------------------------------------------- long blocks (one workgroup per block)
@pytest.mark.parametrize("name", ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int8dv", "int4dv",
                                  "int16d"])
@pytest.mark.parametrize("block", [264, 512, 1000, 2048, 8192])
@pytest.mark.parametrize("n", [8192 * 3, 8192 * 3 - 100])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_quantize_long_blocks(qa, name, block, n, src):
    g = torch.Generator()
    g.manual_seed(block + n)
    x = torch.randn(n, generator=g)
    x[::997] *= 40.0
    if src == "bf16":
        x = x.bfloat16()
    dt = qa.get_mx_dtype(name)
    packed, scales, nn = qa.ops.quantize(x.to(dev()), dt, block)
    rp, rs, rn = orc.quantize(x, name, block)
    assert nn == rn
    assert _bits_eq(packed, rp), "packed codes differ"
    assert _bits_eq(scales, rs), "scales differ"


@pytest.mark.parametrize("src", [torch.float32, torch.float16])
@pytest.mark.parametrize("bits", [4, 8])
def test_float_bucket_boundaries(qa, src, bits):
    """float4d/float8d codes at every float32 within 2^13 (FP4) or 2^9 (FP8)
    ulps of each grid mid and of each key boundary of the keyed bucket, in
    both signs, plus zeros and subnormals.  Each block of 128 starts with
    1.0, so its scale is 1 and the bucket sees the value itself; codes and
    scales bit-exact against the oracle's bucketize.  fp16 input covers the
    16-bit load path on the values fp16 can hold."""
    n_keys, shift, base = {4: (32, 21, 488), 8: (305, 19, 1728)}[bits]
    mids = orc.float_mids(bits).numpy()
    pm = mids[mids > 0].astype(np.float32)
    bounds = ((np.arange(1, n_keys, dtype=np.uint64) + base) << shift).astype(np.uint32)
    centers = np.concatenate([pm.view(np.uint32), bounds]).astype(np.int64)
    radius = 1 << 13 if bits == 4 else 1 << 9
    off = np.arange(-radius, radius, dtype=np.int64)
    near = (centers[:, None] + off[None, :]).reshape(-1)
    near = near[(near >= 0) & (near <= 0x3F800000)].astype(np.uint32)
    special = np.array([0, 1, 2, 0x007FFFFF, 0x00800000, 0x3F800000], dtype=np.uint32)
    mag = np.concatenate([near, special])
    vals = np.concatenate([mag, mag | np.uint32(0x80000000)]).view(np.float32)
    per = 127
    nblk = -(-vals.size // per)
    body = np.zeros(nblk * per, dtype=np.float32)
    body[:vals.size] = vals
    x = np.concatenate([np.ones((nblk, 1), dtype=np.float32), body.reshape(nblk, per)], axis=1)
    xin = torch.from_numpy(x).to(src)
    name = f"float{bits}d"
    dt = qa.get_mx_dtype(name)
    packed, scales, n = qa.ops.quantize(xin.to(dev()), dt, 128)
    rp, rs, rn = orc.quantize(xin, name, 128)
    assert n == rn
    assert _bits_eq(scales, rs), "scales differ"
    assert _bits_eq(packed, rp), "packed codes differ"
