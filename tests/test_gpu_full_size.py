"""GPU parity at the benchmark's full sizes and at the empty edge.

Blocks of the quantizer are independent and rows of the packed GEMM are
independent, so a full-size GPU result is checked bitwise against the CPU
oracle on a seeded sample of blocks (rows), plus whole-tensor invariants
that need no oracle:
  * config 4 (2^28 fp32 viewed as [2^21, 128]): every int dtype's codes
    reach +-q in every non-zero block and dequantize(quantize(x)) stays
    within half a step, |x - x_dq| <= s/2 (int widths 2-8);
  * config 5 (fp16 K [8,32,4096,128]): int8dv / int4d per row;
  * config 3 (8192^3 int8d GEMM): sampled rows of C;
  * empty inputs give empty outputs, as in the reference.
"""
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


def _sample_blocks(nb, count, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, nb, (count,), generator=g)
    return torch.unique(torch.cat([idx, torch.tensor([0, nb - 1])]))


def _block_codes(packed, bits, blocks, block=128):
    """Packed bytes of the given blocks (bits in {1,2,4,8}), as a flat uint8 tensor."""
    per = block * bits // 8
    p = packed.view(torch.uint8).reshape(-1, per)
    return p[blocks.to(packed.device)].cpu().reshape(-1)


@pytest.fixture(scope="module")
def config4_x():
    n = 1 << 28
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(n, generator=g, device="cuda")
    mask = torch.rand(n, generator=torch.Generator(device="cuda").manual_seed(8), device="cuda") < 1e-3
    x[mask] *= 50
    del mask
    return x.view(1 << 21, 128)


@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int4dh"])
def test_config4_full_size_sampled_blocks(qa, config4_x, dtype):
    x = config4_x
    dt = qa.get_mx_dtype(dtype)
    seed = 1534857261 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(x, dt, 128, seed=seed)
    nb = x.shape[0]
    assert n == x.numel() and scales.numel() == nb
    blocks = _sample_blocks(nb, 2048, 11 + dt.bits)
    xs = x[blocks.to(x.device)].cpu()
    rp, rs, _ = orc.quantize(xs, dtype, 128, seed=seed)
    assert _bits_eq(_block_codes(packed, dt.bits, blocks), rp.view(torch.uint8))
    assert _bits_eq(scales[blocks.to(x.device)], rs)
    dq = qa.ops._dequant(packed, scales, dt, n, 128, orig_shape=tuple(x.shape), seed=seed, hadamard_mode="rows")
    rdq = orc.dequant(rp, rs, dtype, xs.numel(), 128, seed=seed, orig_shape=tuple(xs.shape), hadamard_mode="rows")
    assert _bits_eq(dq.view(nb, 128)[blocks.to(x.device)], rdq.view(-1, 128))
    if not dt.is_float and not dt.is_hadamard and dt.bits > 1:
        # whole tensor: |x - dequant| <= s/2 in every block, up to the few fp32
        # roundings of inv = fl(fl(1/a)*q), fl(x*inv) and RN(code*s) (< 1e-4 s)
        err = (x - dq.view(nb, 128)).abs().amax(dim=1)
        assert bool((err <= scales * (0.5 + 1e-4)).all())
    del packed, scales, dq
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", ["int8dv", "int4d"])
@pytest.mark.parametrize("which", ["K", "V"])
def test_config5_kv_full_size_sampled_rows(qa, dtype, which):
    """Config 5: fp16 K and V [8, 32, 4096, 128] (the seeds bench.py uses),
    quantized per row of head_dim and dequantized; sampled blocks bitwise
    against the oracle."""
    g = torch.Generator(device="cuda").manual_seed(9 if which == "K" else 10)
    t = torch.randn(8, 32, 4096, 128, generator=g, device="cuda").half()
    rows = t.view(-1, 128)
    dt = qa.get_mx_dtype(dtype)
    packed, scales, n = qa.ops.quantize(rows, dt, 128)
    nb = rows.shape[0]
    blocks = _sample_blocks(nb, 2048, 21 if which == "K" else 23)
    ks = rows[blocks.to(rows.device)].cpu()
    rp, rs, _ = orc.quantize(ks, dtype, 128)
    assert _bits_eq(_block_codes(packed, dt.bits, blocks), rp.view(torch.uint8))
    assert _bits_eq(scales[blocks.to(rows.device)], rs)
    dq = qa.ops._dequant(packed, scales, dt, n, 128)
    assert _bits_eq(dq.view(nb, 128)[blocks.to(rows.device)], orc.dequant(rp, rs, dtype, ks.numel(), 128).view(-1, 128))


@pytest.mark.parametrize("dtype", ["int8d", "int4d"])
def test_config3_gemm_full_size_sampled_rows(qa, dtype):
    """8192^3 as bench.py runs it (config 3 for int8d; the int4d GEMM
    extra): sampled rows of the fp32 C bitwise against the oracle."""
    M = K = N = 8192
    dt = qa.get_mx_dtype(dtype)
    A = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(5), device="cuda")
    B = torch.randn(K, N, generator=torch.Generator(device="cuda").manual_seed(6), device="cuda")
    pa, sa, _ = qa.ops.quantize(A, dt, 128)
    pb, sb, _ = qa.ops.quantize(B, dt, 128)
    del A, B
    res = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, 16, want_packed=False, want_c=True)
    rows = sorted({0, 1, 127, 128, 255, 4095, 4096, 8190, 8191})
    ac = orc.unpack_auto(pa.cpu(), dt.bits, M * K).to(torch.int32).view(M, K)[rows].reshape(-1)
    bc = orc.unpack_auto(pb.cpu(), dt.bits, K * N).to(torch.int32)
    sa_rows = sa.view(M, 64)[rows].cpu().reshape(-1)
    _, _, C = orc.qscale_matmul(ac, sa_rows, bc, sb.cpu(), len(rows), K, N, dt.bits, 128, 16, return_c=True)
    assert _bits_eq(res["c"][rows], C.view(len(rows), N))
    del res
    # qa @ qb's packed output (int16d / int8d), requantized in the GEMM's epilogue
    ob = qa.matmul_output_dtype(dt, dt).bits
    pk = qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, dt.bits, 128, ob)
    codes, scales = orc.qscale_matmul(ac, sa_rows, bc, sb.cpu(), len(rows), K, N, dt.bits, 128, ob)
    got = orc.unpack_auto(pk["packed"].cpu(), ob, M * N).view(M, N)[rows].to(torch.int32)
    assert torch.equal(got, codes.view(len(rows), N))
    assert _bits_eq(pk["scales"].cpu().view(M, N // 128)[rows], scales.view(len(rows), N // 128))
    del pk, pa, pb
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", ["int8d", "int4d", "int1d", "float4d", "int8dv", "int4dh"])
def test_empty_inputs(qa, dtype):
    dt = qa.get_mx_dtype(dtype)
    seed = 5 if dt.is_hadamard else None
    packed, scales, n = qa.ops.quantize(torch.empty(0, device=dev()), dt, 128, seed=seed)
    rp, rs, rn = orc.quantize(torch.empty(0), dtype, 128, seed=seed)
    assert n == rn == 0 and packed.numel() == rp.numel() == 0 and scales.numel() == rs.numel() == 0
    assert packed.dtype == rp.dtype
    dq = qa.ops._dequant(packed, scales, dt, 0, 128, seed=seed)
    assert dq.numel() == 0


def test_empty_batch_linear_and_gemm(qa):
    lin = torch.nn.Linear(256, 128, bias=False)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    y = m(torch.empty(0, 256, device=dev()))
    assert tuple(y.shape) == (0, 128)
    dt = qa.get_mx_dtype("int8d")
    pb, sb, _ = qa.ops.quantize(torch.randn(256, 128, device=dev()), dt, 128)
    res = qa.ops.qscale_gemm(torch.empty(0, dtype=torch.int8, device=dev()), torch.empty(0, device=dev()), pb, sb,
                             0, 256, 128, 8, 128, 16, want_c=True)
    assert res["packed"].numel() == 0 and res["scales"].numel() == 0 and tuple(res["c"].shape) == (0, 128)


@pytest.mark.parametrize("dtype,src,n", [
    ("float4d", torch.float32, (1 << 28) + 3 * 128 + 5),   # 1-2 steps per workgroup (384 per CU)
    ("float8d", torch.float32, (1 << 28) + 7 * 128 + 100),  # 2-3 steps (192 per CU): pairs and an odd step
    ("int4d", torch.float16, (1 << 28) + 128 + 1),          # 2 steps (128 per CU), a pair
    ("int8dv", torch.float16, (1 << 28) + 9 * 128),         # 4 steps (64 per CU), pairs
    ("int4dh", torch.float32, (1 << 29) + 5 * 128),          # 2 steps (256 per CU)
])
def test_quantize_steps_match_chunked(qa, dtype, src, n):
    """The quantizers walk a capped grid in steps of whole blocks: steps that
    end inside the data load and store through buffer resources with the
    loop unrolled twice, the steps reaching the end check each lane.  Large
    ragged tensors (several steps per workgroup, odd and even counts, a
    tail) must give the codes and scales of the same tensor quantized in
    2^24-element chunks (one step per workgroup, blocks being independent),
    every block bitwise."""
    g = torch.Generator(device="cuda").manual_seed(n % 1000)
    x = torch.randn(n, generator=g, device="cuda").to(src)
    dt = qa.get_mx_dtype(dtype)
    seed = 99 if dt.is_hadamard else None
    if dt.is_hadamard:
        # the rotation runs along the last dimension: rows of 128, as config 4
        x = x[: n - n % 128].reshape(-1, 128)
        n = x.numel()
    packed, scales, nn = qa.ops.quantize(x, dt, 128, seed=seed)
    assert nn == n
    chunk = 1 << 24
    parts_p, parts_s = [], []
    for lo in range(0, n, chunk):
        part = x[lo // 128: (lo + chunk) // 128] if dt.is_hadamard else x[lo: lo + chunk]
        p, s, _ = qa.ops.quantize(part, dt, 128, seed=seed)
        parts_p.append(p.view(torch.uint8).reshape(-1))
        parts_s.append(s.reshape(-1))
    cp = torch.cat(parts_p)
    cs = torch.cat(parts_s)
    pw = packed.view(torch.uint8).reshape(-1)
    assert pw.numel() == cp.numel() and scales.numel() == cs.numel()
    assert torch.equal(scales.reshape(-1).view(torch.int32), cs.view(torch.int32)), "scales differ"
    bad = (pw != cp).nonzero()
    assert bad.numel() == 0, f"{bad.numel()} packed bytes differ, first at {int(bad[0])}"
    del x, packed, scales, cp, cs, pw
    torch.cuda.empty_cache()
