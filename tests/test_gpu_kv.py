"""GPU parity of the KV-cache ring (kv_cache_quantizer, mxtorch.py:2998-3090)
against the CPU oracle's per-step restatement (oracle.kv_append / kv_get),
which the reference's own golden KV fixtures pin for int8d, int4d and
int8dv (tests/test_oracle_golden.py).  Codes, scales, zero points and the
dequantized history must be bitwise equal."""
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


def _steps(T, B, H, D, seed, dtype=torch.float32, layout="bhtd"):
    g = torch.Generator()
    g.manual_seed(seed)
    out = []
    for _ in range(T):
        shape = (B, H, 1, D) if layout == "bhtd" else (B, 1, H, D)
        k = torch.randn(*shape, generator=g) * 3.0
        v = torch.randn(*shape, generator=g) * 2.0 + 0.5
        # outliers and exact zeros in a few places
        k.view(-1)[:: 97] *= 40.0
        v.view(-1)[5:: 131] = 0.0
        out.append((k.to(dtype), v.to(dtype)))
    return out


def _check(qa, cache, steps, dtype, D, H, asym):
    ref = [orc.kv_append(k, v, dtype, D, asymmetric_v=asym) for k, v in steps]
    kq, vq = cache.get_quantized()
    assert len(kq) == len(ref) == cache.seq_len
    for t, (rk, rv, rz) in enumerate(ref):
        assert _bits_eq(kq[t]._mx_packed, rk[0]), f"K codes of step {t}"
        assert _bits_eq(kq[t]._mx_scales, rk[1]), f"K scales of step {t}"
        assert _bits_eq(vq[t]._mx_packed, rv[0]), f"V codes of step {t}"
        assert _bits_eq(vq[t]._mx_scales, rv[1]), f"V scales of step {t}"
    K, V = cache.get()
    if dtype.endswith("h"):
        # mx_tensor.dequantize unrotates each row of D here (the inverse of the
        # rotation quantize applied), where the reference unrotates the whole
        # flattened step (mxtorch.py:1582-1595): the oracle's "rows" mode
        rows = ref[0][0][2] // D
        deq = lambda q: orc.dequant(q[0], q[1], dtype, q[2], D, orig_shape=(rows, D),
                                    hadamard_mode="rows").reshape(rows, D)
        RK = torch.stack([deq(rk) for rk, _, _ in ref], dim=1)
        RV = torch.stack([deq(rv) for _, rv, _ in ref], dim=1)
        if asym:
            RV = RV + torch.stack([rz for _, _, rz in ref], dim=1).unsqueeze(-1)
        RK, RV = RK.reshape(-1, H, len(ref), D), RV.reshape(-1, H, len(ref), D)
    else:
        RK, RV = orc.kv_get(ref, dtype, D, H)
    assert K.shape == RK.shape and V.shape == RV.shape
    assert _bits_eq(K, RK), "K history"
    assert _bits_eq(V, RV), "V history"


FUSED = ["int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int8dv", "int4dv", "float4dv"]


@pytest.mark.parametrize("asym", [True, False], ids=["asym", "sym"])
@pytest.mark.parametrize("xdt", [torch.float16, torch.float32, torch.bfloat16], ids=["f16", "f32", "bf16"])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", FUSED)
def test_kv_ring_fused_vs_oracle(qa, dtype, D, xdt, asym):
    """One fused launch per step; B*H = 6 rows (not a multiple of the rows a
    workgroup takes), 5 steps."""
    B, H, T = 2, 3, 5
    steps = _steps(T, B, H, D, 7 + D + len(dtype), xdt)
    cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype=dtype, asymmetric_v=asym)
    for k, v in steps:
        cache.append_kv(k.to(dev()), v.to(dev()))
    _check(qa, cache, steps, dtype, D, H, asym)


@pytest.mark.parametrize("dtype,D", [("int4dh", 128), ("int3d", 128), ("int8d", 96), ("float8dh", 64)])
def test_kv_ring_generic_path_vs_oracle(qa, dtype, D):
    """Dtypes and head sizes outside the fused kernels: the regular quantizer
    writes the same ring; get() dequantizes slot by slot."""
    B, H, T = 2, 2, 4
    steps = _steps(T, B, H, D, 31 + D)
    cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype=dtype)
    for k, v in steps:
        cache.append_kv(k.to(dev()), v.to(dev()))
    _check(qa, cache, steps, dtype, D, H, True)


def test_kv_ring_layout_b1hd(qa):
    """[B, 1, H, D] steps flatten in their own row-major order (mxtorch.py:3055)."""
    B, H, D, T = 2, 4, 128, 3
    steps = _steps(T, B, H, D, 5, torch.float16, layout="b1hd")
    cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype="int4d")
    for k, v in steps:
        cache.append_kv(k.to(dev()), v.to(dev()))
    _check(qa, cache, steps, "int4d", D, H, True)


def test_kv_ring_growth_and_eviction(qa):
    """100 steps into a cache of max_seq_len 70: the ring grows past its first
    64 slots, then evicts FIFO; the live window is the last 70 steps."""
    B, H, D, T, cap = 1, 4, 64, 100, 70
    steps = _steps(T, B, H, D, 11, torch.float16)
    cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype="int8dv", max_seq_len=cap)
    for t, (k, v) in enumerate(steps):
        cache.append_kv(k.to(dev()), v.to(dev()))
        assert cache.seq_len == min(t + 1, cap)
    _check(qa, cache, steps[-cap:], "int8dv", D, H, True)
    per_step = 2 * (H * D + 4 * H) + 4 * H
    assert cache.memory_bytes() == cap * per_step
    assert cache.compression_vs_fp16() == pytest.approx(cap * 2 * H * D * 2 / (cap * per_step))


def test_kv_ring_reset_and_errors(qa):
    H, D = 2, 128
    cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype="int4d")
    with pytest.raises(RuntimeError):
        cache.get()
    assert cache.get_quantized() == ([], [])
    steps = _steps(2, 3, H, D, 3)
    for k, v in steps:
        cache.append_kv(k.to(dev()), v.to(dev()))
    with pytest.raises(ValueError):  # another batch size within one request
        cache.append_kv(torch.zeros(1, H, 1, D, device=dev()), torch.zeros(1, H, 1, D, device=dev()))
    cache.reset()
    assert cache.seq_len == 0 and cache.memory_bytes() == 0
    steps = _steps(3, 1, H, D, 4)  # a new request with another batch size
    for k, v in steps:
        cache.append_kv(k.to(dev()), v.to(dev()))
    _check(qa, cache, steps, "int4d", D, H, True)
    with pytest.raises(Exception):
        cache.append_kv(torch.zeros(1, H, 1, D), torch.zeros(1, H, 1, D))  # CPU tensors: GPU only


@pytest.mark.parametrize("dtype", ["float4dv", "float8dv"])
def test_quantize_float_vector_dtypes(qa, dtype):
    """The 'v' rule on float dtypes rounds to integers clamped at max_val
    (6, 448) and packs them as ints (mxtorch.py:1739-1752); dequantize reads
    them as grid indices (mxtorch.py:1558-1569)."""
    x = torch.randn(64, 256) * 4.0
    x.view(-1)[::53] *= 100.0
    dt = qa.get_mx_dtype(dtype)
    p, s, n = qa.ops.quantize(x.to(dev()), dt, 128)
    rp, rs, rn = orc.quantize(x, dtype, 128)
    assert n == rn
    assert _bits_eq(p, rp) and _bits_eq(s, rs)
    dq = qa.ops._dequant(p, s, dt, n, 128)
    assert _bits_eq(dq, orc.dequant(rp, rs, dtype, n, 128))

