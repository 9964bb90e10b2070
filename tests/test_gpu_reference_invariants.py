"""The reference's own checks of this path (mxtorch_test.py), run against the
HIP path.  They are loose invariants and statistics, not bit-level pins
(the parity modules pin bits against the oracle and golden vectors); each
test cites the reference test it mirrors.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qtpytorch_amd
    return qtpytorch_amd


def dev():
    return torch.device("cuda:0")


def _x(shape, seed=0):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(*shape, generator=g)


def _snr_db(x, y):
    return 10.0 * math.log10(x.pow(2).mean().item() / max((x - y).pow(2).mean().item(), 1e-30))


def test_snr_ordering_and_floors(qa):
    """SNR int8 > int4 > int2 (mxtorch_test.py:313-320); int8 > 20 dB and
    int4 > 5 dB (mxtorch_test.py:1166-1182)."""
    x = _x((256, 512), 1).to(dev())
    snr = {}
    for name in ("int8d", "int4d", "int2d"):
        q = qa.mx_tensor.quantize(x, qa.get_mx_dtype(name), 128)
        snr[name] = _snr_db(x.cpu(), q.dequantize().cpu())
    assert snr["int8d"] > snr["int4d"] > snr["int2d"]
    assert snr["int8d"] > 20.0 and snr["int4d"] > 5.0


def test_scale_counts_and_int8_scale(qa):
    """One scale per block (mxtorch_test.py:1319-1328, 4274-4281); int8
    scale = absmax / 127 within 1e-4 (mxtorch_test.py:4283-4295)."""
    x = _x((64, 1000), 2).to(dev())
    for block in (32, 64, 128, 256):
        q = qa.mx_tensor.quantize(x, qa.get_mx_dtype("int8d"), block)
        assert q._mx_scales.numel() == -(-x.numel() // block)
    q = qa.mx_tensor.quantize(x, qa.get_mx_dtype("int8d"), 128)
    flat = x.reshape(-1).cpu()
    pad = q._mx_scales.numel() * 128 - flat.numel()
    amax = torch.cat([flat, flat.new_zeros(pad)]).reshape(-1, 128).abs().amax(dim=1)
    assert torch.allclose(q._mx_scales.cpu(), amax / 127.0, rtol=1e-4, atol=0)


def test_zeros_and_ones(qa):
    """Zeros dequantize to zeros within 1e-5, ones within 0.5
    (mxtorch_test.py:1274-1284, there for int4d).  int1d dequantizes a zero
    to +s = 1e-12 (code 0 is +s, mxtorch.py:1553-1557); the other widths give
    exact zeros."""
    for name in ("int8d", "int4d", "int2d", "int1d", "float4d", "float8d"):
        dt = qa.get_mx_dtype(name)
        z = qa.mx_tensor.quantize(torch.zeros(4, 256, device=dev()), dt, 128).dequantize()
        assert torch.allclose(z.cpu(), torch.zeros(4, 256), atol=1e-5)
        if name != "int1d":
            assert torch.equal(z.cpu(), torch.zeros(4, 256))
        o = qa.mx_tensor.quantize(torch.ones(4, 256, device=dev()), dt, 128).dequantize()
        assert (o.cpu() - 1.0).abs().max().item() <= 0.5


def test_negation_exact(qa):
    """-q dequantizes to exactly -(q.dequantize()) (mxtorch_test.py:3303-3314)."""
    q = qa.mx_tensor.quantize(_x((32, 128), 3).to(dev()), qa.get_mx_dtype("int8d"), 128)
    assert torch.equal((-q).dequantize().cpu(), -q.dequantize().cpu())


def test_fp4_representable_and_fp8_error(qa):
    """FP4 grid values survive within 1.0 (mxtorch_test.py:3412-3423); FP8
    relative RMSE < 0.25 (mxtorch_test.py:3425-3434)."""
    vals = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.5, -1.0, -2.0, -6.0] * 16)
    q4 = qa.mx_tensor.quantize(vals.to(dev()), qa.get_mx_dtype("float4d"), 64)
    assert (q4.dequantize().cpu() - vals).abs().max().item() <= 1.0
    x = _x((128, 256), 4).to(dev())
    q8 = qa.mx_tensor.quantize(x, qa.get_mx_dtype("float8d"), 128).dequantize()
    rel = ((q8 - x).pow(2).mean().sqrt() / x.pow(2).mean().sqrt()).item()
    assert rel < 0.25


def test_int8_matmul_error(qa):
    """int8 packed matmul within RMSE/sigma < 0.5 of A.dq @ B.dq
    (mxtorch_test.py:3368-3380); shapes of `@` (mxtorch_test.py:142-146)."""
    A, B = _x((64, 256), 5).to(dev()), _x((256, 96), 6).to(dev())
    d8 = qa.get_mx_dtype("int8d")
    qa_, qb = qa.mx_tensor.quantize(A, d8, 128), qa.mx_tensor.quantize(B, d8, 128)
    # the GEMM reads B's flat scales as [K/128, N] (mxtorch.py:1352-1355), so it
    # differs from the product of the dequantized operands; the bound holds anyway
    C = (qa_ @ qb)
    assert tuple(C.shape) == (64, 96) and C._mx_dtype.name == "int16d"
    ref = qa_.dequantize() @ qb.dequantize()
    err = (C.dequantize() - ref).pow(2).mean().sqrt().item() / ref.std().item()
    assert err < 0.5


def test_flatten_protocol_and_device_round_trip(qa):
    """__tensor_flatten__ / __tensor_unflatten__ round trip (mxtorch_test.py:4146-4196)
    and CPU -> CUDA -> CPU exactness of the packed data (mxtorch_test.py:4301-4316)."""
    q = qa.mx_tensor.quantize(_x((16, 384), 7).to(dev()), qa.get_mx_dtype("int4d"), 128)
    names, meta = q.__tensor_flatten__()
    assert names == ["_mx_packed", "_mx_scales"]
    r = qa.mx_tensor.__tensor_unflatten__({n: getattr(q, n) for n in names}, meta, None, None)
    assert torch.equal(r.dequantize().cpu(), q.dequantize().cpu())
    c = q.cpu()
    assert c._mx_packed.device.type == "cpu"
    back = c.cuda()
    assert torch.equal(back._mx_packed.cpu(), q._mx_packed.cpu())
    assert torch.equal(back._mx_scales.cpu(), q._mx_scales.cpu())
    assert torch.equal(back.dequantize().cpu(), q.dequantize().cpu())


def test_module_shapes(qa):
    """mx_linear and _QGemmSTE shapes and types (mxtorch_test.py:156-161,
    3452-3463, 3840-3858), int4dh / int4dv round trips (mxtorch_test.py:529-542),
    KV cache shapes (mxtorch_test.py:432-449)."""
    lin = torch.nn.Linear(64, 32).to(dev())
    m = qa.mx_linear.from_linear(lin, qa.get_mx_dtype("int4d"))
    y = m(torch.randn(4, 64, device=dev()))
    assert y.shape == (4, 32) and y.dtype == torch.float32
    a = torch.randn(8, 128, device=dev(), requires_grad=True)
    b = torch.randn(128, 16, device=dev(), requires_grad=True)
    out = qa._QGemmSTE.apply(a, b, qa.get_mx_dtype("int8d"), 128)
    assert out.shape == (8, 16)
    out.sum().backward()
    assert a.grad.shape == a.shape and b.grad.shape == b.shape
    x = torch.randn(64, 128, device=dev())
    for name in ("int4dh", "int4dv"):
        r = qa.mx_tensor.quantize(x, qa.get_mx_dtype(name), 128).dequantize()
        assert r.shape == x.shape and _snr_db(x.cpu(), r.cpu()) > 5.0
    cache = qa.kv_cache_quantizer(n_heads=4, head_dim=64, dtype="int8d")
    for _ in range(3):
        cache.append_kv(torch.randn(2, 4, 1, 64, device=dev()), torch.randn(2, 4, 1, 64, device=dev()))
    K, V = cache.get()
    assert K.shape == (2, 4, 3, 64) and V.shape == (2, 4, 3, 64)
