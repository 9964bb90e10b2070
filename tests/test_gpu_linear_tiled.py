"""The tiled int4 decode path (mxk_linear_prepack_weight + mxk_linear_wq_tiled),
the kernel mx_linear.forward (mxtorch.py:7454-7473) runs for x of at most 16
rows.

  * the library's tiled copy equals the CPU restatement of the layout byte
    for byte (tests/test_cpu_tiled_layout.py pins that restatement against
    the kernel's operand construction);
  * y = x.float() @ dequant(W) within 1e-3 of the oracle (per output row) for
    x in float32 / float16 / bfloat16, M in 1..16, with and without bias,
    and K that is or is not a multiple of a split (2048 rows), including a
    single split and splits whose last waves lie past K;
  * the same products through mxk_linear_wq (no tiled copy) agree within
    the same bar;
  * two streams at once, each with its own workspace, give the results of
    the calls alone, bit for bit;
  * shapes the tiled kernel does not take fall back to mxk_linear_wq.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G
from tests.test_cpu_tiled_layout import tile_w4

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


def _randn(shape, seed, outliers=0.0, scale=20.0):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        m = torch.rand(*shape, generator=g) < outliers
        x[m] *= scale
    return x


def _rowwise_ok(y, y_ref):
    err = (y - y_ref).abs().amax(dim=1)
    lim = RTOL * y_ref.abs().amax(dim=1)
    return bool((err <= lim).all()), (err / lim.clamp_min(1e-300)).max().item()


def _weights(qa, K, N, seed, name="int4d"):
    W = _randn((N, K), seed, outliers=1e-3) * 0.02
    wp, ws, _ = orc.linear_from_weight(W, name, 128)
    wpg, wsg = wp.to(dev()), ws.to(dev())
    return wp, ws, wpg, wsg, qa.ops.prepack_scales(wsg, K, N, 128), qa.ops.prepack_weight(wpg, K, N, 128)


@pytest.mark.parametrize("K,N", [(32, 128), (2080, 384), (4096, 1024)])
def test_prepack_weight_matches_layout(qa, K, N):
    wp = torch.randint(0, 256, (K * N // 2,), dtype=torch.uint8, generator=torch.Generator().manual_seed(K + N))
    tiled = qa.ops.prepack_weight(wp.to(dev()), K, N, 128).cpu().numpy()
    assert np.array_equal(tiled, tile_w4(wp.numpy(), K, N))


def test_prepack_weight_config2_sampled(qa):
    """8192 x 8192: the chunks of a few blocks and steps against the layout."""
    K = N = 8192
    wp = torch.randint(0, 256, (K * N // 2,), dtype=torch.uint8, generator=torch.Generator().manual_seed(7))
    tiled = qa.ops.prepack_weight(wp.to(dev()), K, N, 128).cpu().numpy()
    rows = wp.numpy().reshape(K, N // 2)
    for nb in (0, 17, 63):
        for ks in (0, 100, 255):
            sub = np.ascontiguousarray(rows[ks * 32:(ks + 1) * 32, nb * 64:(nb + 1) * 64]).reshape(-1)
            want = tile_w4(sub, 32, 128)
            c = (nb * (K // 32) + ks) * 2048
            assert np.array_equal(tiled[c:c + 2048], want), f"chunk nb={nb} ks={ks}"


CASES = [
    # M, K, N, x dtype, bias
    (16, 8192, 8192, torch.float32, False),
    (16, 8192, 8192, torch.bfloat16, True),
    (1, 4096, 1024, torch.float32, True),
    (5, 2080, 384, torch.float16, False),      # the last split's waves lie past K
    (16, 2048, 256, torch.bfloat16, False),    # one split of 16 x 128 rows
    (9, 96, 128, torch.float32, True),         # short waves, one split
    (16, 12288, 640, torch.float32, False),
    (40, 2048, 512, torch.float32, True),      # more than 16 rows: the MFMA kernel on the tiled copy
    (300, 1024, 256, torch.bfloat16, False),
]


@pytest.mark.parametrize("name", ["int4d", "float4d"])
@pytest.mark.parametrize("M,K,N,xdt,use_bias", CASES)
def test_tiled_linear_vs_oracle(qa, M, K, N, xdt, use_bias, name):
    """int4 and FP4 codes (the same tiled layout) through the tiled decode
    kernel (at most 16 rows) and the MFMA kernel on the tiled copy (more),
    and the same product from the packed codes."""
    print(f"tiled {name} M={M} K={K} N={N} {xdt} bias={use_bias}", flush=True)
    dt = qa.get_mx_dtype(name)
    wp, ws, wpg, wsg, st, wt = _weights(qa, K, N, 31 + K % 97, name)
    x = _randn((M, K), 37 + M).to(xdt)
    bias = _randn((N,), 41) if use_bias else None
    y = qa.ops.linear_wq(x.to(dev()), wpg, wsg, dt, K, N, 128, bias=None if bias is None else bias.to(dev()),
                         w_scales_t=st, w_tiled=wt).cpu()
    y_ref = orc.linear_forward(x, wp, ws, name, K, N, 128)
    if bias is not None:
        y_ref = y_ref + bias
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"
    y_plain = qa.ops.linear_wq(x.to(dev()), wpg, wsg, dt, K, N, 128,
                               bias=None if bias is None else bias.to(dev()), w_scales_t=st).cpu()
    ok, worst = _rowwise_ok(y_plain, y_ref)
    assert ok, f"untiled path: worst row error {worst:.3g} x the bar"


def test_mx_linear_keeps_one_tiled_copy(qa):
    """mx_linear holds an eligible int4 weight as its tiled copy only, from
    the first forward (any row count) on: one copy of the weight's bytes.
    The packed codes come back bit for bit on demand (dequantize,
    state_dict), the decode and MFMA kernels read the tiled copy, an
    in-place copy_ turns the weight back to packed storage (and the next
    forward tiles the new codes), and tiled_decode = False keeps the packed
    codes."""
    K, N = 1024, 256
    W = _randn((N, K), 61) * 0.03
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    wp, ws, _ = orc.linear_from_weight(W, "int4d", 128)
    w = m._mx_weight
    for M in (4, 40):
        x = _randn((M, K), 63 + M)
        y = m(x.to(dev())).cpu()
        assert w.__dict__["_mx_tiled"] is not None and w.__dict__["_mx_packed_store"] is None
        assert _rowwise_ok(y, orc.linear_forward(x, wp, ws, "int4d", K, N, 128))[0]
    assert w.nbytes_packed == K * N // 2 + ws.numel() * 4          # one copy of the codes
    assert G.bits_equal(w._mx_packed.cpu(), wp)                       # rebuilt on demand
    assert w._mx_packed.dtype == wp.dtype
    assert G.bits_equal(w.dequantize().cpu().reshape(-1), orc.dequant(wp, ws, "int4d", K * N, 128))
    sd = {k: v for k, v in m.state_dict().items()}
    m2 = qa.mx_linear.from_linear(torch.nn.Linear(K, N, bias=False).to(dev()), qa.get_mx_dtype("int4d"), 128)
    m2.load_state_dict(sd)
    x = _randn((9, K), 65).to(dev())
    assert G.bits_equal(m2(x).cpu(), m(x).cpu())
    # an in-place change of the codes
    W2 = _randn((N, K), 67) * 0.03
    q2 = qa.mx_tensor.quantize(W2.t().contiguous().to(dev()), qa.get_mx_dtype("int4d"), 128)
    w.copy_(q2)
    assert w.__dict__["_mx_tiled"] is None
    wp2, ws2, _ = orc.linear_from_weight(W2, "int4d", 128)
    y2 = m(x).cpu()
    assert w.__dict__["_mx_tiled"] is not None
    assert _rowwise_ok(y2, orc.linear_forward(x.cpu(), wp2, ws2, "int4d", K, N, 128))[0]
    m3 = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("int4d"), 128)
    m3.tiled_decode = False
    m3(x)
    assert m3._mx_weight.__dict__["_mx_tiled"] is None


@pytest.mark.parametrize("K,N", [(32, 128), (96, 384), (1024, 256), (8192, 8192)])
def test_unpack_weight_inverts_prepack(qa, K, N):
    """mxk_linear_unpack_weight gives back the packed bytes of any codes."""
    g = torch.Generator()
    g.manual_seed(K + N)
    pk = torch.randint(0, 256, (K * N // 2,), generator=g, dtype=torch.uint8).to(dev())
    t = qa.ops.prepack_weight(pk, K, N, 128)
    assert not torch.equal(t, pk) or K * N <= 4096
    assert torch.equal(qa.ops.unpack_weight(t, K, N, 128), pk)


def test_tiled_two_streams_concurrently(qa):
    dt = qa.get_mx_dtype("int4d")
    cases = []
    for (M, K, N, seed) in ((16, 8192, 4096, 91), (7, 4096, 8192, 93)):
        wp, ws, wpg, wsg, st, wt = _weights(qa, K, N, seed)
        x = _randn((M, K), seed + 1).to(dev())
        alone = qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st, w_tiled=wt)
        torch.cuda.synchronize()
        y_ref = orc.linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128)
        assert _rowwise_ok(alone.cpu(), y_ref)[0]
        cases.append((x, wpg, wsg, st, wt, K, N, alone))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(20):
        for i, s in enumerate(streams):
            x, wpg, wsg, st, wt, K, N, _ = cases[i]
            with torch.cuda.stream(s):
                outs[i].append(qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st, w_tiled=wt))
    torch.cuda.synchronize()
    for i in range(2):
        ref = cases[i][7].cpu()
        for k, y in enumerate(outs[i]):
            assert G.bits_equal(y.cpu(), ref), f"stream {i}, call {k} differs from the call alone"


def test_tiled_fallback_for_other_shapes(qa):
    """x with 17 rows, or a misaligned x view, takes mxk_linear_wq."""
    dt = qa.get_mx_dtype("int4d")
    K, N = 1024, 256
    wp, ws, wpg, wsg, st, wt = _weights(qa, K, N, 51)
    big = _randn((4 * K + 1,), 55).to(dev())
    for x in (_randn((17, K), 53).to(dev()), big[1:].view(4, K)):
        assert x.shape[0] > 16 or x.data_ptr() % 16 != 0
        y = qa.ops.linear_wq(x, wpg, wsg, dt, K, N, 128, w_scales_t=st, w_tiled=wt).cpu()
        y_ref = orc.linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128)
        assert _rowwise_ok(y, y_ref)[0]


def test_mx_linear_float4d_tiled(qa):
    """An FP4 (float4d) mx_linear weight is held as its tiled copy like int4:
    forwards at 4 and 40 rows, the input gradient (from the packed codes
    rebuilt on demand) against float64, and dequantize bit for bit."""
    K, N = 1024, 256
    W = _randn((N, K), 71) * 0.03
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W)
    m = qa.mx_linear.from_linear(lin.to(dev()), qa.get_mx_dtype("float4d"), 128)
    wp, ws, _ = orc.linear_from_weight(W, "float4d", 128)
    w = m._mx_weight
    for M in (4, 40):
        x = _randn((M, K), 73 + M)
        y = m(x.to(dev())).cpu()
        assert w.__dict__["_mx_tiled"] is not None and w.__dict__["_mx_packed_store"] is None
        ok, worst = _rowwise_ok(y, orc.linear_forward(x, wp, ws, "float4d", K, N, 128))
        assert ok, f"M={M}: worst row error {worst:.3g} x the bar"
    xg = _randn((24, K), 79).to(dev()).requires_grad_(True)
    g = _randn((24, N), 83)
    m(xg).backward(g.to(dev()))
    w_dq = orc.dequant(wp, ws, "float4d", K * N, 128).reshape(K, N).double()
    ok, worst = _rowwise_ok(xg.grad.cpu(), (g.double() @ w_dq.t()).float())
    assert ok, f"input gradient: worst row error {worst:.3g} x the bar"
    assert G.bits_equal(w._mx_packed.cpu(), wp)
    assert G.bits_equal(w.dequantize().cpu().reshape(-1), orc.dequant(wp, ws, "float4d", K * N, 128))
