"""The tiled int4 decode path for [N][K] weights (mxk_linear_prepack_weight_nt
+ mxk_linear_wq_nt_tiled), the kernel mx_dynamic_linear.forward
(mxtorch.py:8949-8962) runs for x of at most 16 rows, and the long-wave
kernel mxk_linear_wq_nt runs on the weight as stored for the same shapes.

  * the library's tiled copy equals the CPU restatement of the layout byte
    for byte (tests/test_cpu_tiled_layout_nt.py pins that restatement
    against the kernel's operand construction);
  * y = x.float() @ dequant(W).t() (+ bias) within 1e-3 of the oracle (per
    output row) for x in float32 / float16 / bfloat16, M in 1..16, with and
    without bias, K that is or is not a multiple of a split (2048 rows,
    including waves wholly past K), and activations and weights from 1e-6 to
    1e6 and rows of different magnitudes; the untiled call agrees within the
    same bar;
  * two streams at once, each with its own workspace, give the results of
    the calls alone, bit for bit;
  * mx_dynamic_linear holds an int4 weight as its tiled copy only (the
    packed codes rebuilt on demand, bit for bit), more than 16 rows run the
    MFMA kernel on the tiled copy (bitwise equal to the packed-code MFMA
    kernel); shapes the tiled kernels do not take fall back.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G
from tests.test_cpu_tiled_layout_nt import tile_w4t

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


def _weights(qa, N, K, seed, mag=0.02):
    W = _randn((N, K), seed, outliers=1e-3) * mag
    wp, ws, _ = orc.dynamic_linear_from_weight(W, "int4d", 128)
    wpg, wsg = wp.to(dev()), ws.to(dev())
    st = qa.ops.prepack_scales(wsg, N, K, 128)
    return wp, ws, wpg, wsg, st, qa.ops.prepack_weight_nt(wpg, N, K, 128)


@pytest.mark.parametrize("N,K", [(128, 128), (384, 2176), (1024, 4096)])
def test_prepack_weight_nt_matches_layout(qa, N, K):
    wp = torch.randint(0, 256, (N * K // 2,), dtype=torch.uint8, generator=torch.Generator().manual_seed(N + K))
    tiled = qa.ops.prepack_weight_nt(wp.to(dev()), N, K, 128).cpu().numpy()
    assert np.array_equal(tiled, tile_w4t(wp.numpy(), N, K))


def test_prepack_weight_nt_config2_sampled(qa):
    """8192 x 8192: a few chunks against the layout."""
    N = K = 8192
    wp = torch.randint(0, 256, (N * K // 2,), dtype=torch.uint8, generator=torch.Generator().manual_seed(9))
    tiled = qa.ops.prepack_weight_nt(wp.to(dev()), N, K, 128).cpu().numpy()
    rows = wp.numpy().reshape(N, K // 2)
    KB = K // 128
    for nt in (0, 77, 511):
        for kb in (0, 31, 63):
            sub = np.ascontiguousarray(rows[nt * 16:(nt + 1) * 16, kb * 64:(kb + 1) * 64]).reshape(-1)
            want = tile_w4t(sub, 16, 128)
            c = (nt * KB + kb) * 1024
            assert np.array_equal(tiled[c:c + 1024], want), f"chunk nt={nt} kb={kb}"


CASES = [
    # M, N, K, x dtype, bias
    (16, 8192, 8192, torch.float32, False),
    (16, 4096, 8192, torch.bfloat16, True),
    (1, 1024, 4096, torch.float32, True),
    (5, 384, 2176, torch.float16, False),      # the last split's waves lie past K
    (16, 256, 2048, torch.bfloat16, False),    # one split
    (9, 128, 128, torch.float32, True),        # one block of K: seven waves past K
    (16, 640, 12288, torch.float32, False),
]


@pytest.mark.parametrize("M,N,K,xdt,use_bias", CASES)
def test_tiled_nt_linear_vs_oracle(qa, M, N, K, xdt, use_bias):
    print(f"tiled nt decode M={M} N={N} K={K} {xdt} bias={use_bias}", flush=True)
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 41 + K % 89)
    x = _randn((M, K), 43 + M).to(xdt)
    bias = _randn((N,), 47) if use_bias else None
    bg = None if bias is None else bias.to(dev())
    y = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, bias=bg, w_scales_t=st, w_tiled=wt).cpu()
    y_ref = orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128, bias)
    ok, worst = _rowwise_ok(y, y_ref)
    assert ok, f"worst row error {worst:.3g} x the bar"
    for sc in (st, None):
        y_plain = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, bias=bg, w_scales_t=sc).cpu()
        ok, worst = _rowwise_ok(y_plain, y_ref)
        assert ok, f"untiled path (scales_t={sc is not None}): worst row error {worst:.3g} x the bar"


MAGS = [1e-6, 1e-3, 1e4, 1e6]


@pytest.mark.parametrize("wmag", MAGS)
@pytest.mark.parametrize("xmag", MAGS)
def test_tiled_nt_magnitudes(qa, xmag, wmag):
    M, N, K = 16, 512, 2048
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 53, mag=wmag)
    x = _randn((M, K), 59) * xmag
    y = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt).cpu()
    ok, worst = _rowwise_ok(y, orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128))
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_tiled_nt_mixed_row_magnitudes(qa):
    """Rows from 1e-7 to 1e7 in one call, and a row of zeros: each row within
    the bar of its own magnitude (the range of x is taken per row)."""
    M, N, K = 16, 1024, 4096
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 61)
    x = _randn((M, K), 67)
    x[: M - 1] *= torch.logspace(-7, 7, M - 1)[:, None]
    x[M - 1] = 0.0
    y = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt).cpu()
    y_ref = orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128)
    assert torch.equal(y[M - 1], torch.zeros(N))
    ok, worst = _rowwise_ok(y[: M - 1], y_ref[: M - 1])
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_tiled_nt_two_streams_concurrently(qa):
    cases = []
    for (M, N, K, seed) in ((16, 4096, 8192, 71), (7, 8192, 4096, 73)):
        wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, seed)
        x = _randn((M, K), seed + 1).to(dev())
        alone = qa.ops.linear_wq_nt(x, wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt)
        torch.cuda.synchronize()
        assert _rowwise_ok(alone.cpu(), orc.dynamic_linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128))[0]
        cases.append((x, wpg, wsg, st, wt, N, K, alone))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(20):
        for i, s in enumerate(streams):
            x, wpg, wsg, st, wt, N, K, _ = cases[i]
            with torch.cuda.stream(s):
                outs[i].append(qa.ops.linear_wq_nt(x, wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt))
    torch.cuda.synchronize()
    for i in range(2):
        ref = cases[i][7].cpu()
        for k, y in enumerate(outs[i]):
            assert G.bits_equal(y.cpu(), ref), f"stream {i}, call {k} differs from the call alone"


def test_mx_dynamic_linear_keeps_one_tiled_copy(qa):
    """mx_dynamic_linear holds an eligible int4 weight as its tiled copy only,
    from the first forward (any row count) on: one copy of the weight's
    bytes.  The packed codes come back bit for bit on demand (dequantize,
    state_dict), the decode and MFMA kernels read the tiled copy, an in-place
    copy_ turns the weight back to packed storage (and the next forward tiles
    the new codes), the input gradient matches the oracle's, and
    tiled_decode = False keeps the packed codes."""
    K, N = 1024, 256
    lin = torch.nn.Linear(K, N, bias=True)
    m = qa.mx_dynamic_linear.from_linear(lin.to(dev()), "int4d", "int8d")
    wp, ws, _ = orc.dynamic_linear_from_weight(lin.weight.data.cpu(), "int4d", 128)
    bias = lin.bias.data.cpu()
    w = m.weight
    for M in (4, 40):
        x = _randn((M, K), 171 + M).to(dev())
        y = m(x).cpu()
        assert w.__dict__["_mx_tiled"] is not None and w.__dict__["_mx_packed_store"] is None
        assert _rowwise_ok(y, orc.dynamic_linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128, bias))[0]
    assert w.nbytes_packed == K * N // 2 + ws.numel() * 4          # one copy of the codes
    assert G.bits_equal(w._mx_packed.cpu(), wp)                       # rebuilt on demand
    assert w._mx_packed.dtype == wp.dtype
    assert G.bits_equal(w.dequantize().cpu().reshape(-1), orc.dequant(wp, ws, "int4d", K * N, 128))
    # the input gradient (the [in, out] product on the rebuilt codes)
    x = _randn((24, K), 181).to(dev()).requires_grad_(True)
    g = _randn((24, N), 183).to(dev())
    m(x).backward(g)
    gi_ref = g.cpu() @ orc.dequant(wp, ws, "int4d", K * N, 128).reshape(N, K)
    assert _rowwise_ok(x.grad.cpu(), gi_ref)[0]
    sd = {k: v for k, v in m.state_dict().items()}
    m2 = qa.mx_dynamic_linear.from_linear(torch.nn.Linear(K, N, bias=True).to(dev()), "int4d", "int8d")
    m2.load_state_dict(sd)
    x = _randn((9, K), 185).to(dev())
    assert G.bits_equal(m2(x).cpu(), m(x).cpu())
    # an in-place change of the codes
    W2 = _randn((N, K), 187) * 0.03
    q2 = qa.mx_tensor.quantize(W2.to(dev()), qa.get_mx_dtype("int4d"), 128)
    w.copy_(q2)
    assert w.__dict__["_mx_tiled"] is None
    wp2, ws2, _ = orc.dynamic_linear_from_weight(W2, "int4d", 128)
    y2 = m(x).cpu()
    assert w.__dict__["_mx_tiled"] is not None
    assert _rowwise_ok(y2, orc.dynamic_linear_forward(x.cpu(), wp2, ws2, "int4d", K, N, 128, bias))[0]
    m3 = qa.mx_dynamic_linear.from_linear(lin.to(dev()), "int4d", "int8d")
    m3.tiled_decode = False
    m3(x)
    assert m3.weight.__dict__.get("_mx_tiled") is None


@pytest.mark.parametrize("N,K", [(128, 128), (384, 2176), (1024, 4096)])
def test_unpack_weight_nt_inverts_prepack(qa, N, K):
    """unpack_weight_nt(prepack_weight_nt(p)) == p byte for byte."""
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 191 + N)
    assert G.bits_equal(qa.ops.unpack_weight_nt(wt, N, K, 128).cpu(), wp.view(torch.uint8))


@pytest.mark.parametrize("M", [17, 64, 300])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_tiled_nt_mfma_vs_oracle(qa, M, xdt):
    """More than 16 rows on the tiled copy alone (w_packed None): the MFMA
    kernel reading the tiled [N][K] layout, within the bar of the oracle, and
    equal to the MFMA kernel on the packed codes bit for bit."""
    N, K = 384, 2176
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 193 + M)
    x = _randn((M, K), 197 + M).to(xdt)
    b = _randn((N,), 199)
    y = qa.ops.linear_wq_nt(x.to(dev()), None, wsg, "int4d", N, K, 128, bias=b.to(dev()), w_scales_t=st,
                            w_tiled=wt).cpu()
    ok, worst = _rowwise_ok(y, orc.dynamic_linear_forward(x.float(), wp, ws, "int4d", K, N, 128, b))
    assert ok, f"worst row error {worst:.3g} x the bar"
    y_packed = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, bias=b.to(dev()), w_scales_t=st).cpu()
    assert G.bits_equal(y, y_packed)


def _mfma_nt_shapes(seed, count):
    g = np.random.default_rng(seed)
    return [(int(g.integers(17, 400)), int(g.integers(1, 13)) * 128, int(g.integers(1, 9)) * 128) for _ in range(count)]


@pytest.mark.parametrize("M,K,N", _mfma_nt_shapes(777, 8))
def test_tiled_nt_mfma_random_shapes(qa, M, K, N):
    """Seeded random shapes beyond the decode (M 17..399, K and N multiples
    of 128) on the tiled [N][K] copy alone, within the bar of the oracle."""
    print(f"tiled nt mfma M={M} K={K} N={N}", flush=True)
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 211 + N + K)
    x = _randn((M, K), 223 + M)
    y = qa.ops.linear_wq_nt(x.to(dev()), None, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt).cpu()
    ok, worst = _rowwise_ok(y, orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128))
    assert ok, f"worst row error {worst:.3g} x the bar"


def test_tiled_nt_fallback_for_other_shapes(qa):
    """x with 17 rows, or a misaligned x view, takes mxk_linear_wq_nt."""
    N, K = 256, 1024
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 79)
    big = _randn((4 * K + 1,), 83).to(dev())
    for x in (_randn((17, K), 89).to(dev()), big[1:].view(4, K)):
        assert x.shape[0] > 16 or x.data_ptr() % 16 != 0
        y = qa.ops.linear_wq_nt(x, wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt).cpu()
        assert _rowwise_ok(y, orc.dynamic_linear_forward(x.cpu(), wp, ws, "int4d", K, N, 128))[0]


def _sweep_shapes(seed, count):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        M = int(g.integers(1, 17))
        K = int(g.integers(1, 49)) * 128
        N = int(g.integers(1, 17)) * 128
        out.append((M, K, N))
    return out


@pytest.mark.parametrize("M,K,N", _sweep_shapes(2024, 12))
def test_tiled_decodes_random_shapes(qa, M, K, N):
    """Seeded random decode shapes (M 1..16, K and N multiples of 128) through
    both tiled kernels: mx_linear's [K][N] path (x @ dequant(W)) and the
    [N][K] path (x @ dequant(W)^T), each within the bar of the oracle."""
    print(f"random tiled shapes M={M} K={K} N={N}", flush=True)
    x = _randn((M, K), 97 + M + K)
    # [N][K] weight, blocks along K
    wp, ws, wpg, wsg, st, wt = _weights(qa, N, K, 101 + N)
    y = qa.ops.linear_wq_nt(x.to(dev()), wpg, wsg, "int4d", N, K, 128, w_scales_t=st, w_tiled=wt).cpu()
    ok, worst = _rowwise_ok(y, orc.dynamic_linear_forward(x, wp, ws, "int4d", K, N, 128))
    assert ok, f"[N][K] tiled: worst row error {worst:.3g} x the bar"
    # [K][N] weight of quantize(W.t()), blocks along N
    W = _randn((N, K), 103 + K, outliers=1e-3) * 0.02
    fp, fs, _ = orc.linear_from_weight(W, "int4d", 128)
    fpg, fsg = fp.to(dev()), fs.to(dev())
    y2 = qa.ops.linear_wq(x.to(dev()), fpg, fsg, "int4d", K, N, 128, w_scales_t=qa.ops.prepack_scales(fsg, K, N, 128),
                          w_tiled=qa.ops.prepack_weight(fpg, K, N, 128)).cpu()
    ok, worst = _rowwise_ok(y2, orc.linear_forward(x, fp, fs, "int4d", K, N, 128))
    assert ok, f"[K][N] tiled: worst row error {worst:.3g} x the bar"
