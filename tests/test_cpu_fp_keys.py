"""The FP4/FP8 bucket of the quantize kernels (build_fp_keys, bucket_signed
and fp_quot in qtpytorch_amd/csrc/mxk_internal.h), restated in numpy and
checked against the definition the reference uses (_quant_float,
mxtorch.py:1465-1528: torch.bucketize over the grid mids, i.e. the count of
mids below y):

  * magnitude key k = (bits(clamp(|y|, LO, HI)) >> SHIFT) - BASE: FP4 a
    quarter binade from 2^-5 on (N 32, SHIFT 21, BASE 488), FP8 a sixteenth
    of a binade from 2^-19 on (N 305, SHIFT 19, BASE 1728);
  * one table half per sign (FP4: the sign is bit 10 of the key, the
    negative half 1024 entries on; FP8: 305 entries on); entry = (base,
    threshold) and code = base + (y > threshold): positive (H + c_k, m_k),
    negative (H - 2 - c_k, -m_k), no mid in the key (H + c_k, +inf) /
    (H - 1 - c_k, +inf), positive key 0 (H - 1, +0).

Patterns: every float32 within 2^15 (FP4) or 2^11 (FP8) ulps of each mid
and of each key boundary, in both signs; zeros, subnormals, infinities; and
a stride through all 2^32 patterns (NaN codes come from the kernels'
non-finite path, not from this table).  Planted mistakes (a key one quarter
binade off the table's, +m as the negative threshold, +inf as the threshold
of positive key 0) must fail.  The quotient the bucket is taken of (div_rn:
Markstein's correction, IEEE division for |a| < 2^-96) is checked with an
exact FMA emulation where only its sign and zero-ness matter (quotients
near 2^-150), and the small-numerator branch is shown to be needed.  The GPU side runs the same patterns through the
quantize kernel against the oracle
(tests/test_gpu_parity.py::test_float_bucket_boundaries).
"""
import numpy as np
import pytest

from oracle import mx_oracle as orc

KEYS = {4: (32, 21, 488), 8: (305, 19, 1728)}   # N, SHIFT, BASE
NEG = {4: 1024, 8: 305}                          # index of the negative half


def _mids(bits):
    m = orc.float_mids(bits).numpy().astype(np.float32)
    return m, m[m > 0]


def _table(bits):
    n, shift, base = KEYS[bits]
    _, pm = _mids(bits)
    lo = ((np.arange(n, dtype=np.uint64) + base) << shift).astype(np.uint32).view(np.float32).copy()
    lo[0] = 0.0
    hi = ((np.arange(n, dtype=np.uint64) + base + 1) << shift).astype(np.uint32).view(np.float32).copy()
    hi[-1] = np.inf
    cnt = np.searchsorted(pm, lo, side="left").astype(np.int64)
    mid = np.full(n, np.inf, dtype=np.float32)
    for k in range(n):
        inside = pm[(pm >= lo[k]) & (pm < hi[k])]
        assert inside.size <= 1, f"key {k} holds {inside.size} mids"
        if inside.size:
            mid[k] = inside[0]
    return cnt, mid


def signed_table(bits, plant=None):
    """build_fp_keys: (base, threshold) per (sign, key); entries between the
    FP4 halves are never read (left at -1)."""
    n, _, _ = KEYS[bits]
    h = 1 << (bits - 1)
    cnt, mid = _table(bits)
    base = np.full(NEG[bits] + n, -1, dtype=np.int64)
    thr = np.full(NEG[bits] + n, np.nan, dtype=np.float32)
    has = np.isfinite(mid)
    base[:n] = h + cnt
    thr[:n] = mid
    base[0], thr[0] = h - 1, 0.0 if plant != "key0_inf" else np.inf
    base[NEG[bits]:] = np.where(has, h - 2 - cnt, h - 1 - cnt)
    thr[NEG[bits]:] = np.where(has, mid if plant == "neg_plus_mid" else -mid, np.inf)
    return base, thr


def signed_codes(y: np.ndarray, bits: int, key_shift=0, plant=None) -> np.ndarray:
    n, shift, base0 = KEYS[bits]
    base, thr = signed_table(bits, plant)
    lo = np.uint32(base0 << shift).view(np.float32)
    hi = np.uint32((base0 + n - 1) << shift).view(np.float32)
    c = np.minimum(np.maximum(np.abs(y), lo), hi)
    neg = (y.view(np.uint32) >> 31).astype(np.int64)
    k = (c.view(np.uint32) >> shift).astype(np.int64) - base0 - key_shift
    k = np.clip(k, 0, n - 1)
    idx = k + neg * NEG[bits]
    with np.errstate(invalid="ignore"):
        return base[idx] + (y > thr[idx]).astype(np.int64)


def bucketize_codes(y: np.ndarray, bits: int) -> np.ndarray:
    full, _ = _mids(bits)
    # count of mids < y; a NaN sorts last (the last index, as torch.bucketize gives it)
    return np.searchsorted(full, y, side="left").astype(np.int64)


def patterns(bits: int, radius=None) -> np.ndarray:
    n, shift, base = KEYS[bits]
    radius = radius or (1 << 15 if bits == 4 else 1 << 11)
    _, pm = _mids(bits)
    lo_bits = ((np.arange(1, n, dtype=np.uint64) + base) << shift).astype(np.uint32)
    centers = np.concatenate([pm.view(np.uint32), lo_bits]).astype(np.int64)
    off = np.arange(-radius, radius, dtype=np.int64)
    near = (centers[:, None] + off[None, :]).reshape(-1)
    near = near[(near >= 0) & (near < 0x7F800000)].astype(np.uint32)
    special = np.array([0, 1, 2, 0x007FFFFF, 0x00800000, 0x3F800000, 0x7F7FFFFF, 0x7F800000],
                       dtype=np.uint32)
    stride = np.arange(0, 1 << 31, 2039, dtype=np.uint64).astype(np.uint32)
    mag = np.concatenate([near, special, stride])
    y = np.concatenate([mag, mag | np.uint32(0x80000000)]).view(np.float32)
    return y[~np.isnan(y)]


@pytest.mark.parametrize("bits", [4, 8])
def test_signed_bucket_equals_bucketize(bits):
    y = patterns(bits)
    assert y.size > 3_000_000
    got = signed_codes(y, bits)
    ref = bucketize_codes(y, bits)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first y = {y[bad[0]]!r} ({y[bad[:1]].view(np.uint32)})"
    # the codes need no mask before packing
    assert got.min() == 0 and got.max() == (1 << bits) - 1


@pytest.mark.parametrize("bits", [4, 8])
def test_signed_bucket_planted_mistakes_fail(bits):
    """A key one interval off the table's, +m as a negative threshold (ties
    at -mid and the values between go the wrong way), or +inf as positive
    key 0's threshold (tiny positives take the code of zero) must fail."""
    y = patterns(bits)
    ref = bucketize_codes(y, bits)
    assert (signed_codes(y, bits, key_shift=-1) != ref).any()
    assert (signed_codes(y, bits, key_shift=1) != ref).any()
    assert (signed_codes(y, bits, plant="neg_plus_mid") != ref).any()
    assert (signed_codes(y, bits, plant="key0_inf") != ref).any()


@pytest.mark.parametrize("bits", [4, 8])
def test_key_tables(bits):
    """Every key's interval holds at most one mid (asserted while building),
    and a mid's count is the number of mids below it."""
    _, pm = _mids(bits)
    cnt, mid = _table(bits)
    h = 1 << (bits - 1)
    assert cnt.min() == 0 and cnt.max() == h - 1
    fin = np.isfinite(mid)
    assert fin.sum() == h - 1       # every positive mid sits in exactly one key
    assert np.array_equal(cnt[fin], np.searchsorted(pm, mid[fin], side="left"))
    assert not fin[0]               # positive key 0's entry (H - 1, +0) assumes no mid in it


# ---------------------------------------------------------------- fp_quot
def fma32(a, b, c):
    """RN32(a * b + c) exactly: the product is exact in float64, the sum's
    float64 rounding error comes from TwoSum, and it only decides the
    float32 rounding where the float64 sum sits on a float32 midpoint."""
    a, b, c = (np.asarray(t, dtype=np.float32) for t in (a, b, c))
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    nb = np.nextafter(r, toward)
    mid = (r64 + nb.astype(np.float64)) * 0.5
    on_mid = (s != r64) & (s == mid) & (e != 0)
    # the exact sum lies beyond the midpoint toward nb when e points that way
    go = on_mid & (np.sign(e) == np.sign(nb.astype(np.float64) - r64))
    # elsewhere the exact sum is within half a float64 ulp of s, on the same
    # side of every float32 midpoint, so it rounds like s
    return np.where(go, nb, r)


def markstein_np(a, b):
    y = (np.float32(1.0) / b).astype(np.float32)
    q0 = (a.astype(np.float64) * y.astype(np.float64)).astype(np.float32)
    return fma32(fma32(-q0, b, a), y, q0)


def div_rn_np(a, b):
    """div_rn: IEEE division below 2^-96, Markstein's correction above."""
    return np.where(np.abs(a) < np.float32(2.0 ** -96), (a / b).astype(np.float32), markstein_np(a, b))


def test_fma32_emulation():
    """The emulation against exact rational arithmetic on tie-prone cases."""
    from fractions import Fraction
    rng = np.random.default_rng(3)
    a = rng.standard_normal(3000).astype(np.float32)
    b = rng.standard_normal(3000).astype(np.float32)
    c = (-(a.astype(np.float64) * b) * (1 + rng.integers(-4, 5, 3000) * 2.0 ** -24)).astype(np.float32)
    c[:1000] = np.ldexp(rng.standard_normal(1000), -30).astype(np.float32)
    got = fma32(a, b, c)
    for i in range(a.size):
        ex = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        want = np.float32(float(ex))  # nearest double, then float32: exact unless on a midpoint
        lo = np.float32(want)
        cand = [lo, np.nextafter(lo, np.float32(-np.inf)), np.nextafter(lo, np.float32(np.inf))]
        best = min(cand, key=lambda v: (abs(Fraction(float(v)) - ex),
                                        int(np.asarray(v).view(np.uint32)) & 1))
        assert got[i] == best, (a[i], b[i], c[i], got[i], best)


def _tiny_cases(rng):
    """Numerators and scales around a / b = 2^-150 (where RN(a / b) turns
    zero): every subnormal k * 2^-149 up to 2^16 and random ones above with
    b near 2k, random normal numerators below 2^-96 with b near a * 2^150,
    and numerators in [2^-96, 2^-60) with b near a * 2^150 (clipped to
    float32 range), each at the 7 scales within 3 ulps."""
    k = np.concatenate([np.arange(1, 1 << 16), rng.integers(1 << 16, 1 << 23, 1 << 17)]).astype(np.int64)
    a_sub = (k.astype(np.float64) * 2.0 ** -149).astype(np.float32)
    b_sub = (2.0 * k).astype(np.float32)
    m = rng.integers(1 << 23, 1 << 24, 1 << 17).astype(np.float64)
    a_nrm = np.ldexp(m, rng.integers(-126, -96, 1 << 17) - 23).astype(np.float32)
    a_mid = np.ldexp(m, rng.integers(-96, -60, 1 << 17) - 23).astype(np.float32)
    a0 = np.concatenate([a_sub, a_nrm, a_mid])
    b0 = np.minimum(np.concatenate([b_sub, a_nrm.astype(np.float64) * 2.0 ** 150,
                                    a_mid.astype(np.float64) * 2.0 ** 150]), 3.0e38).astype(np.float32)
    out = []
    for j in range(-3, 4):
        b = b0.copy()
        for _ in range(abs(j)):
            b = np.nextafter(b, np.float32(np.inf if j > 0 else 0.0)).astype(np.float32)
        ok = (b >= np.float32(1e-12)) & (np.abs(a0) <= b)
        out.append((a0[ok], b[ok]))
    return out


def test_div_rn_sign_at_tiny_quotients():
    """div_rn(a, b) > 0 exactly when RN(a / b) > 0 for quotients around
    2^-150, the only property of a quotient below the lowest key that the
    float bucket reads; negative numerators never give a positive one."""
    for a, b in _tiny_cases(np.random.default_rng(11)):
        exact = (a / b).astype(np.float32)  # IEEE float32 division
        got = div_rn_np(a, b)
        assert np.array_equal(got > 0, exact > 0), a[(got > 0) != (exact > 0)][:3]
        assert not (div_rn_np(-a, b) > 0).any()


def test_div_rn_needs_its_small_numerator_branch():
    """Without the branch the correction's residual is rounded on the
    subnormal grid: a = 2^-149, b = 2 - 2^-23 gives 0 where RN(a / b) =
    2^-149 (the bucket would take the code of zero)."""
    a = np.array([2.0 ** -149], dtype=np.float32)
    b = np.array([2.0 - 2.0 ** -23], dtype=np.float32)
    assert (a / b).astype(np.float32)[0] == np.float32(2.0 ** -149)
    assert markstein_np(a, b)[0] == 0.0
    assert div_rn_np(a, b)[0] == np.float32(2.0 ** -149)
    wrong = 0
    for a, b in _tiny_cases(np.random.default_rng(11)):
        wrong += int(((markstein_np(a, b) > 0) != ((a / b).astype(np.float32) > 0)).sum())
    assert wrong > 0
