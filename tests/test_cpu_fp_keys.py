"""The FP4/FP8 bucket of the quantize kernels (bucket_keyed in
qtpytorch_amd/csrc/mxk_internal.h), restated in numpy and checked against
the definition the reference uses (_quant_float, mxtorch.py:1465-1528:
torch.bucketize over the grid mids, i.e. the count of mids below y):

  * key k = clamp((bits(|y|) >> SHIFT) - BASE, 0, N - 1): FP4 a quarter
    binade from 2^-5 on (N 32, SHIFT 21, BASE 488), FP8 a sixteenth of a
    binade from 2^-19 on (N 305, SHIFT 19, BASE 1728); table entry k =
    (#mids below the key's interval, the mid inside it or +inf); count =
    entry.x + (a > entry.y);
  * y <= 0 counts the mids below nextup(|y|); the code is count ^ H for
    y > 0 (or NaN) and count ^ (H - 1) otherwise (H = 8 or 128).

Patterns: every float32 within 2^15 (FP4) or 2^11 (FP8) ulps of each mid
and of each key boundary, in both signs; zeros, subnormals, infinities,
NaNs; and a stride through all 2^32 patterns.  Planted mistakes (a key one quarter binade off
the table's, no nextup for y <= 0) must fail.  The
GPU side runs the same patterns through the quantize kernel against the
oracle (tests/test_gpu_parity.py::test_float_bucket_boundaries).
"""
import numpy as np
import pytest

from oracle import mx_oracle as orc

KEYS = {4: (32, 21, 488), 8: (305, 19, 1728)}   # N, SHIFT, BASE


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


def keyed_codes(y: np.ndarray, bits: int, key_shift=0, nextup=True) -> np.ndarray:
    n, shift, base = KEYS[bits]
    h = 1 << (bits - 1)
    cnt, mid = _table(bits)
    with np.errstate(invalid="ignore"):
        pos = ~(y <= 0)
    ab = (y.view(np.uint32) & np.uint32(0x7FFFFFFF)) + ((~pos).astype(np.uint32) if nextup else np.uint32(0))
    k = np.clip((ab >> shift).astype(np.int64) - base - key_shift, 0, n - 1)
    with np.errstate(invalid="ignore"):
        c = cnt[k] + (ab.view(np.float32) > mid[k]).astype(np.int64)
    return c ^ np.where(pos, h, h - 1)


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
    special = np.array([0, 1, 2, 0x007FFFFF, 0x00800000, 0x3F800000, 0x7F7FFFFF, 0x7F800000, 0x7F800001,
                        0x7FC00000, 0x7FFFFFFF], dtype=np.uint32)
    stride = np.arange(0, 1 << 31, 2039, dtype=np.uint64).astype(np.uint32)
    mag = np.concatenate([near, special, stride])
    return np.concatenate([mag, mag | np.uint32(0x80000000)]).view(np.float32)


@pytest.mark.parametrize("bits", [4, 8])
def test_keyed_bucket_equals_bucketize(bits):
    y = patterns(bits)
    assert y.size > 3_000_000
    got = keyed_codes(y, bits)
    ref = bucketize_codes(y, bits)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first y = {y[bad[0]]!r} ({y[bad[:1]].view(np.uint32)})"


@pytest.mark.parametrize("bits", [4, 8])
def test_keyed_bucket_planted_mistakes_fail(bits):
    """A key one interval off the table's, or no nextup for y <= 0 (ties at
    -mid then go the wrong way), must fail on these patterns."""
    y = patterns(bits)
    ref = bucketize_codes(y, bits)
    assert (keyed_codes(y, bits, key_shift=-1) != ref).any()
    assert (keyed_codes(y, bits, key_shift=1) != ref).any()
    assert (keyed_codes(y, bits, nextup=False) != ref).any()


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
