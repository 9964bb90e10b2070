"""The FP4 bucket of the quantize kernels (bucket_fp4_keyed in
qtpytorch_amd/csrc/mxk_internal.h), restated in numpy and checked against
the definition the reference uses (_quant_float, mxtorch.py:1465-1528:
torch.bucketize over the grid mids, i.e. the count of mids below y):

  * key k = clamp((bits(|y|) >> 21) - 488, 0, 31), a quarter binade from
    2^-5 on; table entry k = (#mids below the key's interval, the mid inside
    it or +inf); count = entry.x + (a > entry.y);
  * y <= 0 counts the mids below nextup(|y|); the code is count ^ 8 for
    y > 0 (or NaN) and count ^ 7 otherwise.

Patterns: every float32 within 2^15 ulps of each mid and of each key
boundary, in both signs; zeros, subnormals, infinities, NaNs; and a stride
through all 2^32 patterns.  Planted mistakes (a key one quarter binade off
the table's, no nextup for y <= 0) must fail.  The
GPU side runs the same patterns through the quantize kernel against the
oracle (tests/test_gpu_parity.py::test_float4_bucket_boundaries).
"""
import numpy as np
import pytest

from oracle import mx_oracle as orc

KEYS = 32


def _mids():
    m = orc.float_mids(4).numpy().astype(np.float32)
    return m, m[m > 0]


def _table(pos_mids, base=488):
    lo_bits = (np.arange(KEYS, dtype=np.uint64) + base) << 21
    lo = lo_bits.astype(np.uint32).view(np.float32).copy()
    lo[0] = 0.0
    hi = ((np.arange(KEYS, dtype=np.uint64) + base + 1) << 21).astype(np.uint32).view(np.float32).copy()
    hi[-1] = np.inf
    cnt = np.array([(pos_mids < l).sum() for l in lo], dtype=np.int64)
    mid = np.full(KEYS, np.inf, dtype=np.float32)
    for k in range(KEYS):
        inside = pos_mids[(pos_mids >= lo[k]) & (pos_mids < hi[k])]
        assert inside.size <= 1, f"key {k} holds {inside.size} mids"
        if inside.size:
            mid[k] = inside[0]
    return cnt, mid


def keyed_codes(y: np.ndarray, key_base=488, nextup=True) -> np.ndarray:
    _, pm = _mids()
    cnt, mid = _table(pm)
    bits = y.view(np.uint32)
    with np.errstate(invalid="ignore"):
        pos = ~(y <= 0)
    ab = (bits & np.uint32(0x7FFFFFFF)) + ((~pos).astype(np.uint32) if nextup else np.uint32(0))
    k = np.clip((ab >> 21).astype(np.int64) - key_base, 0, KEYS - 1)
    with np.errstate(invalid="ignore"):
        c = cnt[k] + (ab.view(np.float32) > mid[k]).astype(np.int64)
    return c ^ np.where(pos, 8, 7)


def bucketize_codes(y: np.ndarray) -> np.ndarray:
    full, _ = _mids()
    # count of mids < y; a NaN sorts last (the last index, as torch.bucketize gives it)
    return np.searchsorted(full, y, side="left").astype(np.int64)


def _patterns():
    _, pm = _mids()
    lo_bits = ((np.arange(1, KEYS, dtype=np.uint64) + 488) << 21).astype(np.uint32)
    centers = np.concatenate([pm.view(np.uint32), lo_bits]).astype(np.int64)
    off = np.arange(-(1 << 15), 1 << 15, dtype=np.int64)
    near = (centers[:, None] + off[None, :]).reshape(-1)
    near = near[(near >= 0) & (near < 0x7F800000)].astype(np.uint32)
    special = np.array([0, 1, 2, 0x007FFFFF, 0x00800000, 0x3F800000, 0x7F7FFFFF, 0x7F800000, 0x7F800001,
                        0x7FC00000, 0x7FFFFFFF], dtype=np.uint32)
    stride = np.arange(0, 1 << 31, 2039, dtype=np.uint64).astype(np.uint32)
    mag = np.concatenate([near, special, stride])
    return np.concatenate([mag, mag | np.uint32(0x80000000)]).view(np.float32)


def test_keyed_bucket_equals_bucketize():
    y = _patterns()
    assert y.size > 4_000_000
    got = keyed_codes(y)
    ref = bucketize_codes(y)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first y = {y[bad[0]]!r} ({y[bad[:1]].view(np.uint32)})"


def test_keyed_bucket_planted_mistakes_fail():
    """A key one quarter binade off the table's, or no nextup for y <= 0
    (ties at -mid then go the wrong way), must fail on these patterns."""
    y = _patterns()
    ref = bucketize_codes(y)
    assert (keyed_codes(y, key_base=487) != ref).any()
    assert (keyed_codes(y, key_base=489) != ref).any()
    assert (keyed_codes(y, nextup=False) != ref).any()


@pytest.mark.parametrize("k", range(KEYS))
def test_each_key_interval_holds_at_most_one_mid(k):
    _, pm = _mids()
    cnt, mid = _table(pm)
    assert 0 <= cnt[k] <= 7
    if np.isfinite(mid[k]):
        assert cnt[k] == (pm < mid[k]).sum()
