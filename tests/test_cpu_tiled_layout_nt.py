"""The tiled int4 [N][K] weight layout of mxk_linear_prepack_weight_nt, restated
on the CPU twice and checked against itself:

  * ``tile_w4t`` builds the tiled bytes from the [N][K] packing as the header
    describes it (1 KiB per 16-row group and 128-wide block of K, lane
    j + 16 g at +16 lane; word 2 sp + h, byte q = code (2 sp, i) |
    code (2 sp + 1, i) << 4 with i = 4 h + {0, 2, 1, 3}[q], where code
    (st, i) is row 16 nt + j at k = 128 kb + 32 g + 8 st + i);
  * ``codes_from_tiles_nt`` reads every code back the way the decode kernel
    builds its MFMA operands (step 2 sp from the masks 0x000F000F of words
    2 sp, 2 sp + 1 and of the same words shifted right by 8, step 2 sp + 1
    from the masks 0x00F000F0; operand slot i of lane (j, g) = code k =
    128 kb + 32 g + 8 st + i of column j).

Their round trip must give back every code of random weights: a layout
mistake on either side (a swapped byte order, a wrong nibble, a lane or
chunk offset) breaks it.  The GPU tests compare the library's prepack with
``tile_w4t`` byte for byte.  This layout has no counterpart in the reference.
"""
import numpy as np
import pytest

ORDER = np.array([0, 2, 1, 3])


def tile_w4t(packed: np.ndarray, N: int, K: int, order=ORDER) -> np.ndarray:
    """Tiled bytes (uint8, N*K/2) of an int4 [N][K] packing (uint8, N*K/2)."""
    rows = packed.reshape(N, K // 2)
    lo_n = (rows & 0xF).astype(np.uint8)
    hi_n = (rows >> 4).astype(np.uint8)
    codes = np.empty((N, K), dtype=np.uint8)           # unsigned nibbles, k in natural order
    codes[:, 0::2], codes[:, 1::2] = lo_n, hi_n
    NT, KB = N // 16, K // 128
    nt, kb, g, j, w, q = np.meshgrid(np.arange(NT), np.arange(KB), np.arange(4), np.arange(16), np.arange(4),
                                     np.arange(4), indexing="ij", sparse=True)
    sp, h = w // 2, w % 2
    i = 4 * h + order[q]
    n = 16 * nt + j
    k_lo = 128 * kb + 32 * g + 8 * (2 * sp) + i
    dst = (nt * KB + kb) * 1024 + 16 * (j + 16 * g) + 4 * w + q
    dst, n, k_lo = np.broadcast_arrays(dst, n, k_lo)
    out = np.zeros(N * K // 2, dtype=np.uint8)
    out[dst.reshape(-1)] = codes[n.reshape(-1), k_lo.reshape(-1)] | (codes[n.reshape(-1), k_lo.reshape(-1) + 8] << 4)
    return out


def codes_from_tiles_nt(tiled: np.ndarray, N: int, K: int) -> np.ndarray:
    """int4 codes [N][K] (two's complement, as int8) read from the tiled bytes
    with the decode kernel's operand construction."""
    words = tiled.view("<u4").astype(np.int64)
    NT, KB = N // 16, K // 128
    # words[(nt*KB + kb)*256 + 4*lane + wd]
    W = words.reshape(NT, KB, 64, 4)
    codes = np.zeros((N, K), dtype=np.int8)
    for sp in range(2):
        w0, w1 = W[..., 2 * sp], W[..., 2 * sp + 1]
        s0, s1 = w0 >> 8, w1 >> 8
        for st, msk, sh in ((2 * sp, 0x000F000F, 0), (2 * sp + 1, 0x00F000F0, 4)):
            dwords = [w0 & msk, s0 & msk, w1 & msk, s1 & msk]     # f16 pairs (slots 2p, 2p + 1)
            for p, d in enumerate(dwords):
                for e in range(2):
                    nib = (d >> (16 * e + sh)) & 0xF                # [NT, KB, 64 lanes]
                    code = np.where(nib >= 8, nib - 16, nib).astype(np.int8)
                    slot = 2 * p + e
                    for lane in range(64):
                        jj, gg = lane & 15, lane >> 4
                        n = 16 * np.arange(NT) + jj
                        k = 128 * np.arange(KB) + 32 * gg + 8 * st + slot
                        codes[np.ix_(n, k)] = code[:, :, lane]
    return codes


def codes_from_packed_nt(packed: np.ndarray, N: int, K: int) -> np.ndarray:
    """The reference's [N][K] int4 packing read directly (low nibble = even k,
    mxtorch.py:870-985 bit order), as int8 codes."""
    b = packed.reshape(N, K // 2)
    c = np.empty((N, K), dtype=np.int16)
    c[:, 0::2], c[:, 1::2] = b & 0xF, b >> 4
    return np.where(c >= 8, c - 16, c).astype(np.int8)


@pytest.mark.parametrize("N,K,seed", [(16, 128, 1), (128, 256, 2), (256, 384, 3)])
def test_tiled_nt_round_trip_gives_every_code(N, K, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=N * K // 2, dtype=np.uint8)
    tiled = tile_w4t(packed, N, K)
    assert tiled.shape == packed.shape
    assert np.array_equal(codes_from_tiles_nt(tiled, N, K), codes_from_packed_nt(packed, N, K))


def test_tiled_nt_unit_holds_the_lane_codes():
    """Each 16-byte unit holds exactly the 32 codes of its row and 32-wide
    stretch of K (the bytes the untiled kernel's lane loads), as a multiset."""
    N, K = 32, 256
    rng = np.random.default_rng(4)
    packed = rng.integers(0, 256, size=N * K // 2, dtype=np.uint8)
    tiled = tile_w4t(packed, N, K)
    rows = packed.reshape(N, K // 2)
    for nt in range(N // 16):
        for kb in range(K // 128):
            for lane in (0, 17, 63):
                j, g = lane & 15, lane >> 4
                unit = tiled[(nt * (K // 128) + kb) * 1024 + 16 * lane:][:16]
                src = rows[16 * nt + j, 64 * kb + 16 * g:][:16]
                nibs = lambda b: np.sort(np.concatenate([b & 0xF, b >> 4]))
                assert np.array_equal(nibs(unit), nibs(src))


def test_tiled_nt_round_trip_fails_on_a_planted_order():
    """A layout with the bytes of each word in natural slot order (the
    mistake the {0, 2, 1, 3} order avoids) must not round-trip."""
    N, K = 16, 128
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, size=N * K // 2, dtype=np.uint8)
    wrong = tile_w4t(packed, N, K, order=np.array([0, 1, 2, 3]))
    assert not np.array_equal(codes_from_tiles_nt(wrong, N, K), codes_from_packed_nt(packed, N, K))
