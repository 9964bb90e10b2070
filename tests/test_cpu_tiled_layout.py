"""The tiled int4 weight layout of mxk_linear_prepack_weight, restated on the
CPU twice and checked against itself:

  * ``tile_w4`` builds the tiled bytes from the [K][N] packing as the header
    describes it (2 KiB per 128-column block and 32-row step; lane j + 16 g
    at +16 lane and +1024 + 16 lane; word 2p + e = the byte of columns
    8j + 2p, 8j + 2p + 1 of rows 8g + 4e + {0, 2, 1, 3});
  * ``codes_from_tiles`` reads every code back the way the decode kernel
    builds its MFMA operands (masks 0x000F000F / 0x00F000F0 of the word and
    of the word shifted right by 8, tile t = column 8j + t, operand slot i =
    row 8g + i).

Their round trip must give back every code of random weights: a layout
mistake on either side (a swapped row pair, a wrong nibble, a lane or chunk
offset) breaks it.  The GPU tests compare the library's prepack with
``tile_w4`` byte for byte.  This layout has no counterpart in the reference.
"""
import numpy as np
import pytest


def tile_w4(packed: np.ndarray, K: int, N: int) -> np.ndarray:
    """Tiled bytes (uint8, K*N/2) of an int4 [K][N] packing (uint8, K*N/2)."""
    rows = packed.reshape(K, N // 2)
    NB, S = N // 128, K // 32
    nb, ks, g, j, p, e, b = np.meshgrid(np.arange(NB), np.arange(S), np.arange(4), np.arange(16), np.arange(4),
                                        np.arange(2), np.arange(4), indexing="ij", sparse=True)
    order = np.array([0, 2, 1, 3])
    r = 2 * p + e                              # word of the lane
    dst = (nb * S + ks) * 2048 + (r // 4) * 1024 + 16 * (j + 16 * g) + 4 * (r % 4) + b
    src_row = ks * 32 + 8 * g + 4 * e + order[b]
    src_col = nb * 64 + 4 * j + p              # byte of columns 8j + 2p, 8j + 2p + 1
    out = np.zeros(K * N // 2, dtype=np.uint8)
    dst, src_row, src_col = np.broadcast_arrays(dst, src_row, src_col)
    out[dst.reshape(-1)] = rows[src_row.reshape(-1), src_col.reshape(-1)]
    return out


def codes_from_tiles(tiled: np.ndarray, K: int, N: int) -> np.ndarray:
    """int4 codes [K][N] (two's complement, as int8) read from the tiled bytes
    with the decode kernel's operand construction."""
    words = tiled.view("<u4")
    codes = np.zeros((K, N), dtype=np.int8)
    NB, S = N // 128, K // 32
    for nb in range(NB):
        for ks in range(S):
            cw = (nb * S + ks) * 512
            for g in range(4):
                for j in range(16):
                    lane = j + 16 * g
                    wr = [int(words[cw + (r // 4) * 256 + 4 * lane + (r % 4)]) for r in range(8)]
                    w8 = [w >> 8 for w in wr]
                    for t in range(8):
                        p = t >> 1
                        msk, sh = (0x00F000F0, 4) if t & 1 else (0x000F000F, 0)
                        # the four f16 pairs of tile t: slots (0,1), (2,3), (4,5), (6,7)
                        pairs = [wr[2 * p] & msk, w8[2 * p] & msk, wr[2 * p + 1] & msk, w8[2 * p + 1] & msk]
                        for h, d in enumerate(pairs):
                            for half in range(2):
                                nib = (d >> (16 * half + sh)) & 0xF
                                code = nib - 16 if nib >= 8 else nib
                                codes[ks * 32 + 8 * g + 2 * h + half, nb * 128 + 8 * j + t] = code
    return codes


def codes_from_packed(packed: np.ndarray, K: int, N: int) -> np.ndarray:
    """The reference's [K][N] int4 packing read directly (low nibble = even
    column, mxtorch.py:870-985 bit order), as int8 codes."""
    b = packed.reshape(K, N // 2)
    lo = (b & 0xF).astype(np.int16)
    hi = (b >> 4).astype(np.int16)
    c = np.empty((K, N), dtype=np.int16)
    c[:, 0::2], c[:, 1::2] = lo, hi
    return np.where(c >= 8, c - 16, c).astype(np.int8)


@pytest.mark.parametrize("K,N,seed", [(32, 128, 1), (64, 256, 2), (96, 384, 3)])
def test_tiled_round_trip_gives_every_code(K, N, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=K * N // 2, dtype=np.uint8)
    tiled = tile_w4(packed, K, N)
    assert tiled.shape == packed.shape
    assert np.array_equal(np.sort(tiled), np.sort(packed))          # a permutation of the bytes
    assert np.array_equal(codes_from_tiles(tiled, K, N), codes_from_packed(packed, K, N))


def test_tiled_round_trip_fails_on_a_planted_swap():
    """A layout with rows 1 and 2 of each group of four in natural order
    (the mistake the {0, 2, 1, 3} order avoids) must not round-trip."""
    K, N = 32, 128
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, size=K * N // 2, dtype=np.uint8)
    rows = packed.reshape(K, N // 2).copy()
    rows[[1, 2]] = rows[[2, 1]]
    wrong = tile_w4(rows.reshape(-1), K, N)
    assert not np.array_equal(codes_from_tiles(wrong, K, N), codes_from_packed(packed, K, N))
