"""Pins for the CPU oracle (oracle/mx_oracle.py) that the golden vectors do
not cover on their own: the torch arithmetic facts the restatement relies on,
and closed forms / brute force for the helpers.  Each check is chosen so that
a plausible slip (a dropped rounding, a transposed operand, a wrong sign or
index) fails it; none of them restates the oracle's own formula.

  * torch's ``scalar / tensor`` is ``reciprocal() * scalar`` (two roundings),
    which the int quantizer's scale chain depends on (mxtorch.py:1458-1459);
  * ``torch.round`` rounds half to even; ``bucketize(right=False)`` counts
    boundaries strictly below the value (mxtorch.py:1460, 1524);
  * ``int_accumulators``: per-block products summed over blocks equal the
    full exact integer product, and a hand-computed 2x3x2 case;
  * ``fwht``: H H^T = I (orthonormal after the 1/sqrt(n) division), the
    Sylvester order on unit vectors, unrotate(rotate(x)) = x and norms kept
    for power-of-two rows (the reference's truncation makes other lengths
    lossy);
  * ``qgemm_ste_forward``: close to the fp32 product A @ B when B's blocks
    share one absmax (the reference's scale reading is then immaterial);
  * ``linear_forward``: x @ W for the stored [in, out] weight, not W^T.
"""
import math

import torch

from oracle import mx_oracle as orc


def test_rdiv_is_reciprocal_times_scalar():
    g = torch.Generator().manual_seed(0)
    a = torch.rand(1 << 16, generator=g) * 1e3 + 1e-6
    for q in (127.0, 7.0, 1.0, 3.0):
        assert torch.equal(q / a, a.reciprocal() * q)
    # and it differs from an IEEE division for some inputs (so the fact matters)
    exact = torch.tensor(127.0, dtype=torch.float64) / a.double()
    assert not torch.equal((127.0 / a).double(), exact.float().double())


def test_round_half_even_and_bucketize_ties():
    assert torch.round(torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5])).tolist() == [0, 2, 2, -0, -2, -2]
    mids = torch.tensor([-1.0, 0.0, 1.0])
    y = torch.tensor([-1.0, -0.5, 0.0, 0.5, 1.0, 2.0])
    assert torch.bucketize(y, mids).tolist() == [0, 1, 1, 2, 2, 3]


def test_int_accumulators_brute_force():
    a = torch.tensor([[1, -2, 3], [4, 5, -6]], dtype=torch.int32)
    b = torch.tensor([[7, -8], [9, 10], [-11, 12]], dtype=torch.int32)
    acc = orc.int_accumulators(a.reshape(-1), b.reshape(-1), 2, 3, 2, 2)
    # blocks of 2 along K: k in {0,1} and {2}
    assert acc[0].tolist() == [[1 * 7 + -2 * 9, 1 * -8 + -2 * 10], [4 * 7 + 5 * 9, 4 * -8 + 5 * 10]]
    assert acc[1].tolist() == [[3 * -11, 3 * 12], [-6 * -11, -6 * 12]]
    g = torch.Generator().manual_seed(1)
    M, K, N = 9, 300, 7
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int32)
    B = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int32)
    acc = orc.int_accumulators(A.reshape(-1), B.reshape(-1), M, K, N, 128)
    full = torch.zeros(M, N, dtype=torch.int64)
    for m in range(M):
        for n in range(N):
            full[m, n] = sum(int(A[m, k]) * int(B[k, n]) for k in range(K))
    assert torch.equal(acc.to(torch.int64).sum(0), full)


def test_fwht_orthonormal_sylvester_and_roundtrip():
    for n in (2, 8, 128):
        H = orc.fwht(torch.eye(n))
        assert torch.allclose(H @ H.t(), torch.eye(n), atol=1e-6)
        # Sylvester order: H[i][j] = (-1)^popcount(i & j) / sqrt(n)
        ref = torch.tensor([[(-1.0) ** bin(i & j).count("1") for j in range(n)] for i in range(n)]) / math.sqrt(n)
        assert torch.allclose(H, ref, atol=1e-7)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 128, generator=g)
    s = orc.hadamard_signs(128, 1534857261)
    assert set(s.unique().tolist()) == {-1.0, 1.0}
    y = orc.unrotate(orc.rotate(x, s), s)
    assert (y - x).abs().max().item() < 1e-5
    # a rotation is an isometry: norms are kept
    assert torch.allclose(orc.rotate(x, s).norm(dim=1), x.norm(dim=1), rtol=1e-5)
    # for a non-power-of-two last dim the reference pads to n, transforms and
    # truncates back to d (mxtorch.py:2876-2889), so the round trip is lossy
    x96 = torch.randn(5, 96, generator=g)
    assert (orc.unrotate(orc.rotate(x96, s), s) - x96).abs().max().item() > 0.1


def test_qgemm_ste_forward_is_a_times_b():
    """With every flat 128-block of B holding the same absmax, the
    reference's reading of B's scales as [K/128, N] (mxtorch.py:1352-1355)
    sees one common scale, so the STE forward must approximate A @ B."""
    g = torch.Generator().manual_seed(3)
    A = torch.randn(64, 256, generator=g)
    B = torch.rand(256, 128, generator=g) * 2 - 1
    B[:, 0] = 1.0  # absmax 1 in every block of 128 (one row of B per block)
    C = orc.qgemm_ste_forward(A, B, "int8d", 128)
    ref = A @ B
    assert C.shape == (64, 128)
    assert (C - ref).abs().max().item() < 0.02 * ref.abs().max().item()
    # a transposed or swapped operand would not come close
    assert (C - (A @ B.flip(0))).abs().max().item() > 0.2 * ref.abs().max().item()


def test_linear_forward_uses_stored_in_out_layout():
    g = torch.Generator().manual_seed(4)
    W = torch.randn(24, 256, generator=g)  # nn.Linear weight [out, in]
    x = torch.randn(3, 256, generator=g)
    wp, ws, _ = orc.linear_from_weight(W, "int8d", 128)
    y = orc.linear_forward(x, wp, ws, "int8d", 256, 24, 128)
    ref = x @ W.t()
    assert y.shape == (3, 24)
    assert (y - ref).abs().max().item() < 0.02 * ref.abs().max().item()
