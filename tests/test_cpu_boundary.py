"""CPU-only checks of the drop-in boundary (no GPU compute):

  * libmxk.so loads and exports every entry point include/mxk.h declares;
  * host-side helpers: packed sizes equal the reference packer's lengths,
    the float grids/mids equal the oracle's (torch) tables bit for bit;
  * the dtype registry mirrors the reference's names and properties;
  * the product refuses CPU tensors loudly (no CPU compute path).
"""
import os
import re

import pytest
import torch

from oracle import mx_oracle as orc
from tests import _golden as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "mxk.h")).read()
    return sorted(set(re.findall(r"\b(mxk_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from qtpytorch_amd import _lib as L
    h = L.lib()
    declared = _declared_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(h, name), f"libmxk.so does not export {name}"
        assert name in L.SIGNATURES, f"ctypes binding lacks {name}"
    assert h.mxk_abi_version() == L.ABI_VERSION


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8, 16])
@pytest.mark.parametrize("n", [1, 7, 8, 100, 128, 300, 1000])
def test_packed_nbytes_matches_reference_packer(bits, n):
    from qtpytorch_amd import _lib as L
    codes = torch.zeros(n, dtype=torch.int32)
    ref = orc.pack_auto(codes, bits)
    assert L.lib().mxk_packed_nbytes(bits, n) == ref.numel() * ref.element_size()


@pytest.mark.parametrize("bits", [4, 8])
def test_float_grid_tables_match_oracle(bits):
    from qtpytorch_amd import ops
    g, m = ops.float_grid(bits)
    assert G.bits_equal(g, orc.float_grid(bits))
    assert G.bits_equal(m, orc.float_mids(bits))
    # and the reference's own grid from the golden file
    assert G.bits_equal(g, G.get(f"grid/{bits}"))


def test_dtype_registry_mirrors_reference():
    import qtpytorch_amd as qa
    from qtpytorch_amd.dtypes import _DTYPE_REGISTRY
    assert len(_DTYPE_REGISTRY) == 2 * 12 * 2 * 6
    d = qa.get_mx_dtype("int4d")
    assert (d.kind, d.bits, d.mode, d.variant, d.max_val, d.pack_ratio) == ("int", 4, "d", "", 7.0, 2)
    assert qa.get_mx_dtype("int1d").max_val == 1.0
    assert qa.get_mx_dtype("float8d").max_val == 448.0
    assert qa.get_mx_dtype("int4dh").base is qa.get_mx_dtype("int4d")
    with pytest.raises(ValueError):
        qa.get_mx_dtype("int8v")  # config 5's "int8v" has no mode letter
    for a, b, out in (("int8d", "int8d", "int16d"), ("int4d", "int4d", "int8d"), ("int2d", "int2d", "int4d"),
                      ("int1d", "int1d", "int2d"), ("float4d", "float4d", "float8d"), ("int4u", "int4d", "int8u")):
        assert qa.matmul_output_dtype(qa.get_mx_dtype(a), qa.get_mx_dtype(b)).name == out
        assert orc.matmul_out_bits(qa.get_mx_dtype(a).bits, qa.get_mx_dtype(b).bits) == qa.get_mx_dtype(out).bits


def test_cpu_tensors_are_refused():
    import qtpytorch_amd as qa
    from qtpytorch_amd._lib import MXKError
    with pytest.raises(MXKError):
        qa.mx_tensor.quantize(torch.randn(256), qa.get_mx_dtype("int4d"), 128)


def test_bad_arguments_return_errors_without_gpu():
    """Argument validation happens on the host before any launch."""
    from qtpytorch_amd import _lib as L
    h = L.lib()
    rc = h.mxk_quantize(None, 0, 256, 0, 4, 0, 128, None, 0, None, 0, None, 256, None, 0, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_quantize(8, 0, 256, 1, 5, 0, 128, None, 0, 8, 1024, 8, 256, None, 0, None)
    assert rc == -95
    rc = h.mxk_qgemm(8, 8, 1, 8, 8, 1, 4, 4, 4, 16, 128, 0, None, 0, None, 8, None, None, 0, None)
    assert rc == -95
    rc = h.mxk_linear_prepack_scales(None, 256, 256, 128, 8, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_prepack_scales(8, 256, 200, 128, 8, None)
    assert rc == -22
    rc = h.mxk_linear_prepack_scales(8, 256, 256, 64, 8, None)
    assert rc == -22
    rc = h.mxk_linear_prepack_weight(None, 256, 256, 4, 128, 16, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_prepack_weight(16, 256, 200, 4, 128, 16, None)   # N not a multiple of 128
    assert rc == -22
    rc = h.mxk_linear_prepack_weight(16, 256, 256, 8, 128, 16, None)   # int8 codes
    assert rc == -22
    rc = h.mxk_linear_prepack_weight(16, 256, 256, 4, 128, 8, None)    # w_tiled not 16-byte aligned
    assert rc == -22
    rc = h.mxk_linear_wq_tiled(16, 0, 16, 256, None, 16, 256, 0, None, 16, None, 0, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_wq_tiled(16, 7, 16, 256, 16, 16, 256, 0, None, 16, None, 0, None)   # bad x type
    assert rc == -22
    rc = h.mxk_linear_wq_tiled(16, 0, 16, 256, 16, 16, 256, 5, None, 16, None, 0, None)   # bad kind
    assert rc == -22 and b"kind" in h.mxk_last_error()
    # M > 16 runs the MFMA path on the tiled copy, which needs its workspace
    rc = h.mxk_linear_wq_tiled(16, 0, 17, 256, 16, 16, 256, 0, None, 16, None, 0, None)
    assert rc == -22 and b"workspace" in h.mxk_last_error()
    rc = h.mxk_linear_wq_tiled(16, 0, 16, 256, 16, 16, 200, 0, None, 16, None, 0, None)   # N % 128
    assert rc == -95
    rc = h.mxk_linear_prepack_weight_nt(None, 256, 256, 4, 128, 16, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_prepack_weight_nt(16, 200, 256, 4, 128, 16, None)   # N not a multiple of 128
    assert rc == -22
    rc = h.mxk_linear_prepack_weight_nt(16, 256, 192, 4, 128, 16, None)   # K not a multiple of 128
    assert rc == -22
    rc = h.mxk_linear_prepack_weight_nt(16, 256, 256, 2, 128, 16, None)   # int2 codes
    assert rc == -22
    rc = h.mxk_linear_prepack_weight_nt(8, 256, 256, 4, 128, 16, None)    # w_packed not 16-byte aligned
    assert rc == -22
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 16, 256, None, 16, 256, None, 16, None, 0, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_wq_nt_tiled(16, 5, 16, 256, 16, 16, 256, None, 16, None, 0, None)   # bad x type
    assert rc == -22
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 16, 256, 16, 16, 256, 8, 16, None, 0, None)     # misaligned bias
    assert rc == -22
    # M > 16 runs the MFMA path on the tiled copy, which needs its workspace
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 17, 256, 16, 16, 256, None, 16, None, 0, None)
    assert rc == -22 and b"workspace" in h.mxk_last_error()
    rc = h.mxk_linear_unpack_weight_nt(None, 256, 256, 4, 128, 16, None)
    assert rc == -22 and b"null" in h.mxk_last_error()
    rc = h.mxk_linear_unpack_weight_nt(16, 256, 192, 4, 128, 16, None)   # K not a multiple of 128
    assert rc == -22
    rc = h.mxk_linear_unpack_weight_nt(16, 256, 256, 4, 128, 8, None)    # w_packed not 16-byte aligned
    assert rc == -22
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 16, 192, 16, 16, 256, None, 16, None, 0, None)  # K % 128
    assert rc == -95
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 16, 256, 16, 16, 200, None, 16, None, 0, None)  # N % 128
    assert rc == -95
    # K = 4096: two splits, so the call needs its workspace
    rc = h.mxk_linear_wq_nt_tiled(16, 0, 16, 4096, 16, 16, 256, None, 16, None, 0, None)
    assert rc == -22 and b"workspace" in h.mxk_last_error()


def test_decode_workspace_limits():
    """The int4 decode path counts split arrivals in 8 bits per XCC, so it
    takes no shape that would need more than 255 splits.  Covered shapes get
    a workspace with the 64 KiB counter prefix."""
    from qtpytorch_amd import _lib as L
    h = L.lib()
    assert h.mxk_linear_workspace(16, 8192, 8192, 4, 128) >= 65536
    assert h.mxk_linear_workspace(1, 2048 * 255, 128, 4, 128) > 0
    # past the decode kernels' limits (more than 16 rows, 293 splits, other
    # formats) the MFMA path takes 1-, 2-, 4- and 8-bit codes: its row exponents,
    # scaled x (fp32), scaled scales and any split partials follow the 64 KiB
    # counter prefix, which it leaves alone
    for M, K, N, bits in ((17, 8192, 8192, 4), (1, 600000, 128, 4), (512, 8192, 8192, 8), (16, 4096, 256, 8),
                          (64, 8192, 8192, 2), (64, 8192, 8192, 1)):
        Kp = -(-K // 256) * 256
        assert h.mxk_linear_workspace(M, K, N, bits, 128) >= 65536 + M * Kp * 4 + (N // 128) * Kp * 4
    for bits in (3, 5, 16):
        assert h.mxk_linear_workspace(64, 8192, 8192, bits, 128) == 0  # other widths: generic kernel, no workspace
    assert h.mxk_linear_workspace(64, 8192, 8000, 4, 128) == 0     # N not whole 128-column blocks
    # [out, in] weights: K must be whole blocks of 128; x as f16 hi + lo
    assert h.mxk_linear_nt_workspace(64, 8192, 8192, 4, 128) >= 65536 + 64 * 8192 * 4
    assert h.mxk_linear_nt_workspace(64, 8000, 8192, 4, 128) == 0


def test_qgemm_workspace_queries():
    """mxk_qgemm_workspace sizes the workspace for packed operands on 16
    bytes; mxk_qgemm_workspace_any for any alignment (misaligned operands
    are unpacked into it first).  With N a multiple of 128 the int16 / int8
    requantization runs in the GEMM's epilogue: no M*N float32 buffer."""
    from qtpytorch_amd import _lib as L
    h = L.lib()
    M = K = N = 8192
    for bits, ob in ((8, 16), (4, 8)):
        fused = h.mxk_qgemm_workspace(M, K, N, bits, 128, ob)
        c_only = h.mxk_qgemm_workspace(M, K, N, bits, 128, 0)
        assert fused == c_only < M * N * 4          # no C buffer for the packed output
        assert h.mxk_qgemm_workspace_any(M, K, N, bits, 128, ob) >= fused + M * N * 4
    # N not whole 128-column blocks: a second pass over an fp32 C buffer
    assert h.mxk_qgemm_workspace(M, K, 8160, 8, 128, 16) >= M * 8160 * 4
    # the misaligned call names the other query
    rc = h.mxk_qgemm(8, 8, M * (K // 128), 24, 8, (K // 128) * N, M, K, N, 8, 128, 16, 16, M * N * 2, 16, None,
                     None, 16, h.mxk_qgemm_workspace(M, K, N, 8, 128, 16), None)
    assert rc == -22 and b"mxk_qgemm_workspace_any" in h.mxk_last_error()
