"""CPU oracle for the mxtorch quantize / pack / block-scaled GEMM path.

TEST INFRASTRUCTURE ONLY.  This module is the parity checker: only the test
suite (tests/), ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package ``qtpytorch_amd`` never
imports, links or calls anything under ``oracle/``; on a GPU it runs the HIP
kernels in ``libmxk.so`` and fails loudly when that library is missing.

What it is: a restatement of the reference's CPU path (mxtorch.py, one
module, referenced below as ``mxtorch.py:LINE``) written with the same torch
CPU operators in the same order, so that every intermediate is rounded the
way the reference rounds it.  The arithmetic of the reference lives in torch
CPU kernels (torch is the third-party dependency; the reference pins no
version, this restatement runs on the torch in this image).  The facts it
relies on are pinned by tests in tests/test_oracle_*.py:

  * ``scalar / tensor`` is ``tensor.reciprocal() * scalar``
    (torch/_tensor.py ``__rdiv__``), so the int quantizer rounds twice:
    inv = fl(fl(1/a)*q), s = fl(1/inv)  (mxtorch.py:1458-1459);
  * ``tensor / python_float`` on CPU is an IEEE division by fl32(value);
  * ``round`` is round-half-to-even; ``bucketize`` (right=False) returns the
    number of boundaries strictly below the value.

Every function cites the reference lines it restates.  Pins (golden vectors
written by importing the reference, the reference's own pack KATs, closed
forms, brute force) are listed in the header of each test module.
"""
from __future__ import annotations

import functools
import math
import re
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

# ---------------------------------------------------------------------------
# dtype names  (mxtorch.py:413-547, 567-581)
# ---------------------------------------------------------------------------
_NAME_RE = re.compile(r"^(int|float)(1|2|3|4|5|6|7|8|16|32|64|128)(d|u)(h|v|s|b|2)?$")


def parse_dtype(name: str):
    """Split an mxtorch dtype name into (kind, bits, mode, variant).

    mxtorch.py:464-466 builds names as f"{kind}{bits}{mode}{variant}";
    get_mx_dtype raises ValueError on anything else (mxtorch.py:577-581).
    """
    m = _NAME_RE.match(name)
    if m is None:
        raise ValueError(f"Unknown MX dtype {name!r}")
    kind, bits, mode, variant = m.group(1), int(m.group(2)), m.group(3), m.group(4) or ""
    return kind, bits, mode, variant


def max_val(name: str) -> float:
    """mx_dtype.max_val (mxtorch.py:509-523)."""
    kind, bits, _, variant = parse_dtype(name)
    if variant == "b":
        return 1.0
    if kind == "int":
        return 1.0 if bits == 1 else float((1 << (bits - 1)) - 1)
    fmax = {1: 1.0, 2: 1.5, 3: 3.5, 4: 6.0, 5: 14.0, 6: 28.0, 7: 56.0, 8: 448.0, 16: 65504.0}
    return fmax.get(bits, float("inf"))


# ---------------------------------------------------------------------------
# bit packing  (mxtorch.py:870-985)
# ---------------------------------------------------------------------------
def pack(vals: Tensor, bits: int) -> Tensor:
    """bit_packer.pack (mxtorch.py:882-910): LSB-first fields in int8 bytes."""
    assert bits in (1, 2, 4, 8)
    if bits == 8:
        return vals.to(torch.int8)
    ratio = 8 // bits
    n = vals.numel()
    pad = (-n) % ratio
    if pad:
        vals = torch.cat([vals.flatten(), vals.new_zeros(pad, dtype=vals.dtype)])
    vals = vals.flatten().to(torch.int8)
    mask = (1 << bits) - 1
    packed = torch.zeros(vals.numel() // ratio, dtype=torch.int8)
    for i in range(ratio):
        slot = (vals[i::ratio] & mask).to(torch.int8)
        packed = packed | (slot << (i * bits))
    return packed


def unpack(packed: Tensor, bits: int, n: int) -> Tensor:
    """bit_packer.unpack (mxtorch.py:912-935): sign-extended codes as float32."""
    assert bits in (1, 2, 4, 8)
    if bits == 8:
        return packed[:n].to(torch.float32)
    ratio = 8 // bits
    mask = (1 << bits) - 1
    sign = 1 << (bits - 1)
    out = torch.empty(len(packed) * ratio, dtype=torch.int8)
    for i in range(ratio):
        slot = ((packed >> (i * bits)) & mask).to(torch.int8)
        signed = torch.where((slot.to(torch.int16) & sign) != 0,
                             (slot.to(torch.int16) | (~mask & 0xFF)).to(torch.int8), slot)
        out[i::ratio] = signed
    return out[:n].to(torch.float32)


def pack_arb(vals: Tensor, bits: int) -> Tensor:
    """bit_packer.pack_arb (mxtorch.py:939-955): floor(32/bits) fields per int32 word."""
    if bits in (1, 2, 4, 8):
        return pack(vals.to(torch.int8), bits)
    ratio = 32 // bits
    n = vals.numel()
    pad = (-n) % ratio
    if pad:
        vals = torch.cat([vals.flatten(), vals.new_zeros(pad, dtype=vals.dtype)])
    v32 = vals.flatten().to(torch.int32)
    mask = (1 << bits) - 1
    packed = torch.zeros(len(v32) // ratio, dtype=torch.int32)
    for i in range(ratio):
        packed |= (v32[i::ratio] & mask) << (i * bits)
    return packed


def unpack_arb(packed: Tensor, bits: int, n: int) -> Tensor:
    """bit_packer.unpack_arb (mxtorch.py:957-972)."""
    if bits in (1, 2, 4, 8):
        return unpack(packed.view(torch.int8) if packed.dtype != torch.int8 else packed, bits, n)
    ratio = 32 // bits
    mask = (1 << bits) - 1
    sign = 1 << (bits - 1)
    out = torch.empty(len(packed) * ratio, dtype=torch.int32)
    for i in range(ratio):
        slot = (packed >> (i * bits)) & mask
        signed = torch.where((slot & sign) != 0, slot | ~mask, slot)
        out[i::ratio] = signed
    return out[:n].to(torch.float32)


def pack_auto(vals: Tensor, bits: int) -> Tensor:
    """bit_packer.pack_auto (mxtorch.py:976-980)."""
    if bits in (1, 2, 4, 8):
        return pack(vals.to(torch.int8), bits)
    return pack_arb(vals, bits)


def unpack_auto(packed: Tensor, bits: int, n: int) -> Tensor:
    """bit_packer.unpack_auto (mxtorch.py:982-985)."""
    if bits in (1, 2, 4, 8):
        return unpack(packed.to(torch.int8), bits, n)
    return unpack_arb(packed.to(torch.int32), bits, n)


# ---------------------------------------------------------------------------
# mini-float grids  (mxtorch.py:992-1054)
# ---------------------------------------------------------------------------
@functools.lru_cache(maxsize=8)
def float_grid(bits: int) -> Tensor:
    """_get_minifloat_grid for the FP4 E2M1 and FP8 E4M3 cases.

    FP4: mxtorch.py:1023-1035.  FP8 (exponent 15 treated as a normal
    binade, max 480): mxtorch.py:1038-1054.
    """
    if bits == 4:
        pos = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float32)
        scale = pos.abs().max().clamp(min=1e-9)
        pos_n = pos / scale
        neg_n = -pos_n.flip(0)
        grid = torch.cat([neg_n, pos_n])
        return grid.sort().values
    if bits == 8:
        vals = []
        for code in range(256):
            sign = -1.0 if (code >> 7) else 1.0
            e = (code >> 3) & 0xF
            m = code & 0x7
            if e == 0:
                v = sign * (m / 8.0) * (2.0 ** -6)
            elif e == 0xF:
                v = sign * (1.0 + m / 8.0) * (2.0 ** 8)
            else:
                v = sign * (1.0 + m / 8.0) * (2.0 ** (e - 7))
            vals.append(v)
        raw = torch.tensor(vals, dtype=torch.float32)
        scale = raw.abs().max().clamp(min=1e-9)
        return (raw / scale).sort().values
    if bits == 16:
        # every non-NaN/Inf half-precision value (NaN/Inf codes become 0.0),
        # normalised by the largest magnitude (mxtorch.py:1117-1143); this
        # is what float16d GEMM outputs (float8d @ float8d) dequantize with.
        import numpy as np
        h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
        h[~np.isfinite(h)] = 0.0
        raw = torch.from_numpy(h)
        mx = raw.abs().max().clamp(min=1e-9)
        return (raw / mx).sort().values
    raise NotImplementedError(f"oracle grid for float{bits}")


def float_mids(bits: int) -> Tensor:
    """Bucket boundaries used by _quant_float (mxtorch.py:1523)."""
    g = float_grid(bits)
    return (g[:-1] + g[1:]) * 0.5


# ---------------------------------------------------------------------------
# quantizers  (mxtorch.py:1426-1528, 1684-1763)
# ---------------------------------------------------------------------------
def _blocks(x: Tensor, block: int):
    flat = x.float().reshape(-1)
    n = flat.numel()
    nb = math.ceil(n / block)
    pad = nb * block - n
    if pad:
        flat = torch.cat([flat, flat.new_zeros(pad)])
    return flat.reshape(nb, block), n


def quant_int(x: Tensor, bits: int, block: int) -> Tuple[Tensor, Tensor, int]:
    """_quant_int (mxtorch.py:1426-1463)."""
    blk, n = _blocks(x, block)
    if bits == 1:  # mxtorch.py:1442-1454
        scales = blk.abs().amax(dim=1).clamp(min=1e-12)
        codes = torch.where(blk >= 0, torch.zeros_like(blk, dtype=torch.int32),
                            torch.full_like(blk, -1, dtype=torch.int32))
        return pack_auto(codes.reshape(-1), bits), scales, n
    max_int = float((1 << (bits - 1)) - 1)
    scale_inv = max_int / blk.abs().amax(dim=1).clamp(min=1e-12)   # reciprocal() * max_int
    scales = scale_inv.reciprocal()
    codes = (blk * scale_inv.unsqueeze(1)).clamp(-max_int, max_int).round_().to(torch.int32)
    return pack_auto(codes.reshape(-1), bits), scales, n


def quant_float(x: Tensor, bits: int, block: int) -> Tuple[Tensor, Tensor, int]:
    """_quant_float for sub-16-bit grids (mxtorch.py:1465-1528)."""
    blk, n = _blocks(x, block)
    scales = blk.abs().amax(dim=1).clamp(min=1e-12)
    normed = blk / scales.unsqueeze(1)
    grid = float_grid(bits)
    flat = normed.reshape(-1)
    mids = (grid[:-1] + grid[1:]) * 0.5
    idx = torch.bucketize(flat, mids)
    codes = idx.to(torch.int32)
    return pack_auto(codes, bits), scales, n


def quant_vector(x: Tensor, name: str, block: int) -> Tuple[Tensor, Tensor, int]:
    """The 'v' (per-row) branch of quantize (mxtorch.py:1739-1752)."""
    _, bits, _, _ = parse_dtype(name)
    blk, n = _blocks(x, block)
    mx = max_val(name)
    scales = blk.abs().amax(dim=1).clamp(min=1e-12) / mx
    codes = (blk / scales.unsqueeze(1)).clamp(-mx, mx).round_().to(torch.int32)
    return pack_auto(codes.reshape(-1), bits), scales, n


# ---------------------------------------------------------------------------
# Hadamard rotation  (mxtorch.py:2811-2904)
# ---------------------------------------------------------------------------
def hadamard_signs(n: int, seed: int) -> Tensor:
    """hadamard_rotation.__init__ sign vector (mxtorch.py:2856-2864)."""
    gen = torch.Generator()
    gen.manual_seed(seed)
    return torch.randint(0, 2, (n,), generator=gen).float() * 2 - 1


@functools.lru_cache(maxsize=None)
def reference_hadamard_seed(name: str) -> int:
    """The seed quantize() derives for 'h' dtypes, ``hash(name) % 2**31``
    (mxtorch.py:1723), as it evaluates in a Python process started with
    PYTHONHASHSEED=0: the expression is run in such a subprocess of this
    interpreter.  (``hash(str)`` is salted per process otherwise, so the
    reference's own seed changes from run to run.)"""
    import subprocess
    import sys
    out = subprocess.run([sys.executable, "-c", f"print(hash({name!r}) % (2 ** 31))"],
                         env={"PYTHONHASHSEED": "0", "PATH": "/usr/bin:/bin"}, capture_output=True, text=True,
                         check=True)
    return int(out.stdout.strip())


def fwht(x: Tensor) -> Tensor:
    """_fast_hadamard_transform (mxtorch.py:2811-2832): butterflies with
    half-width n/2, n/4, ..., 1 along the last dim, then an IEEE division by
    fl32(sqrt(n))."""
    n = x.shape[-1]
    assert (n & (n - 1)) == 0
    orig_shape = x.shape
    h = x.reshape(-1, n).clone()
    h2 = n
    while h2 > 1:
        h2 //= 2
        h = h.reshape(h.shape[0], -1, 2 * h2)
        even = h[..., :h2]
        odd = h[..., h2:]
        h = torch.cat([even + odd, even - odd], dim=-1)
    return h.reshape(*orig_shape[:-1], n) / math.sqrt(n)


def _pow2_ceil(d: int) -> int:
    return 1 << math.ceil(math.log2(max(d, 1)))


def rotate(x: Tensor, signs: Tensor) -> Tensor:
    """hadamard_rotation.rotate (mxtorch.py:2866-2889); ``signs`` has the
    rotation's power-of-two length."""
    d = x.shape[-1]
    n = _pow2_ceil(d)
    x_f = x.float()
    if n != d:
        x_f = F.pad(x_f, (0, n - d))
    s = signs if d == signs.numel() else signs[:d].sign()
    sp = F.pad(s, (0, n - len(s)), value=1.0) if n > len(s) else s[:n]
    return fwht(x_f * sp)[..., :d]


def unrotate(x: Tensor, signs: Tensor) -> Tensor:
    """hadamard_rotation.unrotate (mxtorch.py:2891-2904)."""
    d = x.shape[-1]
    n = _pow2_ceil(d)
    x_f = x.float()
    if n != d:
        x_f = F.pad(x_f, (0, n - d))
    x_rot = fwht(x_f)
    s = signs if d == signs.numel() else signs[:d].sign()
    sp = F.pad(s, (0, n - len(s)), value=1.0) if n > len(s) else s[:n]
    return (x_rot * sp)[..., :d]


def rotation_dim(shape) -> int:
    """The rotated length quantize() picks (mxtorch.py:1721)."""
    shape = tuple(shape)
    if len(shape) >= 2:
        return shape[-1]
    return int(math.prod(shape))


# ---------------------------------------------------------------------------
# quantize / dequantize dispatch  (mxtorch.py:1530-1597, 1684-1763)
# ---------------------------------------------------------------------------
def quantize(x: Tensor, name: str, block: int = 128, seed: Optional[int] = None
             ) -> Tuple[Tensor, Tensor, int]:
    """quantize() CPU branch (mxtorch.py:1684-1763) for the base, 'h' and 'v'
    variants.  For 'h' the seed defaults to the reference's hash-derived one as it
    evaluates under PYTHONHASHSEED=0."""
    kind, bits, mode, variant = parse_dtype(name)
    base = f"{kind}{bits}{mode}"
    x_f = x.float()
    if variant == "h":
        d = x_f.shape[-1] if x_f.ndim >= 2 else x_f.numel()
        if seed is None:
            seed = reference_hadamard_seed(name)
        signs = hadamard_signs(_pow2_ceil(d), seed)
        x_rot = rotate(x_f, signs)
        return quant_int(x_rot, bits, block) if kind == "int" else quant_float(x_rot, bits, block)
    if variant == "v":
        return quant_vector(x_f, name, block)
    if variant != "":
        raise NotImplementedError(f"oracle variant {variant!r}")
    if kind == "int":
        return quant_int(x_f, bits, block)
    return quant_float(x_f, bits, block)


def dequant(packed: Tensor, scales: Tensor, name: str, n: int, block: int,
            seed: Optional[int] = None, orig_shape=None, hadamard_mode: str = "reference"
            ) -> Tensor:
    """_dequant (mxtorch.py:1530-1597).

    hadamard_mode="reference" reproduces the reference's unrotation over the
    whole flattened tensor (d = numel, mxtorch.py:1582-1595).  "rows"
    unrotates each row of length rotation_dim(orig_shape), i.e. the inverse
    of what quantize() rotated; both agree for 1-D tensors.
    """
    kind, bits, _, variant = parse_dtype(name)
    codes = unpack_auto(packed, bits, n)
    nb = scales.numel()
    pad = nb * block - n
    if pad > 0:
        codes = torch.cat([codes, codes.new_zeros(pad)])
    elif pad < 0:
        codes = codes[:nb * block]
    blk = codes.reshape(nb, block)
    if kind == "int" and bits == 1 and variant != "b":
        dq = torch.where(blk == 0, torch.ones_like(blk, dtype=torch.float32),
                         torch.full_like(blk, -1.0, dtype=torch.float32))
    elif kind == "float":
        mask = (1 << bits) - 1
        indices = (blk.to(torch.int64) & mask).long()
        grid = float_grid(bits)
        indices = indices.clamp(0, len(grid) - 1)
        dq = grid[indices]
    else:
        dq = blk
    flat = (dq * scales.unsqueeze(1)).reshape(-1)[:n]
    if variant == "h":
        if seed is None:
            seed = reference_hadamard_seed(name)
        if hadamard_mode == "reference" or orig_shape is None:
            d = flat.numel()
            n2 = _pow2_ceil(d)
            signs = hadamard_signs(n2, seed)
            flat = unrotate(flat.unsqueeze(0), signs).squeeze(0)[:d]
        else:
            d = rotation_dim(orig_shape)
            signs = hadamard_signs(_pow2_ceil(d), seed)
            flat = unrotate(flat.reshape(-1, d), signs).reshape(-1)
    return flat


# ---------------------------------------------------------------------------
# GEMM  (mxtorch.py:1299-1423, 5497-5573)
# ---------------------------------------------------------------------------
_VALID_BITS = (1, 2, 3, 4, 5, 6, 7, 8, 16, 32, 64, 128)


def matmul_out_bits(a_bits: int, b_bits: int) -> int:
    """_optimal_output_dtype("matmul", ...) bit width (mxtorch.py:1393-1418)."""
    ideal = min(32, a_bits + b_bits)
    return min(_VALID_BITS, key=lambda x: (abs(x - ideal), -x))


def qscale_matmul(a_codes: Tensor, a_scales: Tensor, b_codes: Tensor, b_scales: Tensor,
                  M: int, K: int, N: int, bits: int, block: int, out_bits: int,
                  return_c: bool = False):
    """_qscale_matmul (mxtorch.py:1299-1385).

    Returns (codes [M*N] int32, scales [ceil(M*N/block)]); with return_c the
    fp32 accumulator C [M, N] before requantization is returned as well.
    """
    max_out = float((1 << (out_bits - 1)) - 1)
    a_mat = a_codes.reshape(M, K).float()
    b_mat = b_codes.reshape(K, N).float()
    kba = math.ceil(K / block)
    c_mat = torch.zeros(M, N, dtype=torch.float32)
    a_s = a_scales.reshape(M, kba) if a_scales.numel() == M * kba else a_scales.new_ones(M, kba)
    b_s = b_scales.reshape(kba, N) if b_scales.numel() == kba * N else b_scales.new_ones(kba, N)
    for kb in range(kba):
        k0, k1 = kb * block, min(kb * block + block, K)
        prod = torch.mm(a_mat[:, k0:k1], b_mat[k0:k1, :])
        c_mat += prod * a_s[:, kb].unsqueeze(1) * b_s[kb, :].unsqueeze(0)
    nb_c = math.ceil(M * N / block)
    c_flat = c_mat.reshape(-1)
    pad = nb_c * block - c_flat.numel()
    c_p = torch.cat([c_flat, c_flat.new_zeros(pad)]) if pad else c_flat
    c_blk = c_p.reshape(nb_c, block)
    c_scale = c_blk.abs().amax(dim=1).clamp(min=1e-12) / max_out
    c_codes = (c_blk / c_scale.unsqueeze(1)).clamp(-max_out, max_out).round_()
    c_codes = c_codes.to(torch.int32).reshape(-1)[:M * N]
    if return_c:
        return c_codes, c_scale, c_mat
    return c_codes, c_scale


def int_accumulators(a_codes: Tensor, b_codes: Tensor, M: int, K: int, N: int, block: int) -> Tensor:
    """Per-K-block exact integer products P[kb] = A[:, kb] @ B[kb, :]
    (the ``int_prod`` of mxtorch.py:1365), as int32 [KB, M, N]."""
    a = a_codes.reshape(M, K).to(torch.int64)
    b = b_codes.reshape(K, N).to(torch.int64)
    kba = math.ceil(K / block)
    out = torch.empty(kba, M, N, dtype=torch.int32)
    for kb in range(kba):
        k0, k1 = kb * block, min(kb * block + block, K)
        out[kb] = (a[:, k0:k1] @ b[k0:k1, :]).to(torch.int32)
    return out


def dispatch_qgemm(a_packed: Tensor, a_scales: Tensor, a_name: str, a_shape, a_n: int,
                   b_packed: Tensor, b_scales: Tensor, b_name: str, b_shape, b_n: int,
                   block: int, return_c: bool = False):
    """_dispatch_qgemm CPU branch (mxtorch.py:5497-5573): both operands are
    unpacked with a's bit width (mxtorch.py:5564-5565).  Returns
    (packed, scales, out_name[, C])."""
    M, K = a_shape
    K2, N = b_shape
    assert K == K2
    ak, abits, amode, _ = parse_dtype(a_name)
    bk, bbits, bmode, _ = parse_dtype(b_name)
    out_bits = matmul_out_bits(abits, bbits)
    kind = "float" if (ak == "float" or bk == "float") else "int"
    mode = "u" if (amode == "u" or bmode == "u") else "d"
    out_name = f"{kind}{out_bits}{mode}"
    a_codes = unpack_auto(a_packed, abits, a_n).to(torch.int32)
    b_codes = unpack_auto(b_packed, abits, b_n).to(torch.int32)
    res = qscale_matmul(a_codes, a_scales, b_codes, b_scales, M, K, N, abits, block,
                        out_bits, return_c=return_c)
    packed = pack_auto(res[0], out_bits)
    if return_c:
        return packed, res[1], out_name, res[2]
    return packed, res[1], out_name


def qgemm_ste_forward(a: Tensor, b: Tensor, name: str, block: int) -> Tensor:
    """_QGemmSTE.forward (mxtorch.py:5295-5303): quantize both, packed GEMM,
    dequantize the requantized output."""
    pa, sa, na = quantize(a, name, block)
    pb, sb, nb = quantize(b, name, block)
    pc, sc, out_name = dispatch_qgemm(pa, sa, name, a.shape, na, pb, sb, name, b.shape, nb, block)
    M, N = a.shape[0], b.shape[1]
    return dequant(pc, sc, out_name, M * N, block).reshape(M, N)


# ---------------------------------------------------------------------------
# callers  (mxtorch.py:7439-7473, 3039-3086)
# ---------------------------------------------------------------------------
def linear_from_weight(weight: Tensor, name: str, block: int = 128):
    """mx_linear.from_linear weight storage (mxtorch.py:7439-7452):
    quantize(W.t()) -> [in, out] row-major, blocks along out."""
    return quantize(weight.t(), name, block)


def linear_forward(x: Tensor, w_packed: Tensor, w_scales: Tensor, name: str,
                   in_features: int, out_features: int, block: int = 128,
                   has_bias: bool = False) -> Tensor:
    """mx_linear.forward (mxtorch.py:7454-7473).  A bias, when present, is
    re-quantized from zeros on every call (mxtorch.py:7434-7436), so it adds
    dequant(quantize(zeros))."""
    x_f = x.float()
    w_f = dequant(w_packed, w_scales, name, in_features * out_features, block
                  ).reshape(in_features, out_features)
    b_f = None
    if has_bias:
        pb, sb, nb = quantize(torch.zeros(out_features), name, block)
        b_f = dequant(pb, sb, name, nb, block)
    return F.linear(x_f, w_f.t(), b_f)


def kv_append(k: Tensor, v: Tensor, name: str, head_dim: int, asymmetric_v: bool = True):
    """kv_cache_quantizer.append_kv for one step (mxtorch.py:3039-3067).
    Returns ((k_packed, k_scales, k_n), (v_packed, v_scales, v_n), v_zero_point)."""
    k_f = k.float().reshape(-1, head_dim)
    v_f = v.float().reshape(-1, head_dim)
    kq = quantize(k_f, name, head_dim)
    if asymmetric_v:
        v_min = v_f.min(dim=1, keepdim=True).values
        vq = quantize(v_f - v_min, name, head_dim)
        return kq, vq, v_min.squeeze(1)
    return kq, quantize(v_f, name, head_dim), None


def kv_get(steps, name: str, head_dim: int, n_heads: int):
    """kv_cache_quantizer.get (mxtorch.py:3069-3086); ``steps`` is a list of
    kv_append results."""
    ks, vs, zps = [], [], []
    for kq, vq, zp in steps:
        rows = kq[2] // head_dim
        ks.append(dequant(kq[0], kq[1], name, kq[2], head_dim).reshape(rows, head_dim))
        vs.append(dequant(vq[0], vq[1], name, vq[2], head_dim).reshape(rows, head_dim))
        if zp is not None:
            zps.append(zp)
    T = len(steps)
    k_all = torch.stack(ks, dim=1)
    v_all = torch.stack(vs, dim=1)
    if zps:
        v_all = v_all + torch.stack(zps, dim=1).unsqueeze(-1)
    BH, _, D = k_all.shape
    return k_all.reshape(-1, n_heads, T, D), v_all.reshape(-1, n_heads, T, D)


# ---------------------------------------------------------------------------
# Quantized element-wise arithmetic  (mxtorch.py:1186-1296, 5321-5497, 6177-6193)
# ---------------------------------------------------------------------------
def resolve_mixed(a_name: str, b_name: str) -> str:
    """_resolve_mixed (mxtorch.py:584-598): mode u if either is u, the
    narrower width, float if either is float, the higher-priority variant
    (h > v > s > b > '')."""
    ak, ab, am, av = parse_dtype(a_name)
    bk, bb, bm, bv = parse_dtype(b_name)
    prio = {"h": 4, "v": 3, "s": 2, "b": 1, "": 0}
    mode = "u" if (am == "u" or bm == "u") else "d"
    bits = min(ab, bb)
    kind = "float" if (ak == "float" or bk == "float") else "int"
    variant = av if prio.get(av, 0) >= prio.get(bv, 0) else bv
    bits = min(_VALID_BITS, key=lambda x: abs(x - bits))
    return f"{kind}{bits}{mode}{variant}"


def qmul_out_name(name: str) -> str:
    """Output dtype of _dispatch_qmul (mxtorch.py:5442-5445): {kind}{w}d with
    w the valid width nearest min(2*bits, 16), ties to the wider."""
    kind, bits, _, _ = parse_dtype(name)
    ideal = min(bits * 2, 16)
    w = min(_VALID_BITS, key=lambda x: (abs(x - ideal), -x))
    return f"{kind}{w}d"


def _pad_blocks(codes: Tensor, nb: int, block: int) -> Tensor:
    n = codes.numel()
    if n < nb * block:
        codes = torch.cat([codes, torch.zeros(nb * block - n, dtype=codes.dtype)])
    return codes


def qscale_add(a_codes: Tensor, a_scales: Tensor, b_codes: Tensor, b_scales: Tensor,
               bits: int, block: int) -> Tuple[Tensor, Tensor]:
    """_qscale_add (mxtorch.py:1186-1256): per block, integer-domain add when
    the scales are within 2:1 (rescaled to the larger scale, doubled once on
    overflow), else dequantize, add and requantize with the 'v' rule."""
    max_int = float((1 << (bits - 1)) - 1)
    nb = a_scales.numel()
    ac = _pad_blocks(a_codes, nb, block).reshape(nb, block).float()
    bc = _pad_blocks(b_codes, nb, block).reshape(nb, block).float()
    sa = a_scales.unsqueeze(1)
    sb = b_scales.unsqueeze(1)
    ratio = torch.max(sa, sb) / torch.min(sa, sb).clamp(min=1e-30)
    use_int = (ratio <= 2.0).squeeze(1)
    out_codes = torch.zeros(nb * block, dtype=torch.int32)
    out_scales = torch.zeros(nb, dtype=torch.float32)
    if use_int.any():
        idx = use_int.nonzero(as_tuple=True)[0]
        sc_i = torch.maximum(sa[idx], sb[idx])
        ac_r = (ac[idx] * (sa[idx] / sc_i)).round_()
        bc_r = (bc[idx] * (sb[idx] / sc_i)).round_()
        c_w = ac_r + bc_r
        overflow = c_w.abs().amax(dim=1) > max_int
        if overflow.any():
            sc_i = sc_i.clone()
            sc_i[overflow] *= 2.0
            ac_r = (ac[idx] * (sa[idx] / sc_i)).round_()
            bc_r = (bc[idx] * (sb[idx] / sc_i)).round_()
            c_w = ac_r + bc_r
        out_codes.view(nb, block)[idx] = c_w.clamp(-max_int, max_int).to(torch.int32)
        out_scales[idx] = sc_i.squeeze(1)
    if (~use_int).any():
        idx2 = (~use_int).nonzero(as_tuple=True)[0]
        sum_f = ac[idx2] * sa[idx2] + bc[idx2] * sb[idx2]
        sc_f = sum_f.abs().amax(dim=1).clamp(min=1e-12) / max_int
        c_f = (sum_f / sc_f.unsqueeze(1)).clamp(-max_int, max_int).round_()
        out_codes.view(nb, block)[idx2] = c_f.to(torch.int32)
        out_scales[idx2] = sc_f
    return out_codes, out_scales


def qscale_mul(a_codes: Tensor, a_scales: Tensor, b_codes: Tensor, b_scales: Tensor,
               bits: int, block: int) -> Tuple[Tensor, Tensor]:
    """_qscale_mul (mxtorch.py:1259-1296): codes rne(clamp(RN(RN(a*b)/max_int))),
    scales RN(RN(sa*sb)*max_int)."""
    max_int = float((1 << (bits - 1)) - 1)
    nb = a_scales.numel()
    ac = _pad_blocks(a_codes, nb, block).reshape(nb, block).float()
    bc = _pad_blocks(b_codes, nb, block).reshape(nb, block).float()
    prod = ac * bc
    prod_scales = a_scales * b_scales * max_int
    c_codes = (prod / max_int).clamp(-max_int, max_int).round().to(torch.int32)
    return c_codes.reshape(-1), prod_scales


def dispatch_qelementwise(op: str, a_packed: Tensor, a_scales: Tensor, a_name: str, b_packed: Tensor,
                          b_scales: Tensor, b_name: str, n: int, block: int):
    """CPU branches of _dispatch_qadd / _dispatch_qsub / _dispatch_qmul
    (mxtorch.py:5397-5401, 5425-5431, 5489-5497): both operands unpacked with
    a's width, the codes packed with the output dtype's width.  Returns
    (packed, scales, out_name)."""
    _, bits, _, _ = parse_dtype(a_name)
    ac = unpack_auto(a_packed, bits, n).to(torch.int32)
    bc = unpack_auto(b_packed, bits, n).to(torch.int32)
    if op == "mul":
        out = qmul_out_name(a_name)
        c, s = qscale_mul(ac, a_scales, bc, b_scales, bits, block)
    else:
        out = resolve_mixed(a_name, b_name)
        c, s = qscale_add(ac, a_scales, (-bc).to(torch.int32) if op == "sub" else bc, b_scales, bits, block)
    return pack_auto(c, parse_dtype(out)[1]), s, out


def negate(packed: Tensor, scales: Tensor, name: str, n: int) -> Tuple[Tensor, Tensor]:
    """mx_tensor.__neg__ (mxtorch.py:6177-6193): 8-bit codes negate every
    stored byte (clamped to +-127); other widths unpack n codes, negate,
    clamp and repack.  Scales are copied."""
    _, bits, _, _ = parse_dtype(name)
    max_i = (1 << (bits - 1)) - 1
    if bits == 8:
        return (-packed.to(torch.int16)).clamp(-max_i, max_i).to(torch.int8), scales.clone()
    codes = unpack_auto(packed, bits, n).to(torch.int32)
    return pack_auto((-codes).clamp(-max_i, max_i).to(torch.int32), bits), scales.clone()


# ---------------------------------------------------------------------------
# dynamic activations and the int8 x int8 linear
# (mxtorch.py:2665-2731, 3910-3960, 8870-8968, 6693-6752)
# ---------------------------------------------------------------------------
def dynamic_quantize(x: Tensor, name: str, granularity: str = "per_token", block: int = 64):
    """dynamic_quantize (mxtorch.py:2665-2731) -> (packed, scales, orig_shape,
    n, block) of the mx_tensor it returns; the trailing ``.reshape(*shape)``
    of the per_token / per_channel branches only relabels the shape
    (mx_tensor.reshape, mxtorch.py:6319-6326)."""
    _, bits, _, _ = parse_dtype(name)
    max_int = float((1 << (bits - 1)) - 1)
    x_f = x.float()
    shape = tuple(x_f.shape)
    if granularity == "per_token":            # mxtorch.py:2708-2714
        x2 = x_f.reshape(-1, shape[-1])
        scales = x2.abs().amax(dim=1).clamp(min=1e-12) / max_int
        codes = (x2 / scales.unsqueeze(1)).round().clamp(-max_int, max_int).to(torch.int32)
        return pack_auto(codes.reshape(-1), bits), scales, shape, x2.numel(), x2.shape[-1]
    if granularity == "per_channel":          # mxtorch.py:2716-2722
        x2 = x_f.reshape(shape[0], -1)
        scales = x2.abs().amax(dim=0).clamp(min=1e-12) / max_int
        codes = (x2 / scales.unsqueeze(0)).round().clamp(-max_int, max_int).to(torch.int32)
        return pack_auto(codes.reshape(-1), bits), scales, shape, x2.numel(), x2.shape[0]
    if granularity == "per_tensor":           # mxtorch.py:2724-2729
        scale = x_f.abs().max().clamp(min=1e-12) / max_int
        codes = (x_f / scale).round().clamp(-max_int, max_int).to(torch.int32)
        return pack_auto(codes.reshape(-1), bits), scale.unsqueeze(0), shape, x_f.numel(), x_f.numel()
    p, s, n = quantize(x_f, name, block)      # mxtorch.py:2731
    return p, s, shape, n, block


def fused_int8_linear(x_packed: Tensor, x_scales: Tensor, x_name: str, x_shape, x_n: int, x_block: int,
                      w_packed: Tensor, w_scales: Tensor, w_name: str, w_shape, w_n: int, w_block: int,
                      bias: Optional[Tensor] = None) -> Tensor:
    """fused_int8_linear's CPU branch (mxtorch.py:3957-3960):
    F.linear(x.dequantize(), weight.dequantize(), bias)."""
    x_f = dequant(x_packed, x_scales, x_name, x_n, x_block).reshape(x_shape)
    w_f = dequant(w_packed, w_scales, w_name, w_n, w_block).reshape(w_shape)
    return F.linear(x_f, w_f, bias)


def dynamic_linear_from_weight(weight: Tensor, name: str, block: int = 128):
    """mx_dynamic_linear.from_linear weight storage (mxtorch.py:8916-8917):
    quantize(weight) in nn.Linear's [out, in] layout, not transposed."""
    return quantize(weight, name, block)


def dynamic_linear_forward(x: Tensor, w_packed: Tensor, w_scales: Tensor, name: str, in_features: int,
                           out_features: int, block: int = 128, bias: Optional[Tensor] = None) -> Tensor:
    """mx_dynamic_linear.forward (mxtorch.py:8945-8962).  The per-token
    quantization it computes first (mxtorch.py:8947) does not reach the
    output: the product takes the unquantized tokens (mxtorch.py:8955-8957)."""
    x_f = x.float()
    tokens = x_f.reshape(-1, in_features)
    w_dq = dequant(w_packed, w_scales, name, in_features * out_features, block).reshape(out_features, in_features)
    out = tokens.float() @ w_dq.t()
    out = out.reshape(*x_f.shape[:-1], out_features)
    if bias is not None:
        out = out + bias
    return out


def mx_linear_autograd_forward(x: Tensor, w_packed: Tensor, w_scales: Tensor, w_name: str, x_name: str,
                               in_features: int, out_features: int, block: int,
                               b_packed: Optional[Tensor] = None, b_scales: Optional[Tensor] = None) -> Tensor:
    """_MXLinearAutograd.forward (mxtorch.py:6696-6726) for an [in, out]
    weight: quantize the 2-D input with x_name, _mx_mm -> _dispatch_qgemm
    (packed output of the matmul dtype), dequantize, add the dequantized bias."""
    orig_shape = x.shape
    x2 = x.reshape(-1, in_features) if x.dim() > 2 else x
    xp, xs, xn = quantize(x2, x_name, block)
    pc, sc, out_name = dispatch_qgemm(xp, xs, x_name, tuple(x2.shape), xn, w_packed, w_scales, w_name,
                                      (in_features, out_features), in_features * out_features, block)
    M = x2.shape[0]
    out = dequant(pc, sc, out_name, M * out_features, block).reshape(M, out_features)
    if len(orig_shape) > 2:
        out = out.reshape(*orig_shape[:-1], out_features)
    if b_packed is not None:
        b_f = dequant(b_packed, b_scales, w_name, out_features, block)
        if len(orig_shape) > 2:
            b_f = b_f.unsqueeze(0)
        out = out + b_f
    return out


def mx_linear_autograd_backward(grad: Tensor, w_packed: Tensor, w_scales: Tensor, w_name: str, in_features: int,
                                out_features: int, block: int, orig_shape) -> Tensor:
    """_MXLinearAutograd.backward (mxtorch.py:6729-6746): grad @ w_dq.t()."""
    w_dq = dequant(w_packed, w_scales, w_name, in_features * out_features, block).reshape(in_features, out_features)
    grad_2d = grad.reshape(-1, w_dq.shape[1]) if grad.dim() > 2 else grad
    gi = grad_2d @ w_dq.t()
    if len(orig_shape) > 2:
        gi = gi.reshape(*orig_shape[:-1], in_features)
    return gi


# ---------------------------------------------------------------------------
# model-level modules built around mx_linear (mxtorch.py:7612-7660,
# 7800-7877, 9161-9260)
# ---------------------------------------------------------------------------
def _dq_entry(e, name: str, block: int) -> Tensor:
    """Dequantize (packed, scales, shape) produced by quantize()."""
    packed, scales, shape = e
    n = int(math.prod(shape))
    return dequant(packed, scales, name, n, block, orig_shape=shape, hadamard_mode="rows").reshape(shape)


def layer_norm_from(weight: Tensor, bias: Optional[Tensor], name: str, block: int = 128):
    """mx_layer_norm.from_layer_norm (mxtorch.py:7640-7649): weight and bias
    quantized with the module's dtype.  Returns ((packed, scales, shape) or None) x 2."""
    w = quantize(weight, name, block)[:2] + (tuple(weight.shape),)
    b = quantize(bias, name, block)[:2] + (tuple(bias.shape),) if bias is not None else None
    return w, b


def layer_norm_forward(x: Tensor, w, b, normalized_shape, eps: float, name: str, block: int = 128):
    """mx_layer_norm.forward (mxtorch.py:7651-7657): F.layer_norm of x.float()
    with the dequantized weight and bias, requantized with the module's dtype.
    Returns (packed, scales, shape)."""
    w_f = _dq_entry(w, name, block) if w is not None else None
    b_f = _dq_entry(b, name, block) if b is not None else None
    out = F.layer_norm(x.float(), tuple(normalized_shape), w_f, b_f, eps)
    p, s, _ = quantize(out, name, block)
    return p, s, tuple(out.shape)


def mha_from(in_proj_weight: Tensor, out_proj_weight: Tensor, out_proj_bias: Optional[Tensor], name: str,
             block: int = 128):
    """mx_multihead_attention.from_mha (mxtorch.py:7808-7842) for the packed
    in_proj case: in_proj_weight quantized as stored ([3E, E]); out_proj an
    mx_linear (quantize(W.t()), and its bias quantized)."""
    inp = quantize(in_proj_weight, name, block)[:2] + (tuple(in_proj_weight.shape),)
    outw = quantize(out_proj_weight.t(), name, block)[:2] + (tuple(out_proj_weight.t().shape),)
    outb = (quantize(out_proj_bias, name, block)[:2] + (tuple(out_proj_bias.shape),)
            if out_proj_bias is not None else None)
    return inp, outw, outb


def mha_forward(query: Tensor, key: Tensor, value: Tensor, embed_dim: int, num_heads: int, in_proj, in_proj_bias,
                out_w, out_b, name: str, block: int = 128, need_weights: bool = True):
    """mx_multihead_attention.forward (mxtorch.py:7848-7873), eval mode, no
    masks: F.multi_head_attention_forward on float inputs with the
    dequantized in_proj weight.  The output projection weight is
    mx_linear.weight, the dequantized [in, out] storage, passed where
    F.multi_head_attention_forward expects [out, in]; its bias is the
    dequantized stored bias.  The output is requantized with the module's
    dtype.  Returns ((packed, scales, shape), attn_weights, float output).
    Inputs are passed as given: F.multi_head_attention_forward reads
    dimension 0 as the sequence even for batch_first modules."""
    w_in = _dq_entry(in_proj, name, block)
    w_out = _dq_entry(out_w, name, block)
    b_out = _dq_entry(out_b, name, block) if out_b is not None else None
    # the inputs go to F.multi_head_attention_forward as given, dimension 0
    # read as the sequence, whatever batch_first says (the reference does not
    # transpose)
    q, k, v = query.float(), key.float(), value.float()
    out, attn = F.multi_head_attention_forward(q, k, v, embed_dim, num_heads, w_in, in_proj_bias, None, None, False,
                                               0.0, w_out, b_out, training=False, need_weights=need_weights)
    p, s, _ = quantize(out, name, block)
    return (p, s, tuple(out.shape)), attn, out


def encoder_layer_forward(src: Tensor, params: dict, name: str, block: int = 128, nhead: int = 4,
                          eps: float = 1e-5, activation=F.relu) -> Tensor:
    """mx_transformer_encoder_layer.forward (mxtorch.py:9260-9278), eval mode,
    norm_first=False, from from_encoder_layer (mxtorch.py:9214-9234).
    `params` holds the nn.TransformerEncoderLayer's float parameters by name.
      x  = src.float() + dequant(self_attn(src))          (_sa_block)
      x  = dequant(norm1(x))
      x  = x + linear2(act(linear1(x)))                    (_ff_block; the
           mx_linear biases are re-quantized zeros, mxtorch.py:7434-7436)
      out = dequant(norm2(x))"""
    E = src.shape[-1]
    inp, outw, outb = mha_from(params["self_attn.in_proj_weight"], params["self_attn.out_proj.weight"],
                               params["self_attn.out_proj.bias"], name, block)
    (sp, ss, sshape), _, _ = mha_forward(src, src, src, E, nhead, inp, params["self_attn.in_proj_bias"], outw, outb,
                                         name, block)
    x = src.float() + _dq_entry((sp, ss, sshape), name, block)
    n1w, n1b = layer_norm_from(params["norm1.weight"], params["norm1.bias"], name, block)
    x = _dq_entry(layer_norm_forward(x, n1w, n1b, (E,), eps, name, block), name, block)
    ffs = []
    for lin in ("linear1", "linear2"):
        W = params[f"{lin}.weight"]
        wp, ws, _ = linear_from_weight(W, name, block)
        ffs.append((wp, ws, W.shape[1], W.shape[0]))
    wp, ws, K1, N1 = ffs[0]
    h = linear_forward(x, wp, ws, name, K1, N1, block, has_bias=True)
    wp, ws, K2, N2 = ffs[1]
    ff = linear_forward(activation(h), wp, ws, name, K2, N2, block, has_bias=True)
    x = x + ff
    n2w, n2b = layer_norm_from(params["norm2.weight"], params["norm2.bias"], name, block)
    return _dq_entry(layer_norm_forward(x, n2w, n2b, (E,), eps, name, block), name, block)


# ---------------------------------------------------------------------------
# vector-wise quantization  (mxtorch.py:2946-2994)
# ---------------------------------------------------------------------------
def vector_quantize(x: Tensor, name: str = "int8d", axis: int = 1) -> Tuple[Tensor, Tensor]:
    """vector_quantize (mxtorch.py:2946-2987): s = max(absmax, 1e-12) / max_int
    per row (axis=1) or column (axis=0), codes = round(x / s) clamped, int32."""
    _, bits, _, _ = parse_dtype(name)
    max_int = float((1 << (bits - 1)) - 1)
    x_f = x.float()
    if axis == 1:
        scales = x_f.abs().amax(dim=1).clamp(min=1e-12) / max_int
        codes = (x_f / scales.unsqueeze(1)).round().clamp(-max_int, max_int).to(torch.int32)
    elif axis == 0:
        scales = x_f.abs().amax(dim=0).clamp(min=1e-12) / max_int
        codes = (x_f / scales.unsqueeze(0)).round().clamp(-max_int, max_int).to(torch.int32)
    else:
        raise ValueError(axis)
    return codes, scales


def vector_dequantize(codes: Tensor, scales: Tensor, axis: int = 1) -> Tensor:
    """vector_dequantize (mxtorch.py:2989-2994)."""
    return codes.float() * (scales.unsqueeze(1) if axis == 1 else scales.unsqueeze(0))
