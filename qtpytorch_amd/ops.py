"""Functional entry points of the hot path, on GPU tensors, through libmxk.so.

Each function keeps the signature and return convention of the reference
function it replaces:

  quantize(x, dt, block) -> (packed, scales, n)         mxtorch.py:1684-1763
  _dequant(packed, scales, dt, n, block) -> float32[n]   mxtorch.py:1530-1597
  _qscale_gemm(...) -> (packed, scales[, C])             mxtorch.py:1299-1385, 5497-5573
  linear_wq(x, w_packed, w_scales, dt, K, N, block)      mxtorch.py:7454-7473
  linear_wq_nt(x, w_packed, w_scales, dt, N, K, block)   mxtorch.py:8949-8962, 6729-6740
  linear_i8(x codes, w codes, ...)                       mxtorch.py:3910-3960
  dynamic_quantize(x, dt, granularity)                   mxtorch.py:2665-2731

Inputs must live on a GPU; every computation is a HIP kernel (no CPU path).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib as L
from .dtypes import get_mx_dtype, matmul_output_dtype, mx_dtype

Tensor = torch.Tensor

# dequantize of Hadamard ('h') dtypes: "rows" inverts exactly the rotation
# quantize() applied (rows of the last dimension); "reference" reproduces the
# reference's whole-tensor unrotation (mxtorch.py:1582-1595), which is the
# inverse only for 1-D tensors.  Both agree on 1-D tensors.
HADAMARD_DEQUANT_MODE = "rows"

_SIGNS_CACHE = {}


def packed_nbytes(bits: int, n_codes: int) -> int:
    return int(L.lib().mxk_packed_nbytes(bits, n_codes))


def packed_storage(bits: int, n_codes: int, device) -> Tensor:
    """Empty packed buffer with the reference's dtype and length: int8 of
    ceil(n/(8/bits)) for bits in {1,2,4,8}, else int32 words (mxtorch.py:882-955)."""
    nbytes = packed_nbytes(bits, n_codes)
    if bits in (1, 2, 4, 8):
        return torch.empty(nbytes, dtype=torch.int8, device=device)
    return torch.empty(nbytes // 4, dtype=torch.int32, device=device)


_M64 = (1 << 64) - 1


def _rotl64(v: int, b: int) -> int:
    return ((v << b) | (v >> (64 - b))) & _M64


def _siphash24(data: bytes, k0: int = 0, k1: int = 0) -> int:
    """SipHash-2-4 (Aumasson and Bernstein, 2012) of `data` under the 128-bit
    key (k0, k1): 64-bit little-endian message words, 2 compression rounds
    per word, the length in the top byte of the last word, 4 finalization
    rounds."""
    v = [k0 ^ 0x736F6D6570736575, k1 ^ 0x646F72616E646F6D, k0 ^ 0x6C7967656E657261, k1 ^ 0x7465646279746573]

    def rounds(count: int) -> None:
        for _ in range(count):
            v[0] = (v[0] + v[1]) & _M64
            v[1] = _rotl64(v[1], 13) ^ v[0]
            v[0] = _rotl64(v[0], 32)
            v[2] = (v[2] + v[3]) & _M64
            v[3] = _rotl64(v[3], 16) ^ v[2]
            v[0] = (v[0] + v[3]) & _M64
            v[3] = _rotl64(v[3], 21) ^ v[0]
            v[2] = (v[2] + v[1]) & _M64
            v[1] = _rotl64(v[1], 17) ^ v[2]
            v[2] = _rotl64(v[2], 32)

    tail = len(data) % 8
    for off in range(0, len(data) - tail, 8):
        m = int.from_bytes(data[off:off + 8], "little")
        v[3] ^= m
        rounds(2)
        v[0] ^= m
    last = ((len(data) & 0xFF) << 56) | int.from_bytes(data[len(data) - tail:], "little")
    v[3] ^= last
    rounds(2)
    v[0] ^= last
    v[2] ^= 0xFF
    rounds(4)
    return v[0] ^ v[1] ^ v[2] ^ v[3]


def hadamard_seed(dt) -> int:
    """Default seed of the 'h' rotation of dtype `dt`, the same in every process.

    The reference seeds it with ``hash(dt.name) % 2**31`` (mxtorch.py:1723,
    1584), and Python salts str hashes per process, so the reference's signs
    change between runs.  This returns the value that expression has in a
    CPython 3.10 process started with PYTHONHASHSEED=0: there the salt is
    zero and the hash of an ASCII str is SipHash-2-4 of its bytes under the
    all-zero key, read as a signed 64-bit integer (-1 becomes -2)."""
    name = dt.name if isinstance(dt, mx_dtype) else str(dt)
    h = _siphash24(name.encode("latin-1"))
    if h >= 1 << 63:
        h -= 1 << 64
    if h == -1:
        h = -2
    return h % (2 ** 31)


# the reference's name for the seed rule, kept for callers of the older API
reference_hadamard_seed = hadamard_seed


def hadamard_signs(n: int, seed: int, device) -> Tensor:
    """Sign vector of hadamard_rotation(n, seed) (mxtorch.py:2856-2864): the
    CPU generator's randint(0, 2, (n,)) * 2 - 1, moved to the device.  This
    builds the rotation's parameters (n values); no tensor data touches it."""
    key = (n, seed, str(device))
    s = _SIGNS_CACHE.get(key)
    if s is None:
        gen = torch.Generator()
        gen.manual_seed(seed)
        s = (torch.randint(0, 2, (n,), generator=gen).float() * 2 - 1).to(device)
        _SIGNS_CACHE[key] = s
    return s


def _pow2(d: int) -> int:
    return 1 << math.ceil(math.log2(max(d, 1)))


def rotation_dim(shape) -> int:
    """Length quantize() rotates for 'h' dtypes (mxtorch.py:1721)."""
    shape = tuple(shape)
    if len(shape) >= 2:
        return int(shape[-1])
    return int(math.prod(shape)) if shape else 1


def _kind_variant(dt: mx_dtype):
    kind = L.MXK_KIND_FLOAT if dt.is_float else L.MXK_KIND_INT
    if dt.is_hadamard:
        var = L.MXK_VAR_HADAMARD
    elif dt.is_vector:
        var = L.MXK_VAR_VECTOR
    elif dt.variant == "":
        var = L.MXK_VAR_BASE
    else:
        raise L.MXKError(f"variant {dt.variant!r} of {dt.name} is outside this build's hot path "
                         f"(base, 'h' and 'v' variants are implemented)")
    return kind, var


def _workspace(nbytes: int, device) -> Optional[Tensor]:
    if nbytes <= 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


# split-K workspaces of the decode linears, one per (device, stream): the
# arrival counters in their first COUNTER_BYTES bytes start at zero and every
# call leaves them zero, so calls on one stream can share a buffer, and calls
# on different streams never do.
COUNTER_BYTES = 65536
_ZEROED_WS = {}
# buffers replaced by larger ones: a captured HIP graph keeps the address of
# the buffer it was captured with, so none is ever freed
_RETIRED_WS = []
# data pointers of workspaces whose counter prefix an eager (not captured)
# fill has cleared; every call leaves the counters zero after that
_WS_CLEARED = set()


def _zeroed_workspace(nbytes: int, device, stream: int) -> Optional[Tensor]:
    """The split-K workspace of `stream` on `device`, at least `nbytes` long.

    A new (or larger) buffer is allocated when needed.  The counter prefix
    must be zero when a call starts, and every call leaves it zero, so it
    needs clearing once, outside any capture.  A buffer made inside a graph
    capture holds whatever its memory held: until an eager call has cleared
    it, every capture that uses it records a fill kernel of the prefix
    (no memset node), so that each replay of each such graph starts from
    zeroed counters, and the first eager call clears it for good.  Calls that
    overlap on one stream cannot happen; graphs captured on the same stream
    share its buffer, so their replays must not overlap either."""
    if nbytes <= 0:
        return None
    key = (str(device), int(stream))
    ws = _ZEROED_WS.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is None or ws.numel() < nbytes:
        size = int(max(nbytes, 2 * ws.numel() if ws is not None else 0))
        new = torch.empty(size, dtype=torch.uint8, device=device)
        if ws is not None:
            _RETIRED_WS.append(ws)
        _ZEROED_WS[key] = ws = new
    if ws.data_ptr() not in _WS_CLEARED:
        ws[:min(ws.numel(), COUNTER_BYTES)].zero_()
        if not capturing:
            _WS_CLEARED.add(ws.data_ptr())
    return ws


def quantize(x: Tensor, dt, block: int = 128, *, seed: Optional[int] = None,
             signs: Optional[Tensor] = None, n_store: Optional[int] = None
             ) -> Tuple[Tensor, Tensor, int]:
    """quantize(x, dt, block) -> (packed, scales, n) on the GPU (mxtorch.py:1684-1763)."""
    dt = get_mx_dtype(dt)
    dev = L.require_gpu(x)
    kind, var = _kind_variant(dt)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    xc = x.contiguous()
    n = xc.numel()
    if n == 0:  # the reference returns empty codes and scales (nb = 0)
        return packed_storage(dt.bits, 0, dev), torch.empty(0, dtype=torch.float32, device=dev), 0
    nb = -(-n // block)
    if n_store is None:
        n_store = nb * block
    packed = packed_storage(dt.bits, n_store, dev)
    scales = torch.empty(nb, dtype=torch.float32, device=dev)
    rot_dim = 0
    sg = None
    if var == L.MXK_VAR_HADAMARD:
        rot_dim = rotation_dim(x.shape)
        if signs is None:
            signs = hadamard_signs(_pow2(rot_dim), hadamard_seed(dt) if seed is None else seed, dev)
        sg = signs.to(device=dev, dtype=torch.float32).contiguous()
    lib = L.lib()
    ws_bytes = lib.mxk_quantize_workspace(n, kind, dt.bits, var, block, rot_dim)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_quantize(xc.data_ptr(), L.elem_type(xc.dtype), n, kind, dt.bits, var, block,
                              L.ptr(sg), rot_dim, packed.data_ptr(), packed.numel() * packed.element_size(),
                              scales.data_ptr(), n_store, L.ptr(ws), ws_bytes, L.stream_of(xc))
    L.check(rc, f"quantize({dt.name}, block={block})")
    return packed, scales, n


def _dequant(packed: Tensor, scales: Tensor, dt, n: int, block: int, *, orig_shape=None,
             seed: Optional[int] = None, signs: Optional[Tensor] = None,
             hadamard_mode: Optional[str] = None) -> Tensor:
    """_dequant(packed, scales, dt, n, block) -> float32 [n] (mxtorch.py:1530-1597)."""
    dt = get_mx_dtype(dt)
    dev = L.require_gpu(packed, scales)
    kind, var = _kind_variant(dt)
    if dt.is_float and dt.bits not in (4, 8):
        raise L.MXKError(f"dequantize: {dt.name} grids are outside this build (float4/float8 only)")
    pk = packed.contiguous()
    sc = scales.contiguous().float()
    out = torch.empty(n, dtype=torch.float32, device=dev)
    if n == 0:
        return out
    rot_dim = 0
    sg = None
    if var == L.MXK_VAR_HADAMARD:
        mode = hadamard_mode or HADAMARD_DEQUANT_MODE
        rot_dim = n if (mode == "reference" or orig_shape is None) else rotation_dim(orig_shape)
        if signs is None:
            signs = hadamard_signs(_pow2(rot_dim), hadamard_seed(dt) if seed is None else seed, dev)
        sg = signs.to(device=dev, dtype=torch.float32).contiguous()
    lib = L.lib()
    ws_bytes = lib.mxk_dequantize_workspace(n, var, rot_dim)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_dequantize(pk.data_ptr(), pk.numel() * pk.element_size(), sc.data_ptr(), sc.numel(), n,
                                kind, dt.bits, var, block, L.ptr(sg), rot_dim, out.data_ptr(), L.ptr(ws),
                                ws_bytes, L.stream_of(pk))
    L.check(rc, f"dequantize({dt.name})")
    return out


def qscale_gemm(a_packed: Tensor, a_scales: Tensor, b_packed: Tensor, b_scales: Tensor,
                M: int, K: int, N: int, bits: int, block: int, out_bits: int, *,
                want_packed: bool = True, want_c: bool = False, want_acc: bool = False):
    """The packed GEMM of _dispatch_qgemm's CPU branch (mxtorch.py:5563-5573,
    _qscale_matmul mxtorch.py:1299-1385) on MFMA.

    Returns a dict with any of: "packed" (out_bits codes of the requantized C,
    M*N codes), "scales" ([ceil(M*N/block)]), "c" (float32 [M, N] before
    requantization), "acc" (int32 [ceil(K/block), M, N], per-K-block integer
    products)."""
    dev = L.require_gpu(a_packed, a_scales, b_packed, b_scales)
    out = {}
    cp = cs = cf = acc = None
    if M == 0 or N == 0 or K == 0:
        # empty operands: C is all zeros (an empty K sum) and has no blocks to requantize
        if want_packed:
            out["packed"] = packed_storage(out_bits, M * N, dev)
            out["packed"].zero_()
            # an all-zero block: s = fl32(1e-12) / q in float32, as the 'v' requantizer computes it
            out["scales"] = (torch.full((-(-(M * N) // block),), 1e-12, dtype=torch.float32, device=dev)
                             / float((1 << (out_bits - 1)) - 1))
        if want_c:
            out["c"] = torch.zeros(M, N, dtype=torch.float32, device=dev)
        if want_acc:
            out["acc"] = torch.zeros(0, M, N, dtype=torch.int32, device=dev)
        return out
    if want_packed:
        cp = packed_storage(out_bits, M * N, dev)
        cs = torch.empty(-(-(M * N) // block), dtype=torch.float32, device=dev)
        out["packed"], out["scales"] = cp, cs
    if want_c:
        cf = torch.empty(M, N, dtype=torch.float32, device=dev)
        out["c"] = cf
    if want_acc:
        acc = torch.empty(-(-K // block), M, N, dtype=torch.int32, device=dev)
        out["acc"] = acc
    ap, asc = a_packed.contiguous(), a_scales.contiguous().float()
    bp, bsc = b_packed.contiguous(), b_scales.contiguous().float()
    # an empty scale array is one of the wrong length (ones, as the reference
    # reads it); the C-ABI takes a non-null pointer with a count of 0
    n_asc, n_bsc = asc.numel(), bsc.numel()
    if n_asc == 0:
        asc = torch.ones(1, dtype=torch.float32, device=dev)
    if n_bsc == 0:
        bsc = torch.ones(1, dtype=torch.float32, device=dev)
    # the kernels that read the packed operands as stored load them in
    # 16-byte pieces (the workspace size assumes so): realign views that
    # start inside an allocation
    if ap.data_ptr() % 16:
        ap = ap.clone()
    if bp.data_ptr() % 16:
        bp = bp.clone()
    lib = L.lib()
    ws_bytes = lib.mxk_qgemm_workspace(M, K, N, bits, block, out_bits if want_packed else 0)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_qgemm(ap.data_ptr(), asc.data_ptr(), n_asc, bp.data_ptr(), bsc.data_ptr(), n_bsc,
                           M, K, N, bits, block, out_bits if want_packed else 0,
                           L.ptr(cp), 0 if cp is None else cp.numel() * cp.element_size(), L.ptr(cs), L.ptr(cf),
                           L.ptr(acc), L.ptr(ws), ws_bytes, L.stream_of(ap))
    L.check(rc, f"qgemm(bits={bits}, {M}x{K}x{N})")
    return out


def decode_prepack_eligible(dt, block: int, in_features: int, out_features: int) -> bool:
    """Whether the tiled decode and MFMA kernels take this weight as its
    tiled copy (4-bit base codes: int4 or FP4; block 128, whole 128-column
    blocks)."""
    dt = get_mx_dtype(dt)
    return (dt.bits == 4 and not dt.is_hadamard and not dt.is_vector and block == 128
            and out_features % 128 == 0 and in_features % 32 == 0)


def scales_prepack_eligible(dt, block: int, in_features: int, out_features: int) -> bool:
    """Whether linear_wq's kernels read block-major scales for this weight:
    the int4 decode kernels and the MFMA kernels (int1, int2, int4 and int8
    base codes, FP4 and FP8 grids; block 128, whole 128-column blocks)."""
    dt = get_mx_dtype(dt)
    return (dt.bits in ((4, 8) if dt.is_float else (1, 2, 4, 8)) and not dt.is_hadamard and not dt.is_vector
            and block == 128 and out_features % 128 == 0)


def prepack_scales(w_scales: Tensor, in_features: int, out_features: int, block: int = 128) -> Tensor:
    """Block-major copy [out/128, in] of a quantized [in, out] weight's
    scales (stored [in, out/128]), the layout the decode kernel reads."""
    dev = L.require_gpu(w_scales)
    K, N = in_features, out_features
    sc = w_scales.contiguous().float()
    if sc.numel() != K * (N // block):
        raise L.MXKError(f"prepack_scales: {sc.numel()} scales for a {K}x{N} weight with block {block}")
    out = torch.empty(N // block, K, dtype=torch.float32, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_linear_prepack_scales(sc.data_ptr(), K, N, block, out.data_ptr(), L.stream_of(sc))
    L.check(rc, f"prepack_scales({K}x{N})")
    return out


def prepack_weight(w_packed: Tensor, in_features: int, out_features: int, block: int = 128) -> Tensor:
    """Tiled copy (uint8, in*out/2 bytes) of a quantized 4-bit (int4 or FP4)
    [in, out] weight's packed codes, the layout linear_wq's tiled decode and
    MFMA kernels read (mxk_linear_prepack_weight; the copy only moves
    nibbles)."""
    dev = L.require_gpu(w_packed)
    K, N = in_features, out_features
    pk = w_packed.contiguous()
    if pk.numel() * pk.element_size() < K * N // 2:
        raise L.MXKError(f"prepack_weight: {pk.numel() * pk.element_size()} bytes for a {K}x{N} int4 weight")
    if pk.data_ptr() % 4:
        pk = pk.clone()
    out = torch.empty(K * N // 2, dtype=torch.uint8, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_linear_prepack_weight(pk.data_ptr(), K, N, 4, block, out.data_ptr(), L.stream_of(pk))
    L.check(rc, f"prepack_weight({K}x{N})")
    return out


def unpack_weight(w_tiled: Tensor, in_features: int, out_features: int, block: int = 128) -> Tensor:
    """The packed int4 [in, out] codes (uint8, in*out/2 bytes) rebuilt from
    their tiled copy (mxk_linear_unpack_weight), the inverse of
    prepack_weight."""
    dev = L.require_gpu(w_tiled)
    K, N = in_features, out_features
    if w_tiled.numel() * w_tiled.element_size() != K * N // 2:
        raise L.MXKError(f"unpack_weight: {w_tiled.numel()} bytes for a {K}x{N} int4 weight")
    out = torch.empty(K * N // 2, dtype=torch.uint8, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_linear_unpack_weight(w_tiled.data_ptr(), K, N, 4, block, out.data_ptr(),
                                               L.stream_of(w_tiled))
    L.check(rc, f"unpack_weight({K}x{N})")
    return out


def linear_wq(x: Tensor, w_packed: Optional[Tensor], w_scales: Tensor, dt, in_features: int, out_features: int,
              block: int = 128, bias: Optional[Tensor] = None, w_scales_t: Optional[Tensor] = None,
              w_tiled: Optional[Tensor] = None) -> Tensor:
    """y = x.float() @ dequant(W) (+ bias) for W stored as quantize(weight.t())
    ([in, out] row-major, mxtorch.py:7447), fused: the weight is never
    dequantized to memory (mx_linear.forward, mxtorch.py:7454-7473).
    `w_scales_t` is an optional prepack_scales() copy; without it the int4
    decode path transposes the scales into its workspace on every call.
    With `w_tiled` (prepack_weight()) and `w_scales_t` as well, the int4
    decode shapes run the tiled decode kernel and the other shapes the MFMA
    kernel on the same tiled copy (mxk_linear_wq_tiled); `w_packed` may then
    be None (a weight held as its tiled copy only), and shapes the tiled
    entry point does not take rebuild the packed codes for one call."""
    dt = get_mx_dtype(dt)
    if w_packed is None and w_tiled is None:
        raise L.MXKError("linear_wq: needs the packed weight or its tiled copy")
    dev = L.require_gpu(x, w_packed if w_packed is not None else w_tiled, w_scales)
    kind, var = _kind_variant(dt)
    if var != L.MXK_VAR_BASE:
        raise L.MXKError(f"linear_wq: {dt.name} weights need the base variant")
    lead = x.shape[:-1]
    K, N = in_features, out_features
    if x.shape[-1] != K:
        raise L.MXKError(f"linear_wq: x has {x.shape[-1]} features, weight expects {K}")
    xc = x.reshape(-1, K)
    if xc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        xc = xc.float()
    xc = xc.contiguous()
    M = xc.shape[0]
    if M == 0:
        return torch.empty(*lead, N, dtype=torch.float32, device=dev)
    if w_scales_t is not None:
        if (w_scales_t.device != dev or w_scales_t.dtype != torch.float32 or not w_scales_t.is_contiguous()
                or w_scales_t.numel() != K * (N // block)):
            raise L.MXKError("linear_wq: w_scales_t must be prepack_scales() of this weight (float32, contiguous, "
                             "same device)")
    if w_tiled is not None:
        if (w_tiled.device != dev or w_tiled.dtype != torch.uint8 or not w_tiled.is_contiguous()
                or w_tiled.numel() != K * N // 2):
            raise L.MXKError("linear_wq: w_tiled must be prepack_weight() of this weight (uint8, contiguous, "
                             "same device)")
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    if b is not None and b.data_ptr() % 16:
        b = b.clone()
    lib = L.lib()
    ws_bytes = lib.mxk_linear_workspace(M, K, N, dt.bits, block)
    stream = L.stream_of(xc)
    ws = _zeroed_workspace(ws_bytes, dev, stream)
    with L.on_device(dev):
        rc = L.MXK_EUNSUPPORTED
        if w_tiled is not None and w_scales_t is not None and decode_prepack_eligible(dt, block, K, N):
            rc = lib.mxk_linear_wq_tiled(xc.data_ptr(), L.elem_type(xc.dtype), M, K, w_tiled.data_ptr(),
                                         w_scales_t.data_ptr(), N, kind, L.ptr(b), out.data_ptr(), L.ptr(ws), ws_bytes,
                                         stream)
        if rc == L.MXK_EUNSUPPORTED:
            wp = w_packed.contiguous() if w_packed is not None else unpack_weight(w_tiled, K, N, block)
            rc = lib.mxk_linear_wq(xc.data_ptr(), L.elem_type(xc.dtype), M, K, wp.data_ptr(),
                                   w_scales.contiguous().data_ptr(), L.ptr(w_scales_t), N, kind, dt.bits, block,
                                   L.ptr(b), out.data_ptr(), L.ptr(ws), ws_bytes, stream)
    L.check(rc, f"linear_wq({dt.name}, M={M}, K={K}, N={N})")
    return out.reshape(*lead, N)


def float_grid(bits: int) -> Tuple[Tensor, Tensor]:
    """(grid, mids) as the library builds them (host copy, no GPU needed)."""
    g = torch.empty(1 << bits, dtype=torch.float32)
    m = torch.empty((1 << bits) - 1, dtype=torch.float32)
    L.check(L.lib().mxk_float_grid(bits, g.data_ptr(), m.data_ptr()), "float_grid")
    return g, m


_ELEM_OPS = {"add": 0, "sub": 1, "mul": 2, "neg": 3}


def qelementwise(op: str, a_packed: Tensor, a_scales: Tensor, b_packed: Optional[Tensor],
                 b_scales: Optional[Tensor], n: int, block: int, bits: int, out_bits: int):
    """Packed element-wise arithmetic: the CPU branches of _dispatch_qadd /
    _dispatch_qsub / _dispatch_qmul (mxtorch.py:5397-5401, 5425-5431,
    5489-5497; _qscale_add / _qscale_mul, mxtorch.py:1186-1296) and the code
    negation of mx_tensor.__neg__ (mxtorch.py:6177-6193) on the GPU.

    Both operands' first n codes are read with `bits` (a's width).  Returns
    (packed, scales): for add/sub/mul the nb*block result codes packed with
    out_bits and [nb] scales; for neg the negated codes with a's width (every
    stored byte for 8-bit codes) and a copy of a's scales."""
    code = _ELEM_OPS[op]
    ts = [a_packed, a_scales] + ([] if op == "neg" else [b_packed, b_scales])
    dev = L.require_gpu(*ts)
    nb = a_scales.numel()
    ap = a_packed.contiguous()
    if op == "neg":
        count = ap.numel() * ap.element_size() if bits == 8 else n
        out = packed_storage(bits, count, dev)
        scales = a_scales.clone()
        bp = bsc = None
    else:
        out = packed_storage(out_bits, nb * block, dev)
        scales = torch.empty(nb, dtype=torch.float32, device=dev)
        bp, bsc = b_packed.contiguous(), b_scales.contiguous().float()
    asc = a_scales.contiguous().float()
    lib = L.lib()
    ws_bytes = lib.mxk_qelementwise_workspace(code, n, nb, block, bits, out_bits)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_qelementwise(code, ap.data_ptr(), ap.numel() * ap.element_size(), asc.data_ptr(),
                                  L.ptr(bp), 0 if bp is None else bp.numel() * bp.element_size(), L.ptr(bsc),
                                  n, nb, block, bits, out_bits, out.data_ptr(), out.numel() * out.element_size(),
                                  scales.data_ptr() if op != "neg" else 0, L.ptr(ws), ws_bytes, L.stream_of(ap))
    L.check(rc, f"qelementwise({op}, bits={bits}, n={n}, block={block})")
    return out, scales


_GRANULARITY = {"per_token": 0, "per_channel": 1, "per_tensor": 2}


def dynamic_quantize(x: Tensor, dt, granularity: str = "per_token") -> Tuple[Tensor, Tensor, Tuple[int, int]]:
    """dynamic_quantize's per_token / per_channel / per_tensor branches
    (mxtorch.py:2706-2729) on the GPU.  Returns (packed, scales, (rows, cols))
    where [rows, cols] is the 2-D view the reference quantizes: x.reshape(-1,
    shape[-1]) per token, x.reshape(shape[0], -1) per channel, the flat
    tensor per tensor (rows = 1)."""
    dt = get_mx_dtype(dt)
    g = _GRANULARITY[granularity]
    dev = L.require_gpu(x)
    if dt.bits < 2:
        raise L.MXKError(f"dynamic_quantize: {dt.name} has max_int = 0 in the reference (scales of 1/0); "
                         f"widths of 2 bits and more are supported")
    xs = x if x.dtype in (torch.float32, torch.float16, torch.bfloat16) else x.float()
    xs = xs.contiguous()
    shape = tuple(xs.shape)
    n = xs.numel()
    if g == 0:
        cols = shape[-1] if len(shape) >= 1 else 1
    elif g == 1:
        cols = n // shape[0] if len(shape) >= 1 and shape[0] else 1
    else:
        cols = n
    rows = n // cols if cols else 0
    nscales = rows if g == 0 else (cols if g == 1 else 1)
    packed = packed_storage(dt.bits, n, dev)
    scales = torch.empty(nscales, dtype=torch.float32, device=dev)
    if n == 0:
        return packed, scales, (rows, cols)
    lib = L.lib()
    ws_bytes = lib.mxk_dynamic_quantize_workspace(rows, cols, g, dt.bits)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_dynamic_quantize(xs.data_ptr(), L.elem_type(xs.dtype), rows, cols, g, dt.bits, packed.data_ptr(),
                                      packed.numel() * packed.element_size(), scales.data_ptr(), L.ptr(ws), ws_bytes,
                                      L.stream_of(xs))
    L.check(rc, f"dynamic_quantize({dt.name}, {granularity}, {rows}x{cols})")
    return packed, scales, (rows, cols)


def decode_prepack_nt_eligible(dt, block: int, in_features: int, out_features: int) -> bool:
    """Whether an [out, in] weight can have the tiled copy of
    prepack_weight_nt (int4 base codes, block 128, in and out multiples of
    128)."""
    dt = get_mx_dtype(dt)
    return (not dt.is_float and dt.bits == 4 and not dt.is_hadamard and not dt.is_vector and block == 128
            and out_features % 128 == 0 and in_features % 128 == 0)


def prepack_weight_nt(w_packed: Tensor, out_features: int, in_features: int, block: int = 128) -> Tensor:
    """Tiled copy (uint8, out*in/2 bytes) of a quantized int4 [out, in]
    weight's packed codes (blocks of 128 along in), the layout linear_wq_nt's
    tiled decode kernel reads (mxk_linear_prepack_weight_nt)."""
    dev = L.require_gpu(w_packed)
    N, K = out_features, in_features
    pk = w_packed.contiguous()
    if pk.numel() * pk.element_size() < K * N // 2:
        raise L.MXKError(f"prepack_weight_nt: {pk.numel() * pk.element_size()} bytes for a {N}x{K} int4 weight")
    if pk.data_ptr() % 16:
        pk = pk.clone()
    out = torch.empty(K * N // 2, dtype=torch.uint8, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_linear_prepack_weight_nt(pk.data_ptr(), N, K, 4, block, out.data_ptr(), L.stream_of(pk))
    L.check(rc, f"prepack_weight_nt({N}x{K})")
    return out


def unpack_weight_nt(w_tiled: Tensor, out_features: int, in_features: int, block: int = 128) -> Tensor:
    """The packed int4 [out, in] codes (uint8, out*in/2 bytes) rebuilt from
    their tiled copy (mxk_linear_unpack_weight_nt), the inverse of
    prepack_weight_nt."""
    dev = L.require_gpu(w_tiled)
    N, K = out_features, in_features
    if w_tiled.numel() * w_tiled.element_size() != K * N // 2:
        raise L.MXKError(f"unpack_weight_nt: {w_tiled.numel()} bytes for a {N}x{K} int4 weight")
    out = torch.empty(K * N // 2, dtype=torch.uint8, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_linear_unpack_weight_nt(w_tiled.data_ptr(), N, K, 4, block, out.data_ptr(),
                                                  L.stream_of(w_tiled))
    L.check(rc, f"unpack_weight_nt({N}x{K})")
    return out


def linear_wq_nt(x: Tensor, w_packed: Optional[Tensor], w_scales: Tensor, dt, out_features: int,
                 in_features: int, block: int = 128, bias: Optional[Tensor] = None,
                 w_scales_t: Optional[Tensor] = None, w_tiled: Optional[Tensor] = None) -> Tensor:
    """y = x.float() @ dequant(W).t() (+ bias) for a weight stored [out, in]
    (mx_dynamic_linear.forward, mxtorch.py:8949-8962, and the input gradient
    of _MXLinearAutograd, mxtorch.py:6729-6740); the weight is decoded in
    registers, never dequantized to memory.  `w_scales_t` is an optional
    K-block-major copy [in/128, out] of the scales (prepack_scales(w_scales,
    out, in)), read by the int4 decode path.  With `w_tiled`
    (prepack_weight_nt()) and `w_scales_t` as well, the int4 decode shapes
    run the tiled decode kernel and the other shapes the MFMA kernel on the
    same tiled copy (mxk_linear_wq_nt_tiled); `w_packed` may then be None (a
    weight held as its tiled copy only), and shapes the tiled entry point does
    not take rebuild the packed codes for one call."""
    dt = get_mx_dtype(dt)
    if w_packed is None and w_tiled is None:
        raise L.MXKError("linear_wq_nt: needs the packed codes or their tiled copy")
    dev = L.require_gpu(x, w_packed if w_packed is not None else w_tiled, w_scales)
    kind, var = _kind_variant(dt)
    if var != L.MXK_VAR_BASE:
        raise L.MXKError(f"linear_wq_nt: {dt.name} weights need the base variant")
    N, K = out_features, in_features
    if x.shape[-1] != K:
        raise L.MXKError(f"linear_wq_nt: x has {x.shape[-1]} features, weight expects {K}")
    lead = x.shape[:-1]
    xc = x.reshape(-1, K)
    if xc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        xc = xc.float()
    xc = xc.contiguous()
    M = xc.shape[0]
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    if M == 0 or N == 0:
        return out.reshape(*lead, N)
    if K == 0:
        out.zero_()
        if bias is not None:
            out += bias.to(device=dev, dtype=torch.float32)
        return out.reshape(*lead, N)
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    ws = w_scales.contiguous().float()
    if w_scales_t is not None:
        if (w_scales_t.device != dev or w_scales_t.dtype != torch.float32 or not w_scales_t.is_contiguous()
                or w_scales_t.numel() != ws.numel()):
            raise L.MXKError("linear_wq_nt: w_scales_t must be prepack_scales() of this weight's scales")
    if w_tiled is not None:
        if (w_tiled.device != dev or w_tiled.dtype != torch.uint8 or not w_tiled.is_contiguous()
                or w_tiled.numel() != K * N // 2):
            raise L.MXKError("linear_wq_nt: w_tiled must be prepack_weight_nt() of this weight (uint8, "
                             "contiguous, same device)")
    lib = L.lib()
    ws_bytes = lib.mxk_linear_nt_workspace(M, K, N, dt.bits, block)
    stream = L.stream_of(xc)
    wk = _zeroed_workspace(ws_bytes, dev, stream)
    with L.on_device(dev):
        rc = L.MXK_EUNSUPPORTED
        if w_tiled is not None and w_scales_t is not None and decode_prepack_nt_eligible(dt, block, K, N):
            bt = b if b is None or b.data_ptr() % 16 == 0 else b.clone()
            rc = lib.mxk_linear_wq_nt_tiled(xc.data_ptr(), L.elem_type(xc.dtype), M, K, w_tiled.data_ptr(),
                                            w_scales_t.data_ptr(), N, L.ptr(bt), out.data_ptr(), L.ptr(wk), ws_bytes,
                                            stream)
        if rc == L.MXK_EUNSUPPORTED:
            wp = (w_packed if w_packed is not None else unpack_weight_nt(w_tiled, N, K, block)).contiguous()
            rc = lib.mxk_linear_wq_nt(xc.data_ptr(), L.elem_type(xc.dtype), M, K, wp.data_ptr(),
                                      wp.numel() * wp.element_size(), ws.data_ptr(), ws.numel(), L.ptr(w_scales_t),
                                      N, kind, dt.bits, block, L.ptr(b), out.data_ptr(), L.ptr(wk), ws_bytes, stream)
    L.check(rc, f"linear_wq_nt({dt.name}, M={M}, K={K}, N={N})")
    return out.reshape(*lead, N)


def linear_nt_eligible(dt) -> bool:
    """Weight dtypes linear_wq / linear_wq_nt decode in registers: base
    variant, int widths 1-8 and 16, float widths 4 and 8."""
    dt = get_mx_dtype(dt)
    if not dt.is_base:
        return False
    return dt.bits in (4, 8) if dt.is_float else dt.bits in (1, 2, 3, 4, 5, 6, 7, 8, 16)


def linear_i8_eligible(x_dt, w_dt, K: int, x_block: int, w_block: int) -> bool:
    """Whether mxk_linear_i8 covers these operands: int codes of 2, 4 or 8
    bits (base variant) and 64 dividing K and both block sizes."""
    def ok(d):
        return d.is_int and d.is_base and d.bits in (2, 4, 8)
    return ok(x_dt) and ok(w_dt) and K > 0 and K % 64 == 0 and x_block % 64 == 0 and w_block % 64 == 0


def linear_i8(x_packed: Tensor, x_scales: Tensor, x_dt, x_block: int, w_packed: Tensor, w_scales: Tensor, w_dt,
              w_block: int, M: int, K: int, N: int, bias: Optional[Tensor] = None) -> Tensor:
    """fused_int8_linear on packed int codes (mxtorch.py:3910-3960): out[M, N]
    = dequant(x)[M, K] @ dequant(W)[N, K].t() (+ bias), the integer products on
    int8 MFMA.  The caller checks linear_i8_eligible first."""
    x_dt, w_dt = get_mx_dtype(x_dt), get_mx_dtype(w_dt)
    dev = L.require_gpu(x_packed, x_scales, w_packed, w_scales)
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    if M == 0 or N == 0:
        return out
    xp, xs = x_packed.contiguous(), x_scales.contiguous().float()
    wp, wsc = w_packed.contiguous(), w_scales.contiguous().float()
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    lib = L.lib()
    ws_bytes = lib.mxk_linear_i8_workspace(M, K, N, x_dt.bits, w_dt.bits, x_block, w_block)
    ws = _workspace(ws_bytes, dev)
    with L.on_device(dev):
        rc = lib.mxk_linear_i8(xp.data_ptr(), xp.numel() * xp.element_size(), xs.data_ptr(), xs.numel(), x_block,
                               x_dt.bits, wp.data_ptr(), wp.numel() * wp.element_size(), wsc.data_ptr(), wsc.numel(),
                               w_block, w_dt.bits, M, K, N, L.ptr(b), out.data_ptr(), L.ptr(ws), ws_bytes,
                               L.stream_of(xp))
    L.check(rc, f"linear_i8({x_dt.name} x {w_dt.name}, {M}x{K}x{N})")
    return out


def vector_quantize(x: Tensor, dtype="int8d", axis: int = 1) -> Tuple[Tensor, Tensor]:
    """vector_quantize(x, dtype, axis) (mxtorch.py:2946-2987) on the GPU: one
    absmax scale per row (axis=1) or per column (axis=0) of a 2-D tensor.
    Returns (codes int32 [rows, cols], scales float32 [rows] or [cols]);
    reconstruct with vector_dequantize."""
    dt = get_mx_dtype(dtype)
    dev = L.require_gpu(x)
    if axis not in (0, 1):
        raise ValueError(f"vector_quantize: axis is 0 (per column) or 1 (per row), not {axis}")
    if x.dim() != 2 or x.numel() == 0:
        raise ValueError(f"vector_quantize: expects a non-empty 2-D tensor, got shape {tuple(x.shape)}")
    xs = x if x.dtype in (torch.float32, torch.float16, torch.bfloat16) else x.float()
    xs = xs.contiguous()
    rows, cols = xs.shape
    codes = torch.empty(rows, cols, dtype=torch.int32, device=dev)
    scales = torch.empty(rows if axis == 1 else cols, dtype=torch.float32, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_vector_quantize(xs.data_ptr(), L.elem_type(xs.dtype), rows, cols, axis, dt.bits,
                                         codes.data_ptr(), scales.data_ptr(), L.stream_of(xs))
    L.check(rc, f"vector_quantize({dt.name}, axis={axis}, {rows}x{cols})")
    return codes, scales


def vector_dequantize(codes: Tensor, scales: Tensor, axis: int = 1) -> Tensor:
    """vector_dequantize (mxtorch.py:2989-2994): codes * scale of the row
    (axis=1) or column (axis=0), float32."""
    dev = L.require_gpu(codes, scales)
    if axis not in (0, 1):
        raise ValueError(f"vector_dequantize: axis is 0 (per column) or 1 (per row), not {axis}")
    c = codes.to(torch.int32).contiguous()
    rows, cols = c.shape
    sc = scales.contiguous().float()
    if sc.numel() != (rows if axis == 1 else cols):
        raise ValueError(f"vector_dequantize: {sc.numel()} scales for {rows}x{cols} codes along axis {axis}")
    out = torch.empty(rows, cols, dtype=torch.float32, device=dev)
    with L.on_device(dev):
        rc = L.lib().mxk_vector_dequantize(c.data_ptr(), sc.data_ptr(), rows, cols, axis, out.data_ptr(),
                                           L.stream_of(c))
    L.check(rc, "vector_dequantize")
    return out
