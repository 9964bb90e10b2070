"""mx_tensor: the packed quantized tensor, with the reference's API and layout.

Mirrors mxtorch.mx_tensor (mxtorch.py:6028-6425): a torch.Tensor subclass
over a 0-d placeholder that carries

    _mx_packed      int8 bytes (bits 1/2/4/8) or int32 words (other widths)
    _mx_scales      float32 [ceil(n / block)]
    _mx_dtype       mx_dtype
    _mx_orig_shape  torch.Size of the logical tensor
    _mx_n           number of logical elements
    _mx_block       block size

``quantize``/``dequantize``/``@`` run the HIP kernels of libmxk.so.
Attribute reads (.device, .requires_grad, .dtype, .is_cuda) are answered
from the packed storage instead of dequantizing the whole tensor per read
(the reference routes them through its dequantizing fallback,
mxtorch.py:7315-7337); the answers equal what that fallback returns.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch.utils._pytree import tree_map

from . import ops
from .dtypes import get_mx_dtype, matmul_output_dtype, mx_dtype, qmul_output_dtype, resolve_mixed

Tensor = torch.Tensor


def _as_mx_dtype(v) -> Optional[mx_dtype]:
    """The MX dtype v names (an mx_dtype or a registered name), else None."""
    if isinstance(v, mx_dtype):
        return v
    if isinstance(v, str) and _is_mx_name(v):
        return get_mx_dtype(v)
    return None


def _names_device(v) -> bool:
    if isinstance(v, (torch.device, int)) and not isinstance(v, bool):
        return True
    return isinstance(v, str) and (v in ("cpu", "cuda") or v.startswith(("cuda:", "cpu:")))


def _as_device(v) -> torch.device:
    """torch.device of a device spec; a bare index is a CUDA ordinal."""
    return torch.device("cuda", v) if isinstance(v, int) else torch.device(v)


class mx_tensor(torch.Tensor):
    """A quantized tensor that is a torch.Tensor (mxtorch.py:6028)."""

    def __new__(cls, packed: Tensor, scales: Tensor, mx_dtype: mx_dtype, orig_shape, n: int,
                block: int = 128, requires_grad: bool = False, seed: Optional[int] = None):
        dummy = torch.empty((), dtype=torch.float32, device=packed.device)
        inst = torch.Tensor._make_subclass(cls, dummy, requires_grad)
        inst._mx_packed = packed
        inst._mx_dtype = mx_dtype
        inst._mx_scales = scales
        inst._mx_orig_shape = torch.Size(orig_shape)
        inst._mx_n = int(n)
        inst._mx_block = int(block)
        # seed of the 'h' rotation the codes were made with (None otherwise);
        # it travels with the codes so that dequantize undoes that rotation
        # in any process
        inst._mx_seed = None
        if mx_dtype.is_hadamard:
            inst._mx_seed = int(seed) if seed is not None else ops.hadamard_seed(mx_dtype)
        return inst

    def __init__(self, packed, scales, mx_dtype, orig_shape, n, block=128, requires_grad=False, seed=None):
        pass

    # ---- code storage: the packed codes, or, for an int4 weight that
    # mx_linear ([in, out]) or mx_dynamic_linear ([out, in]) tiles, the tiled
    # copy its kernels read and nothing else (one copy of the weight); the
    # packed codes are then rebuilt on demand (ops.unpack_weight /
    # ops.unpack_weight_nt) for whatever else reads them.
    @property
    def _mx_packed(self) -> Tensor:
        d = self.__dict__
        t = d.get("_mx_tiled")
        if t is not None:
            K, N, dtype, layout = d["_mx_tiled_meta"]
            if layout == "nt":
                return ops.unpack_weight_nt(t, N, K, self._mx_block).view(dtype)
            return ops.unpack_weight(t, K, N, self._mx_block).view(dtype)
        return d["_mx_packed_store"]

    @_mx_packed.setter
    def _mx_packed(self, v: Tensor) -> None:
        self.__dict__["_mx_packed_store"] = v
        self.__dict__["_mx_tiled"] = None

    def _mx_storage(self) -> Tensor:
        """The tensor holding the codes (packed, or the tiled copy), without rebuilding anything."""
        t = self.__dict__.get("_mx_tiled")
        return t if t is not None else self.__dict__["_mx_packed_store"]

    def _mx_tile_(self, in_features: int, out_features: int, layout: str = "kn") -> Tensor:
        """Hold the codes of this 4-bit weight (int4, or FP4 for layout "kn")
        as their tiled copy only and return it; the packed bytes are freed.
        layout "kn": an [in, out] weight (mx_linear, ops.prepack_weight);
        "nt": an [out, in] int4 weight (mx_dynamic_linear,
        ops.prepack_weight_nt)."""
        d = self.__dict__
        t = d.get("_mx_tiled")
        if t is not None:
            if d["_mx_tiled_meta"][3] != layout:
                raise ValueError(f"mx_tensor: the codes are tiled as {d['_mx_tiled_meta'][3]!r}, not {layout!r}")
            return t
        pk = d["_mx_packed_store"]
        d["_mx_tiled_meta"] = (int(in_features), int(out_features), pk.dtype, layout)
        if layout == "nt":
            d["_mx_tiled"] = ops.prepack_weight_nt(pk, out_features, in_features, self._mx_block)
        else:
            d["_mx_tiled"] = ops.prepack_weight(pk, in_features, out_features, self._mx_block)
        d["_mx_packed_store"] = None
        return d["_mx_tiled"]

    def _mx_untile_(self) -> "mx_tensor":
        """Back to packed storage (before an in-place change of the codes)."""
        if self.__dict__.get("_mx_tiled") is not None:
            self._mx_packed = self._mx_packed
        return self

    # ---- tensor-subclass protocol (mxtorch.py:6058-6085) ----
    def __tensor_flatten__(self):
        meta = {"mx_dtype": self._mx_dtype, "orig_shape": self._mx_orig_shape,
                "n": self._mx_n, "block": self._mx_block}
        if self._mx_seed is not None:
            meta["seed"] = self._mx_seed
        return ["_mx_packed", "_mx_scales"], meta

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        return mx_tensor(inner_tensors["_mx_packed"], inner_tensors["_mx_scales"], metadata["mx_dtype"],
                         metadata["orig_shape"], metadata["n"], metadata["block"], seed=metadata.get("seed"))

    # ---- factory / inverse (mxtorch.py:6096-6115) ----
    @classmethod
    def quantize(cls, x: Tensor, dt, block: int = 128, requires_grad: Optional[bool] = None, *,
                 seed: Optional[int] = None) -> "mx_tensor":
        """`seed` (keyword, 'h' dtypes only) overrides the rotation's default
        seed, ops.hadamard_seed(dt)."""
        dt = get_mx_dtype(dt)
        if isinstance(x, mx_tensor):
            x = x.dequantize()
        if dt.is_hadamard and seed is None:
            seed = ops.hadamard_seed(dt)
        packed, scales, n = ops.quantize(x, dt, block, seed=seed)
        return cls(packed, scales, dt, x.shape, n, block, True, seed=seed)

    def dequantize(self) -> Tensor:
        flat = ops._dequant(self._mx_packed, self._mx_scales, self._mx_dtype, self._mx_n, self._mx_block,
                            orig_shape=self._mx_orig_shape, seed=self._mx_seed)
        return flat.reshape(self._mx_orig_shape)

    # ---- shape and metadata ----
    @property
    def shape(self) -> torch.Size:
        return self._mx_orig_shape

    def size(self, dim: Optional[int] = None):
        if dim is None:
            return self._mx_orig_shape
        return self._mx_orig_shape[dim]

    def dim(self) -> int:
        return len(self._mx_orig_shape)

    def numel(self) -> int:
        return self._mx_n

    @property
    def mx_dtype(self) -> mx_dtype:
        return self._mx_dtype

    @property
    def mx_scales(self) -> Tensor:
        return self._mx_scales

    @property
    def mx_block(self) -> int:
        return self._mx_block

    @property
    def packed(self) -> Tensor:
        return self._mx_packed

    @property
    def nbytes_packed(self) -> int:
        return self._mx_storage().nbytes + self._mx_scales.nbytes

    @property
    def compression_ratio(self) -> float:
        return (self._mx_n * 4) / max(self.nbytes_packed, 1)

    # ---- torch function routing ----
    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if getattr(func, "__name__", "") == "__get__" and args and isinstance(args[0], mx_tensor):
            attr = getattr(getattr(func, "__self__", None), "__name__", None)
            getter = _GETTERS.get(attr)
            if getter is not None:
                return getter(args[0])
        if func in _MM_FUNCS and len(args) >= 2 and isinstance(args[0], mx_tensor) and isinstance(args[1], mx_tensor):
            return _mx_mm(args[0], args[1])
        if func in _POINTWISE and len(args) >= 1 and not kwargs.get("out"):
            a = args[0]
            b = args[1] if len(args) > 1 else kwargs.get("other", 1)
            if isinstance(a, mx_tensor) or isinstance(b, mx_tensor):
                # the reference hands _binary_op a wrapper whose name is not
                # add/sub/mul, so two same-shape operands take its
                # dequantize -> op -> requantize branch (mxtorch.py:6807-6819)
                def _pw(x, y, _f=func):
                    with torch._C.DisableTorchFunctionSubclass():
                        return _f(_unwrap(x), _unwrap(y))
                return _binary_op(a, b, _pw)
        return _fallback(func, args, kwargs)

    # ---- arithmetic sugar ----
    def __matmul__(self, o):
        return _mx_mm(self, o)

    def __rmatmul__(self, o):
        return _mx_mm(o, self)

    def __add__(self, o):
        return _binary_op(self, o, torch.add)

    def __radd__(self, o):
        return _binary_op(o, self, torch.add)

    def __sub__(self, o):
        return _binary_op(self, o, torch.sub)

    def __rsub__(self, o):
        return _binary_op(o, self, torch.sub)

    def __mul__(self, o):
        return _binary_op(self, o, torch.mul)

    def __rmul__(self, o):
        return _binary_op(o, self, torch.mul)

    def __truediv__(self, o):
        return _binary_op(self, o, torch.div)

    def __neg__(self):
        """Code negation, scales unchanged (mxtorch.py:6177-6193)."""
        bits = self._mx_dtype.bits
        packed, scales = ops.qelementwise("neg", self._mx_packed, self._mx_scales, None, None, self._mx_n,
                                          self._mx_block, bits, bits)
        return mx_tensor(packed, scales, self._mx_dtype, self._mx_orig_shape, self._mx_n, self._mx_block,
                         seed=self._mx_seed)

    def __repr__(self):
        return (f"mx_tensor({self._mx_dtype.name}, shape={tuple(self._mx_orig_shape)}, "
                f"device={self._mx_storage().device}, {self.compression_ratio:.1f}x compression, "
                f"{self.nbytes_packed / 1024:.2f} KB packed)")

    def __len__(self):
        return self._mx_orig_shape[0]

    def float(self):
        return self.dequantize()

    def half(self):
        return self.dequantize().half()

    def bfloat16(self):
        return self.dequantize().bfloat16()

    # ---- moves, re-quantization and shape (mxtorch.py:6215-6331) ----
    # The accepted forms follow torch.Tensor.to: an MX dtype (name or
    # mx_dtype) re-quantizes, a device (torch.device, "cpu", "cuda[:i]" or a
    # bare index) moves the packed storage, dtype= with an MX dtype moves
    # (device=) then re-quantizes, anything else dequantizes and hands the
    # arguments to the float tensor's .to.
    def to(self, *args, **kwargs):
        first = args[0] if args else None
        device, dtype = kwargs.get("device"), kwargs.get("dtype")
        for want in (first, dtype):
            mx = _as_mx_dtype(want)
            if mx is not None:
                src = self if want is first or device is None else self._move_device(_as_device(device))
                return mx_tensor.quantize(src.dequantize(), mx, self._mx_block)
        if device is None and _names_device(first):
            device = first
        if device is not None:
            return self._move_device(_as_device(device))
        return self.dequantize().to(*args, **kwargs)

    def _derived(self, packed: Tensor, scales: Tensor, shape=None) -> "mx_tensor":
        """Same dtype, element count, block and rotation seed over other storage (or shape)."""
        return mx_tensor(packed, scales, self._mx_dtype, self._mx_orig_shape if shape is None else shape,
                         self._mx_n, self._mx_block, seed=self._mx_seed)

    def _move_device(self, device: torch.device) -> "mx_tensor":
        return self._derived(self._mx_packed.to(device), self._mx_scales.to(device))

    def cuda(self, device=None):
        """.cuda() / .cuda(i) / .cuda("cuda:i") / .cuda("i"); other strings mean device 0."""
        if device is None:
            return self._move_device(torch.device("cuda"))
        if isinstance(device, (int, torch.device)) or (isinstance(device, str) and ":" in device):
            return self._move_device(_as_device(device))
        text = str(device)
        return self._move_device(torch.device("cuda", int(text) if text.isdigit() else 0))

    def cpu(self):
        return self._move_device(torch.device("cpu"))

    def clone(self):
        return self._derived(self._mx_packed.clone(), self._mx_scales.clone())

    def detach(self):
        return self._derived(self._mx_packed.detach(), self._mx_scales.detach())

    def reshape(self, *shape):
        """A copy with another logical shape over the same flat blocks (one -1 is inferred)."""
        dims = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list, torch.Size)) else shape
        fixed = math.prod(d for d in dims if d != -1)
        dims = tuple(self._mx_n // fixed if d == -1 else d for d in dims)
        return self._derived(self._mx_packed.clone(), self._mx_scales.clone(), torch.Size(dims))

    def view(self, *shape):
        return self.reshape(*shape)

    def flatten(self, start=0, end=-1):
        return self.reshape(-1)

    def contiguous(self, *a, **k):
        return self.clone()

    def t(self):
        return mx_tensor.quantize(self.dequantize().t(), self._mx_dtype, self._mx_block)

    def __getitem__(self, idx):
        return mx_tensor.quantize(self.dequantize()[idx], self._mx_dtype, self._mx_block)

    # Module._apply (to / cuda / half) asks these of every floating buffer;
    # answering them directly avoids a dequantize per question
    def is_floating_point(self) -> bool:
        return True

    def is_complex(self) -> bool:
        return False

    def copy_(self, src, non_blocking: bool = False):
        """In-place copy of another mx_tensor's packed data (Module.load_state_dict
        copies saved buffers into the module's own this way)."""
        self._mx_untile_()
        if not isinstance(src, mx_tensor):
            src = mx_tensor.quantize(src.float().to(self._mx_packed.device), self._mx_dtype, self._mx_block)
        if (src._mx_dtype != self._mx_dtype or src._mx_n != self._mx_n or src._mx_block != self._mx_block
                or src._mx_packed.shape != self._mx_packed.shape):
            raise ValueError(f"copy_: {src!r} does not match the layout of {self!r}")
        self._mx_packed.copy_(src._mx_packed, non_blocking=non_blocking)
        self._mx_scales.copy_(src._mx_scales, non_blocking=non_blocking)
        self._mx_orig_shape = src._mx_orig_shape
        self._mx_seed = src._mx_seed
        return self

    def fused_int8_linear(self, weight, bias=None):
        """Tensor-method binding of fused_int8_linear (mxtorch.py:11980-11982)."""
        return fused_int8_linear(self, weight, bias)

    def __reduce_ex__(self, protocol):
        return (_rebuild_mxtensor, (self._mx_packed.cpu(), self._mx_scales.cpu(), self._mx_dtype.name,
                                    tuple(self._mx_orig_shape), self._mx_n, self._mx_block, self._mx_seed))


def _rebuild_mxtensor(packed, scales, dt, shape, n, block, seed=None):
    return mx_tensor(packed, scales, get_mx_dtype(dt), torch.Size(shape), n, block, seed=seed)


def _is_mx_name(s: str) -> bool:
    try:
        get_mx_dtype(s)
        return True
    except ValueError:
        return False


_GETTERS = {
    "device": lambda t: t._mx_storage().device,
    "is_cuda": lambda t: t._mx_storage().is_cuda,
    "requires_grad": lambda t: False,
    "dtype": lambda t: torch.float32,
    "ndim": lambda t: len(t._mx_orig_shape),
    "grad": lambda t: None,
    "is_leaf": lambda t: True,
    "grad_fn": lambda t: None,
    "layout": lambda t: torch.strided,
}

_MM_FUNCS = {torch.mm, torch.matmul, torch.Tensor.mm, torch.Tensor.matmul, torch.Tensor.__matmul__}


def _unwrap(x):
    return x.dequantize() if isinstance(x, mx_tensor) else x


def _pick_ref(*args):
    for a in args:
        if isinstance(a, mx_tensor):
            return a
        if isinstance(a, (list, tuple)):
            r = _pick_ref(*a)
            if r is not None:
                return r
    return None


_POINTWISE = {torch.add, torch.sub, torch.mul, torch.div, torch.pow}


def _dispatch_qelementwise(op: str, a: "mx_tensor", b: "mx_tensor") -> "mx_tensor":
    """_dispatch_qadd / _dispatch_qsub / _dispatch_qmul (mxtorch.py:5321-5497):
    codes of both operands read with a's width, output dtype _resolve_mixed
    (add, sub) or the widened {kind}{2*bits}d (mul)."""
    bits = a._mx_dtype.bits
    out_dt = qmul_output_dtype(a._mx_dtype) if op == "mul" else resolve_mixed(a._mx_dtype, b._mx_dtype)
    packed, scales = ops.qelementwise(op, a._mx_packed, a._mx_scales, b._mx_packed, b._mx_scales, a._mx_n,
                                      a._mx_block, bits, out_dt.bits)
    # codes of 'h' operands live in their rotated domain: the result keeps
    # the operands' Hadamard seed (callers route operands of different seeds
    # through dequantize / requantize instead)
    seed = None
    if out_dt.is_hadamard:
        seed = a._mx_seed if a._mx_seed is not None else b._mx_seed
    return mx_tensor(packed, scales, out_dt, a._mx_orig_shape, a._mx_n, a._mx_block, seed=seed)


def _binary_op(a, b, fn):
    """_binary_op (mxtorch.py:6450-6506).  Two mx_tensors of one shape and
    block: add / sub / mul stay in the code domain (the reference reads
    requires_grad of quantized tensors as False, so its STE branch is not
    taken); otherwise dequantize, apply fn, requantize (two mx_tensors: with
    _resolve_mixed of their dtypes; one: with its dtype)."""
    if isinstance(a, mx_tensor) and isinstance(b, mx_tensor):
        same_rotation = not (a._mx_dtype.is_hadamard and b._mx_dtype.is_hadamard and a._mx_seed != b._mx_seed)
        if a._mx_orig_shape == b._mx_orig_shape and a._mx_block == b._mx_block and same_rotation:
            name = getattr(fn, "__name__", "") or str(fn)
            if "add" in name or fn is torch.add:
                return _dispatch_qelementwise("add", a, b)
            if "sub" in name or fn is torch.sub:
                return _dispatch_qelementwise("sub", a, b)
            if "mul" in name or fn is torch.mul:
                return _dispatch_qelementwise("mul", a, b)
        out_dt = resolve_mixed(a._mx_dtype, b._mx_dtype)
        res = fn(_unwrap(a), _unwrap(b))
        return mx_tensor.quantize(res, out_dt, a._mx_block)
    ref = a if isinstance(a, mx_tensor) else b
    res = fn(_unwrap(a), _unwrap(b))
    if isinstance(res, Tensor) and not isinstance(res, mx_tensor):
        return mx_tensor.quantize(res, ref._mx_dtype, ref._mx_block)
    return res


def _fallback(func, args, kwargs):
    """Any other torch op: dequantize, run it, requantize floating results
    with the first mx_tensor's dtype (the reference's universal fallback,
    mxtorch.py:7315-7337)."""
    ref = _pick_ref(*args, *kwargs.values())
    a2 = tree_map(_unwrap, args)
    k2 = tree_map(_unwrap, kwargs)
    with torch._C.DisableTorchFunctionSubclass():
        out = func(*a2, **k2)
    if ref is not None and isinstance(out, Tensor) and not isinstance(out, mx_tensor):
        if out.ndim > 0 and out.dtype.is_floating_point:
            return mx_tensor.quantize(out, ref._mx_dtype, ref._mx_block)
    return out


# ---------------------------------------------------------------- GEMM
def _dispatch_qgemm(a: mx_tensor, b: mx_tensor) -> mx_tensor:
    """True quantized GEMM (mxtorch.py:5497-5573): packed codes in, packed
    codes out, with the CPU branch's semantics on the GPU."""
    assert len(a._mx_orig_shape) == 2 and len(b._mx_orig_shape) == 2
    M, K = a._mx_orig_shape
    K2, N = b._mx_orig_shape
    assert K == K2, f"GEMM shape mismatch: {a._mx_orig_shape} @ {b._mx_orig_shape}"
    bits = a._mx_dtype.bits
    block = a._mx_block
    out_dt = matmul_output_dtype(a._mx_dtype, b._mx_dtype)
    res = ops.qscale_gemm(a._mx_packed, a._mx_scales, b._mx_packed, b._mx_scales, M, K, N, bits, block,
                          out_dt.bits)
    return mx_tensor(res["packed"], res["scales"], out_dt, torch.Size([M, N]), M * N, block)


def _mx_mm(a, b):
    """Packed matmul routing (mxtorch.py:6508-6549).  The reference reads
    ``requires_grad`` of both operands through its dequantizing fallback,
    which is False for quantized tensors, so 2-D operands always reach
    _dispatch_qgemm; other ranks take dequantize -> matmul -> requantize."""
    if not isinstance(a, mx_tensor) or not isinstance(b, mx_tensor):
        raise TypeError("_mx_mm expects two mx_tensor operands")
    out_dt = matmul_output_dtype(a._mx_dtype, b._mx_dtype)
    if len(a._mx_orig_shape) == 2 and len(b._mx_orig_shape) == 2:
        return _dispatch_qgemm(a, b)
    res = torch.matmul(a.dequantize(), b.dequantize())
    return mx_tensor.quantize(res, out_dt, a._mx_block)


class _QGemmSTE(torch.autograd.Function):
    """Quantized GEMM with a straight-through gradient (mxtorch.py:5284-5311)."""

    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor, mx_dt, block: int) -> Tensor:
        ctx.save_for_backward(a, b)
        with torch.no_grad():
            qa = mx_tensor.quantize(a, mx_dt, block)
            qb = mx_tensor.quantize(b, mx_dt, block)
            result = _dispatch_qgemm(qa, qb).dequantize()
        return result.detach()

    @staticmethod
    def backward(ctx, grad: Tensor):
        a, b = ctx.saved_tensors
        return grad @ b.t(), a.t() @ grad, None, None


def mx_matmul(a: Tensor, b: Tensor, dtype="int4d", block: int = 128):
    """Public packed matmul (mxtorch.py:10694-10723)."""
    dt = get_mx_dtype(dtype)
    if not isinstance(a, mx_tensor):
        a = mx_tensor.quantize(a.float(), dt, block)
    if not isinstance(b, mx_tensor):
        b = mx_tensor.quantize(b.float(), dt, block)
    return _mx_mm(a, b)


def mx_quantize(x: Tensor, dtype="int4d", block: int = 128) -> mx_tensor:
    """Alias of mx_tensor.quantize (mxtorch.py:7391-7396)."""
    return mx_tensor.quantize(x, get_mx_dtype(dtype), block)


# ---------------------------------------------------------------- dynamic activations, int8 x int8 linear
def dynamic_quantize(x: Tensor, dtype="int8d", granularity: str = "per_token", block: int = 64) -> mx_tensor:
    """dynamic_quantize (mxtorch.py:2665-2731): scales computed from the
    input at run time with max_int = 2^(bits-1)-1 of the dtype's width.

    per_token    one scale per row of x.reshape(-1, shape[-1]), block = row length;
    per_channel  one scale per column of x.reshape(shape[0], -1), block =
                 shape[0] (as the reference stores it: the scales are per
                 column, the block records the row count);
    per_tensor   one scale, block = numel;
    otherwise    mx_tensor.quantize(x, dtype, block) (per_block).
    Codes are packed as ints of the dtype's width whatever its kind, as in
    the reference."""
    dt = get_mx_dtype(dtype) if isinstance(dtype, str) else dtype
    if isinstance(x, mx_tensor):
        x = x.dequantize()
    if granularity not in ("per_token", "per_channel", "per_tensor"):
        return mx_tensor.quantize(x.float(), dt, block)
    shape = x.shape
    packed, scales, (rows, cols) = ops.dynamic_quantize(x, dt, granularity)
    n = rows * cols
    # The reference builds the 2-D mx_tensor and reshapes it to x's shape,
    # which clones the codes it has just made; the fresh buffers are handed
    # over directly here (same shape, block and values, no copy).
    if granularity == "per_token":
        return mx_tensor(packed, scales, dt, torch.Size(shape), n, cols)
    if granularity == "per_channel":
        return mx_tensor(packed, scales, dt, torch.Size(shape), n, rows)
    return mx_tensor(packed, scales, dt, torch.Size(shape), n, n)


def fused_int8_linear(x, weight, bias: Optional[Tensor] = None, block: int = 128) -> Tensor:
    """fused_int8_linear (mxtorch.py:3910-3960): the reference's result is
    F.linear(x.dequantize(), weight.dequantize(), bias) (mxtorch.py:3957-3960)
    for x [..., K] and weight [N, K].

    Packed int operands (widths 2-8, 64 dividing K and both block sizes;
    per-token activations from dynamic_quantize qualify) run on int8 MFMA
    (ops.linear_i8).  Other packed weights are decoded in registers
    (ops.linear_wq_nt) after dequantizing x; plain float tensors take
    F.linear."""
    import torch.nn.functional as F

    if isinstance(x, mx_tensor) and isinstance(weight, mx_tensor):
        xs, ws = x._mx_orig_shape, weight._mx_orig_shape
        if len(ws) == 2 and len(xs) >= 1 and xs[-1] == ws[1]:
            N, K = int(ws[0]), int(ws[1])
            M = x._mx_n // K if K else 0
            if ops.linear_i8_eligible(x._mx_dtype, weight._mx_dtype, K, x._mx_block, weight._mx_block):
                out = ops.linear_i8(x._mx_packed, x._mx_scales, x._mx_dtype, x._mx_block, weight._mx_packed,
                                    weight._mx_scales, weight._mx_dtype, weight._mx_block, M, K, N, bias)
                return out.reshape(*xs[:-1], N)
    x_f = x.dequantize() if isinstance(x, mx_tensor) else x
    if isinstance(weight, mx_tensor):
        ws = weight._mx_orig_shape
        if len(ws) == 2 and ops.linear_nt_eligible(weight._mx_dtype):
            return ops.linear_wq_nt(x_f, weight._mx_packed, weight._mx_scales, weight._mx_dtype, int(ws[0]),
                                    int(ws[1]), weight._mx_block, bias=bias)
        weight = weight.dequantize()
    return F.linear(x_f, weight, bias)


class mx_fused_ops:
    """Namespace of the reference's fused ops that lie on this path
    (mxtorch.py:11395-11405)."""

    @staticmethod
    def fused_int8_linear(x, weight, bias: Optional[Tensor] = None, block: int = 128) -> Tensor:
        return fused_int8_linear(x, weight, bias, block)


class _MXLinearAutograd(torch.autograd.Function):
    """mx_linear's quantized-activation forward with a float input gradient
    (mxtorch.py:6693-6746).

    forward: quantize x (2-D view) with mx_dtype, packed GEMM with the
    [in, out] weight (_mx_mm -> _dispatch_qgemm, packed output), dequantize,
    add the dequantized bias.  backward: grad @ dequant(W).t(), with W decoded
    in registers (ops.linear_wq_nt); no gradient for the packed weight."""

    @staticmethod
    def forward(ctx, x: Tensor, w_mx: "mx_tensor", b_mx, mx_dtype, block, in_features, out_features) -> Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, in_features) if x.dim() > 2 else x
        with torch.no_grad():
            x_mx = mx_tensor.quantize(x_2d.detach(), mx_dtype, block)
            out = _mx_mm(x_mx, w_mx).dequantize().detach()
        if len(orig_shape) > 2:
            out = out.reshape(*orig_shape[:-1], out_features)
        if b_mx is not None:
            with torch.no_grad():
                b_f = b_mx.dequantize().detach()
            if len(orig_shape) > 2:
                b_f = b_f.unsqueeze(0)
            out = out + b_f
        ctx.w_mx = w_mx
        ctx.orig_shape = orig_shape
        ctx.in_features = in_features
        return out

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        w = ctx.w_mx
        ws = w._mx_orig_shape   # [in, out] for mx_linear's weight
        grad_2d = grad_output.reshape(-1, ws[1]) if grad_output.dim() > 2 else grad_output
        gi = ops.linear_wq_nt(grad_2d.contiguous(), w._mx_packed, w._mx_scales, w._mx_dtype, int(ws[0]), int(ws[1]),
                              w._mx_block)
        if len(ctx.orig_shape) > 2:
            gi = gi.reshape(*ctx.orig_shape[:-1], ctx.in_features)
        return gi, None, None, None, None, None, None


def _mx_linear_forward(x: Tensor, w_mx: "mx_tensor", b_mx, mx_dtype, block, in_features, out_features) -> Tensor:
    """mxtorch.py:6749-6752."""
    return _MXLinearAutograd.apply(x, w_mx, b_mx, mx_dtype, block, in_features, out_features)
