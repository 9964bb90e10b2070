"""mx_linear and to_mx: the model-level callers of the packed path.

mx_linear (mxtorch.py:7402-7496) keeps the reference's storage: the weight
is ``mx_tensor.quantize(linear.weight.t())``, i.e. [in, out] row-major with
blocks along ``out`` (mxtorch.py:7447).  Its forward computes
``x.float() @ dequant(W)`` in one fused HIP kernel (libmxk.so
mxk_linear_wq) that decodes the packed weight in registers.

Reference behaviours kept or changed, on purpose:
  * the reference re-quantizes its bias from zeros on every forward
    (mxtorch.py:7434-7436), so its output is ``x @ W_dq``; mx_linear does
    the same unless ``apply_bias=True`` (then the stored bias is added);
  * on a device mismatch the reference replaces the weight with a fresh
    random one (mxtorch.py:7429-7433); mx_linear moves the packed weight to
    the input's device instead.
"""
from __future__ import annotations

import gc
import re
import warnings
from typing import Dict, List, Optional, Union

import torch
import torch.nn as nn

from . import ops
from .dtypes import get_mx_dtype, mx_dtype
from .tensor import mx_tensor

Tensor = torch.Tensor


class mx_linear(nn.Module):
    """Drop-in replacement for nn.Linear with MX-packed weights."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, mx_dtype: mx_dtype = None,
                 block: int = 128, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.mx_dtype = get_mx_dtype(mx_dtype) if mx_dtype is not None else get_mx_dtype("int4d")
        self.block = block
        self.apply_bias = False
        # buffers, as in the reference (mxtorch.py:7420-7425, 7447-7451), so
        # that Module.to / cuda / state_dict / named_buffers see the packed data
        self.register_buffer("_mx_weight", None)
        self.register_buffer("_mx_bias", None)
        if device is not None:
            w = torch.randn(in_features, out_features, device=device) * 0.01
            self._mx_weight = mx_tensor.quantize(w, self.mx_dtype, block)
            if bias:
                self._mx_bias = mx_tensor.quantize(torch.zeros(out_features, device=device), self.mx_dtype, block)

    @classmethod
    def from_linear(cls, linear: nn.Linear, mx_dtype, block: int = 128) -> "mx_linear":
        m = cls.__new__(cls)
        nn.Module.__init__(m)
        m.in_features = linear.in_features
        m.out_features = linear.out_features
        m.mx_dtype = get_mx_dtype(mx_dtype)
        m.block = block
        m.apply_bias = False
        m.register_buffer("_mx_weight", mx_tensor.quantize(linear.weight.data.t(), m.mx_dtype, block))
        m.register_buffer("_mx_bias", mx_tensor.quantize(linear.bias.data, m.mx_dtype, block)
                          if linear.bias is not None else None)
        return m

    def forward(self, x: Tensor) -> Tensor:
        w = self._mx_weight
        if w is None:
            raise RuntimeError("mx_linear has no weight (build it with from_linear or device=...)")
        if not isinstance(w, mx_tensor):
            # a float [in, out] weight put in place of the packed one (e.g. by
            # Module.half(), which dequantizes floating buffers): quantize it again
            w = mx_tensor.quantize(w.float(), self.mx_dtype, self.block)
            self._mx_weight = w
        if w._mx_packed.device != x.device:
            w = w._move_device(x.device)
            self._mx_weight = w
            if self._mx_bias is not None:
                self._mx_bias = self._mx_bias._move_device(x.device)
        if isinstance(x, mx_tensor):
            x = x.dequantize()
        bias = None
        if self.apply_bias and self._mx_bias is not None:
            bias = self._mx_bias.dequantize()
        if torch.is_grad_enabled() and x.requires_grad:
            # the reference's F.linear(x, W_dq) carries the input gradient grad @ W_dq^T
            return _LinearWQ.apply(x, w, bias, self.in_features, self.out_features, self._decode_scales(w))
        return ops.linear_wq(x, w._mx_packed, w._mx_scales, w._mx_dtype, self.in_features, self.out_features,
                             w._mx_block, bias=bias, w_scales_t=self._decode_scales(w))

    def _decode_scales(self, w) -> Optional[Tensor]:
        """Block-major copy of the weight's scales for the int4 decode kernel,
        made once per weight tensor and rebuilt when the weight's scales are
        replaced or modified in place."""
        if not ops.decode_prepack_eligible(w._mx_dtype, w._mx_block, self.in_features, self.out_features):
            return None
        sc = w._mx_scales
        key = (sc.data_ptr(), str(sc.device), sc._version)
        cached = self.__dict__.get("_scales_t_cache")
        if cached is None or cached[0] != key:
            cached = (key, ops.prepack_scales(sc, self.in_features, self.out_features, w._mx_block))
            self.__dict__["_scales_t_cache"] = cached
        return cached[1]

    @property
    def weight(self):
        return self._mx_weight.dequantize() if self._mx_weight is not None else None

    @property
    def bias(self):
        return self._mx_bias.dequantize() if self._mx_bias is not None else None

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, dtype={self.mx_dtype.name}, "
                f"bias={self._mx_bias is not None}")


class _LinearWQ(torch.autograd.Function):
    """x @ dequant(W) with W stored [in, out] (mx_linear), and its input
    gradient grad @ dequant(W)^T (mxtorch.py:7473: F.linear(x, W_dq.t())
    differentiates to that); the packed weight gets no gradient."""

    @staticmethod
    def forward(ctx, x, w, bias, in_features, out_features, w_scales_t):
        ctx.w, ctx.w_scales_t = w, w_scales_t
        ctx.in_features, ctx.out_features = in_features, out_features
        return ops.linear_wq(x.detach(), w._mx_packed, w._mx_scales, w._mx_dtype, in_features, out_features,
                             w._mx_block, bias=bias, w_scales_t=w_scales_t)

    @staticmethod
    def backward(ctx, grad):
        w = ctx.w
        # the block-major scales [out/128, in] of the forward are the K-block-major
        # scales of the transposed product
        gi = ops.linear_wq_nt(grad.contiguous(), w._mx_packed, w._mx_scales, w._mx_dtype, ctx.in_features,
                              ctx.out_features, w._mx_block, w_scales_t=ctx.w_scales_t)
        return gi, None, None, None, None, None


class _LinearWQNT(torch.autograd.Function):
    """x @ dequant(W)^T with W stored [out, in] (mx_dynamic_linear), and its
    input gradient grad @ dequant(W), which is the [in, out]-layout product
    of ops.linear_wq with the roles of the two dimensions exchanged."""

    @staticmethod
    def forward(ctx, x, w, bias, in_features, out_features, w_scales_t):
        ctx.w, ctx.w_scales_t = w, w_scales_t
        ctx.in_features, ctx.out_features = in_features, out_features
        return ops.linear_wq_nt(x.detach(), w._mx_packed, w._mx_scales, w._mx_dtype, out_features, in_features,
                                w._mx_block, bias=bias, w_scales_t=w_scales_t)

    @staticmethod
    def backward(ctx, grad):
        w = ctx.w
        gi = ops.linear_wq(grad.contiguous(), w._mx_packed, w._mx_scales, w._mx_dtype, ctx.out_features,
                           ctx.in_features, w._mx_block, w_scales_t=ctx.w_scales_t)
        return gi, None, None, None, None, None


class mx_dynamic_linear(nn.Module):
    """Statically quantized weight with per-token activation quantization
    (mxtorch.py:8870-8968).

    The weight is ``mx_tensor.quantize(linear.weight)`` in nn.Linear's
    [out, in] layout (not transposed, mxtorch.py:8916-8917), the bias is kept
    in float.  The reference's forward quantizes the activations per token
    (mxtorch.py:8947) but multiplies the unquantized tokens by the
    dequantized weight (mxtorch.py:8955-8957), so its output is
    ``x.float() @ dequant(W).t() + bias``; that is what forward computes here,
    in one kernel that decodes the weight in registers (ops.linear_wq_nt),
    without the unused activation quantization.
    ``quantize_activation`` gives the per-token mx_tensor the reference builds."""

    def __init__(self, in_features: int, out_features: int, weight_dtype: mx_dtype = None, act_dtype: mx_dtype = None,
                 bias: bool = True, weight_block: int = 128):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight_dtype = get_mx_dtype(weight_dtype) if weight_dtype is not None else get_mx_dtype("int4d")
        self.act_dtype = get_mx_dtype(act_dtype) if act_dtype is not None else get_mx_dtype("int8d")
        self.weight_block = weight_block
        self.register_buffer("weight", None)
        self.register_buffer("bias", None)

    @classmethod
    def from_linear(cls, linear: nn.Linear, weight_dtype: Union[str, mx_dtype] = "int4d",
                    act_dtype: Union[str, mx_dtype] = "int8d", weight_block: int = 128) -> "mx_dynamic_linear":
        m = cls(linear.in_features, linear.out_features, get_mx_dtype(weight_dtype), get_mx_dtype(act_dtype),
                linear.bias is not None, weight_block)
        m.weight = mx_tensor.quantize(linear.weight.data, m.weight_dtype, weight_block)
        m.bias = linear.bias.data.clone() if linear.bias is not None else None
        return m

    def quantize_activation(self, x: Tensor) -> mx_tensor:
        """_dynamic_quantize_activation (mxtorch.py:8927-8943): per-token codes
        of the activation dtype's width, block = feature count."""
        from .tensor import dynamic_quantize
        return dynamic_quantize(x, self.act_dtype, "per_token")

    _dynamic_quantize_activation = quantize_activation

    def forward(self, x: Tensor) -> Tensor:
        x_f = x.dequantize() if isinstance(x, mx_tensor) else x
        w = self.weight
        if not isinstance(w, mx_tensor):
            w = mx_tensor.quantize(w, self.weight_dtype, self.weight_block)
        if w._mx_packed.device != x_f.device:
            w = w._move_device(x_f.device)
            self.weight = w
        b = self.bias
        if b is not None and b.device != x_f.device:
            b = b.to(x_f.device)
        if not ops.linear_nt_eligible(w._mx_dtype):
            out = x_f.float().reshape(-1, self.in_features) @ w.dequantize().t()
            out = out.reshape(*x_f.shape[:-1], self.out_features)
            return out + b if b is not None else out
        st = self._block_major_scales(w)
        if torch.is_grad_enabled() and x_f.requires_grad:
            return _LinearWQNT.apply(x_f, w, b, self.in_features, self.out_features, st)
        return ops.linear_wq_nt(x_f, w._mx_packed, w._mx_scales, w._mx_dtype, self.out_features, self.in_features,
                                w._mx_block, bias=b, w_scales_t=st)

    def _block_major_scales(self, w) -> Optional[Tensor]:
        """K-block-major copy [in/128, out] of the [out, in] weight's scales,
        read by both int4 decode kernels (this forward and its input
        gradient); made once per weight and rebuilt when the scales change."""
        if not ops.decode_prepack_eligible(w._mx_dtype, w._mx_block, self.out_features, self.in_features):
            return None
        sc = w._mx_scales
        key = (sc.data_ptr(), str(sc.device), sc._version)
        cached = self.__dict__.get("_scales_t_cache")
        if cached is None or cached[0] != key:
            cached = (key, ops.prepack_scales(sc, self.out_features, self.in_features, w._mx_block))
            self.__dict__["_scales_t_cache"] = cached
        return cached[1]

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, "
                f"w={self.weight_dtype.name}, act={self.act_dtype.name}")


def _replace_module(parent: nn.Module, name: str, module: nn.Module, dt: mx_dtype, block: int) -> bool:
    """The nn.Linear branch of _replace_module (mxtorch.py:7977-7989); other
    module kinds are outside this build's path and are left unchanged."""
    if isinstance(module, nn.Linear):
        setattr(parent, name, mx_linear.from_linear(module, dt, block))
        return True
    return False


def to_mx(model: nn.Module, dtype: Union[str, Dict[str, str], mx_dtype] = "int4d", block_size: int = 128,
          low_mem: bool = False, layer_batch_size: int = 4, skip_patterns: Optional[List[str]] = None) -> nn.Module:
    """Quantize a model's Linear layers in place (mxtorch.py:9744-9858):
    regex dtype maps over module names or class names, skip patterns,
    explicit float names skip a layer."""
    if isinstance(dtype, mx_dtype):
        dtype = dtype.name
    if isinstance(dtype, str):
        dtype_map = {".*": dtype}
    elif isinstance(dtype, dict):
        dtype_map = {p: (v.name if isinstance(v, mx_dtype) else v) for p, v in dtype.items()}
    else:
        raise TypeError(f"dtype must be str, dict or mx_dtype, got {type(dtype)}")
    skip = skip_patterns or []
    named = list(model.named_modules())
    processed = 0
    for full_name, module in named:
        if any(re.search(p, full_name) for p in skip):
            continue
        target = None
        for pat, dn in dtype_map.items():
            if re.search(pat, full_name) or re.search(pat, type(module).__name__):
                target = dn
                break
        if target is None or target in ("float32", "fp32", "float", "float64", "float16", "bfloat16"):
            continue
        try:
            dt = get_mx_dtype(target)
        except ValueError:
            warnings.warn(f"[qtpytorch_amd] Unknown dtype {target!r} for {full_name}, skipping.")
            continue
        parent, child = None, None
        for _, pmod in named:
            for cname, cmod in pmod.named_children():
                if cmod is module:
                    parent, child = pmod, cname
                    break
            if parent is not None:
                break
        if parent is not None and _replace_module(parent, child, module, dt, block_size):
            processed += 1
            if processed % layer_batch_size == 0:
                gc.collect()
                if low_mem and torch.cuda.is_available():
                    torch.cuda.empty_cache()
    return model


_orig_module_to = nn.Module.to


def _mx_module_to(self, *args, **kwargs):
    """nn.Module.to accepting MX dtype names (mxtorch.py:9462-9487)."""
    target = args[0] if args else kwargs.get("dtype", None)
    if isinstance(target, mx_dtype) or isinstance(target, dict) or (
            isinstance(target, str) and _is_mx(target)):
        block = kwargs.pop("block_size", 128)
        low_mem = kwargs.pop("low_mem", False)
        return to_mx(self, target, block_size=block, low_mem=low_mem)
    return _orig_module_to(self, *args, **kwargs)


def _is_mx(name: str) -> bool:
    try:
        get_mx_dtype(name)
        return True
    except ValueError:
        return False


def install_module_to() -> None:
    """Make ``model.to("int4d")`` call to_mx, as importing mxtorch does."""
    nn.Module.to = _mx_module_to


def uninstall_module_to() -> None:
    nn.Module.to = _orig_module_to
