"""ctypes binding of libmxk.so (declared in include/mxk.h).

The library is built in-tree by qtpytorch_amd/csrc/build.py.  Loading
fails loudly when it is missing: the package has no CPU compute path.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmxk.so")

MXK_OK = 0
MXK_EINVAL, MXK_EUNSUPPORTED, MXK_ELAUNCH = -22, -95, -5
MXK_IN_F32, MXK_IN_F16, MXK_IN_BF16 = 0, 1, 2
MXK_KIND_INT, MXK_KIND_FLOAT = 0, 1
MXK_VAR_BASE, MXK_VAR_HADAMARD, MXK_VAR_VECTOR = 0, 1, 2
MXK_DYN_PER_TOKEN, MXK_DYN_PER_CHANNEL, MXK_DYN_PER_TENSOR = 0, 1, 2
ABI_VERSION = 10

_lock = threading.Lock()
_lib = None

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_vp = ctypes.c_void_p
c_sz = ctypes.c_size_t

# symbol -> (restype, argtypes)
SIGNATURES = {
    "mxk_abi_version": (c_int, []),
    "mxk_last_error": (ctypes.c_char_p, []),
    "mxk_packed_nbytes": (c_i64, [c_int, c_i64]),
    "mxk_float_grid": (c_int, [c_int, c_vp, c_vp]),
    "mxk_quantize_workspace": (c_sz, [c_i64, c_int, c_int, c_int, c_int, c_i64]),
    "mxk_quantize": (c_int, [c_vp, c_int, c_i64, c_int, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_i64,
                             c_vp, c_i64, c_vp, c_sz, c_vp]),
    "mxk_dequantize": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_int, c_int, c_int, c_int, c_vp, c_i64,
                               c_vp, c_vp, c_sz, c_vp]),
    "mxk_dequantize_workspace": (c_sz, [c_i64, c_int, c_i64]),
    "mxk_qgemm_workspace": (c_sz, [c_i64, c_i64, c_i64, c_int, c_int, c_int]),
    "mxk_qgemm_workspace_any": (c_sz, [c_i64, c_i64, c_i64, c_int, c_int, c_int]),
    "mxk_qgemm": (c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_int, c_int, c_int,
                          c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "mxk_linear_workspace": (c_sz, [c_i64, c_i64, c_i64, c_int, c_int]),
    "mxk_linear_wq": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_int, c_vp,
                              c_vp, c_vp, c_sz, c_vp]),
    "mxk_linear_prepack_scales": (c_int, [c_vp, c_i64, c_i64, c_int, c_vp, c_vp]),
    "mxk_linear_wq_noalloc": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_int, c_vp,
                                      c_vp, c_vp]),
    "mxk_linear_prepack_weight": (c_int, [c_vp, c_i64, c_i64, c_int, c_int, c_vp, c_vp]),
    "mxk_linear_unpack_weight": (c_int, [c_vp, c_i64, c_i64, c_int, c_int, c_vp, c_vp]),
    "mxk_linear_wq_tiled": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_sz,
                                    c_vp]),
    "mxk_kv_append": (c_int, [c_vp, c_vp, c_int, c_i64, c_int, c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp,
                              c_vp, c_vp]),
    "mxk_kv_gather": (c_int, [c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_vp,
                              c_vp]),
    "mxk_qelementwise_workspace": (c_sz, [c_int, c_i64, c_i64, c_int, c_int, c_int]),
    "mxk_qelementwise": (c_int, [c_int, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_int, c_int, c_int,
                                 c_vp, c_i64, c_vp, c_vp, c_sz, c_vp]),
    "mxk_linear_wq_nt": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int,
                                 c_int, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "mxk_linear_nt_workspace": (c_sz, [c_i64, c_i64, c_i64, c_int, c_int]),
    "mxk_linear_prepack_weight_nt": (c_int, [c_vp, c_i64, c_i64, c_int, c_int, c_vp, c_vp]),
    "mxk_linear_unpack_weight_nt": (c_int, [c_vp, c_i64, c_i64, c_int, c_int, c_vp, c_vp]),
    "mxk_linear_wq_nt_tiled": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "mxk_linear_i8_workspace": (c_sz, [c_i64, c_i64, c_i64, c_int, c_int, c_i64, c_i64]),
    "mxk_linear_i8": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_int, c_vp, c_i64, c_vp, c_i64, c_i64, c_int,
                              c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "mxk_dynamic_quantize_workspace": (c_sz, [c_i64, c_i64, c_int, c_int]),
    "mxk_dynamic_quantize": (c_int, [c_vp, c_int, c_i64, c_i64, c_int, c_int, c_vp, c_i64, c_vp, c_vp, c_sz, c_vp]),
    "mxk_vector_quantize": (c_int, [c_vp, c_int, c_i64, c_i64, c_int, c_int, c_vp, c_vp, c_vp]),
    "mxk_vector_dequantize": (c_int, [c_vp, c_vp, c_i64, c_i64, c_int, c_vp, c_vp]),
}


class MXKError(RuntimeError):
    pass


def lib():
    """Load libmxk.so once; raise MXKError if it is absent or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise MXKError(
                f"{LIB_PATH} is missing: build it with `python qtpytorch_amd/csrc/build.py` "
                f"(qtpytorch_amd has no CPU fallback)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name, None)
            if fn is None:
                raise MXKError(f"{LIB_PATH} does not export {name}")
            fn.restype = res
            fn.argtypes = args
        if h.mxk_abi_version() != ABI_VERSION:
            raise MXKError("libmxk.so ABI version mismatch")
        _lib = h
        return h


def check(rc: int, what: str) -> None:
    if rc != MXK_OK:
        msg = lib().mxk_last_error()
        raise MXKError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", None)
_SAME_DEVICE = contextlib.nullcontext()


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device (the raw handle
    query when torch has it: it builds no Stream object)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def on_device(dev: torch.device):
    """Context that makes `dev` the current device for the library's calls:
    nothing to do when it already is."""
    if _GET_DEVICE is not None and (dev.index is None or dev.index == _GET_DEVICE()):
        return _SAME_DEVICE
    return torch.cuda.device(dev)


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise MXKError(
                "qtpytorch_amd computes on the GPU only: move tensors/models to a cuda "
                "device before quantizing, dequantizing or multiplying")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise MXKError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def elem_type(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return MXK_IN_F32
    if dtype == torch.float16:
        return MXK_IN_F16
    if dtype == torch.bfloat16:
        return MXK_IN_BF16
    raise MXKError(f"unsupported input dtype {dtype} (float32, float16, bfloat16)")
