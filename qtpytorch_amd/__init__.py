"""qtpytorch_amd — MI355X (gfx950) kernels for mxtorch's quantize / pack /
block-scaled GEMM path, behind the reference's Python API.

    from qtpytorch_amd import mx_tensor, get_mx_dtype, mx_linear, to_mx
    q = mx_tensor.quantize(x.cuda(), get_mx_dtype("int4d"), 128)
    y = q.dequantize()
    c = qa @ qb                      # packed GEMM, packed result
    model = to_mx(model.cuda(), "int4d")

All computation runs in libmxk.so (HIP, built by qtpytorch_amd/csrc/build.py);
tensors must be on a GPU.
"""
from . import dtypes as _dtypes
from .dtypes import get_mx_dtype, matmul_output_dtype, mx_dtype
from .io import load_quantized, save_quantized
from .kv import kv_cache_quantizer
from .nn import (install_module_to, mx_dynamic_linear, mx_layer_norm, mx_linear, mx_multihead_attention,
                 mx_transformer_encoder_layer, to_mx, uninstall_module_to)
from .ops import HADAMARD_DEQUANT_MODE, _dequant, quantize, vector_dequantize, vector_quantize
from .tensor import (_dispatch_qgemm, _mx_linear_forward, _mx_mm, _MXLinearAutograd, _QGemmSTE,
                     dynamic_quantize, fused_int8_linear, mx_fused_ops, mx_matmul, mx_quantize, mx_tensor)

for _n in _dtypes._DTYPE_REGISTRY:
    globals()[_n] = _dtypes._DTYPE_REGISTRY[_n]

install_module_to()

__all__ = ["mx_dtype", "get_mx_dtype", "matmul_output_dtype", "mx_tensor", "quantize", "_dequant",
           "_dispatch_qgemm", "_mx_mm", "_QGemmSTE", "mx_matmul", "mx_quantize", "mx_linear", "to_mx",
           "kv_cache_quantizer", "install_module_to", "uninstall_module_to", "save_quantized", "load_quantized",
           "dynamic_quantize", "fused_int8_linear", "mx_fused_ops", "mx_dynamic_linear", "_MXLinearAutograd",
           "_mx_linear_forward", "mx_layer_norm", "mx_multihead_attention", "mx_transformer_encoder_layer",
           "vector_quantize", "vector_dequantize"]
