"""kv_cache_quantizer with the reference's API (mxtorch.py:2998-3119).

Each appended step is quantized per row of ``head_dim`` (block = head_dim)
after flattening to [B*H, D]; V is shifted by its row minimum when
``asymmetric_v`` (the default) and the shift is kept as a zero point that
``get()`` adds back (mxtorch.py:3039-3086).  Quantize and dequantize run the
libmxk HIP kernels.
"""
from __future__ import annotations

from typing import List, Tuple, Union

import torch

from .dtypes import get_mx_dtype, mx_dtype
from .tensor import mx_tensor

Tensor = torch.Tensor


class kv_cache_quantizer:
    def __init__(self, n_heads: int, head_dim: int, dtype: Union[str, mx_dtype] = "int8d",
                 max_seq_len: int = 32768, asymmetric_v: bool = True):
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.dtype = get_mx_dtype(dtype)
        self.max_seq_len = max_seq_len
        self.asymmetric_v = asymmetric_v
        self._k_cache: List[mx_tensor] = []
        self._v_cache: List[mx_tensor] = []
        self._v_zp: List[Tensor] = []

    def append_kv(self, k: Tensor, v: Tensor) -> None:
        if len(self._k_cache) >= self.max_seq_len:
            self._k_cache.pop(0)
            self._v_cache.pop(0)
            if self._v_zp:
                self._v_zp.pop(0)
        k_f = k.float().reshape(-1, self.head_dim)
        v_f = v.float().reshape(-1, self.head_dim)
        self._k_cache.append(mx_tensor.quantize(k_f, self.dtype, self.head_dim))
        if self.asymmetric_v:
            v_min = v_f.min(dim=1, keepdim=True).values
            self._v_cache.append(mx_tensor.quantize(v_f - v_min, self.dtype, self.head_dim))
            self._v_zp.append(v_min.squeeze(1))
        else:
            self._v_cache.append(mx_tensor.quantize(v_f, self.dtype, self.head_dim))

    def get(self) -> Tuple[Tensor, Tensor]:
        if not self._k_cache:
            raise RuntimeError("KV cache is empty")
        T = len(self._k_cache)
        k_all = torch.stack([kq.dequantize() for kq in self._k_cache], dim=1)
        v_all = torch.stack([vq.dequantize() for vq in self._v_cache], dim=1)
        if self.asymmetric_v and self._v_zp:
            v_all = v_all + torch.stack(self._v_zp, dim=1).unsqueeze(-1)
        BH, _, D = k_all.shape
        return k_all.reshape(-1, self.n_heads, T, D), v_all.reshape(-1, self.n_heads, T, D)

    def get_quantized(self):
        return self._k_cache, self._v_cache

    def reset(self) -> None:
        self._k_cache.clear()
        self._v_cache.clear()
        self._v_zp.clear()

    @property
    def seq_len(self) -> int:
        return len(self._k_cache)

    def memory_bytes(self) -> int:
        return (sum(q.nbytes_packed for q in self._k_cache) + sum(q.nbytes_packed for q in self._v_cache)
                + sum(z.nbytes for z in self._v_zp))

    def compression_vs_fp16(self) -> float:
        T = len(self._k_cache)
        if T == 0:
            return 0.0
        return T * 2 * self.n_heads * self.head_dim * 2 / max(self.memory_bytes(), 1)

    def __repr__(self):
        return (f"kv_cache_quantizer(heads={self.n_heads}, dim={self.head_dim}, dtype={self.dtype.name}, "
                f"seq={self.seq_len}, mem={self.memory_bytes() // 1024}KB)")
