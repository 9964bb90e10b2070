"""kv_cache_quantizer with the reference's API (mxtorch.py:2998-3119), kept
in a preallocated ring on the GPU.

The reference appends one mx_tensor per step to Python lists and evicts the
oldest entry with ``list.pop(0)`` once ``max_seq_len`` steps are held
(mxtorch.py:3047-3067); ``get()`` dequantizes every step and stacks them
(mxtorch.py:3069-3086).  Here each step is one slot of a ring of device
buffers (codes, scales, V zero points): ``append_kv`` is one libmxk launch
that quantizes the step's K and V rows into the next slot, and ``get()`` is
one launch per tensor that dequantizes the live slots in time order.  The
arithmetic per step is the reference's: ``quantize(k_f, dt, D)`` over
[B*H, D] rows, V shifted by its row minimum when ``asymmetric_v`` (the
minimum kept as the zero point and added back by ``get()``).

Dtypes the fused kernels do not cover (Hadamard variants, the int32-word
widths 3, 5, 6, 7, 16, head_dim outside {64, 128, 256}) quantize with the
regular libmxk quantizer into the same ring and dequantize slot by slot, with
the reference's per-step ``mx_tensor.dequantize`` semantics.

The ring starts small and doubles up to ``max_seq_len`` slots.  Every step
of one cache must have the same number of rows (B*H).  ``get_quantized()``
returns mx_tensor views of the live slots: they alias the ring, so a slot
that is later evicted changes under a view still held.
"""
from __future__ import annotations

from typing import List, Optional, Tuple, Union

import torch

from . import _lib as L
from . import ops
from .dtypes import get_mx_dtype, mx_dtype
from .tensor import mx_tensor

Tensor = torch.Tensor

_FUSED_HEAD_DIMS = (64, 128, 256)


def _fused_ok(dt: mx_dtype, head_dim: int) -> bool:
    if head_dim not in _FUSED_HEAD_DIMS or dt.is_hadamard:
        return False
    if dt.variant not in ("", "v"):
        return False
    if dt.is_float:
        return dt.bits in (4, 8)
    if dt.is_vector and dt.bits == 1:
        return False
    return dt.bits in (1, 2, 4, 8)


class kv_cache_quantizer:
    _INITIAL_SLOTS = 64

    def __init__(self, n_heads: int, head_dim: int, dtype: Union[str, mx_dtype] = "int8d",
                 max_seq_len: int = 32768, asymmetric_v: bool = True):
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.dtype = get_mx_dtype(dtype)
        self.max_seq_len = max_seq_len
        self.asymmetric_v = asymmetric_v
        self._rows: Optional[int] = None
        self._cap = 0
        self._start = 0
        self._len = 0
        self._kc = self._ks = self._vc = self._vs = self._zp = None

    # ---- ring storage ----
    def _slot_bytes(self) -> int:
        return int(L.lib().mxk_packed_nbytes(self.dtype.bits, self._rows * self.head_dim))

    def _alloc(self, cap: int, device) -> tuple:
        sb, rows = self._slot_bytes(), self._rows
        kc = torch.empty(cap, sb, dtype=torch.uint8, device=device)
        vc = torch.empty(cap, sb, dtype=torch.uint8, device=device)
        ks = torch.empty(cap, rows, dtype=torch.float32, device=device)
        vs = torch.empty(cap, rows, dtype=torch.float32, device=device)
        zp = torch.empty(cap, rows, dtype=torch.float32, device=device) if self.asymmetric_v else None
        return kc, ks, vc, vs, zp

    def _order(self) -> Tensor:
        """Ring slots of the live steps, oldest first."""
        return (torch.arange(self._len) + self._start) % self._cap

    def _ensure_capacity(self, device) -> None:
        if self._cap == 0:
            self._cap = min(self.max_seq_len, self._INITIAL_SLOTS)
            self._kc, self._ks, self._vc, self._vs, self._zp = self._alloc(self._cap, device)
            self._start = 0
            return
        if self._len < self._cap or self._cap >= self.max_seq_len:
            return
        # full but below max_seq_len: double, copying the live slots in time order
        new_cap = min(self.max_seq_len, 2 * self._cap)
        bufs = self._alloc(new_cap, device)
        order = self._order().to(device)
        for dst, src in zip(bufs, (self._kc, self._ks, self._vc, self._vs, self._zp)):
            if src is not None:
                dst[: self._len].copy_(src.index_select(0, order))
        self._kc, self._ks, self._vc, self._vs, self._zp = bufs
        self._cap, self._start = new_cap, 0

    # ---- reference API ----
    def append_kv(self, k: Tensor, v: Tensor) -> None:
        """Quantize and store one step (mxtorch.py:3039-3067); k, v are
        [B, H, 1, D] or [B, 1, H, D] (any shape with B*H*D elements)."""
        dev = L.require_gpu(k, v)
        D = self.head_dim
        k2 = k.reshape(-1, D)
        v2 = v.reshape(-1, D)
        if k2.shape != v2.shape:
            raise ValueError(f"append_kv: k and v give {tuple(k2.shape)} and {tuple(v2.shape)} rows")
        rows = k2.shape[0]
        if self._rows is None:
            self._rows = rows
        elif rows != self._rows:
            raise ValueError(f"append_kv: this cache holds steps of {self._rows} rows (B*H); got {rows}")
        self._ensure_capacity(dev)
        if self._len == self._cap:  # full at max_seq_len: the oldest step leaves (FIFO)
            slot = self._start
            self._start = (self._start + 1) % self._cap
        else:
            slot = (self._start + self._len) % self._cap
            self._len += 1
        dt = self.dtype
        kind, var = ops._kind_variant(dt)
        if _fused_ok(dt, D) and k2.dtype in (torch.float32, torch.float16, torch.bfloat16) \
                and k2.dtype == v2.dtype:
            kx, vx = k2.contiguous(), v2.contiguous()
            zp = self._zp[slot] if self.asymmetric_v else None
            with L.on_device(dev):
                rc = L.lib().mxk_kv_append(kx.data_ptr(), vx.data_ptr(), L.elem_type(kx.dtype), rows, D, kind,
                                           dt.bits, var, int(self.asymmetric_v), self._kc[slot].data_ptr(),
                                           self._ks[slot].data_ptr(), self._vc[slot].data_ptr(),
                                           self._vs[slot].data_ptr(), L.ptr(zp), L.stream_of(kx))
            L.check(rc, f"kv_append({dt.name}, rows={rows}, head_dim={D})")
            return
        # other dtypes: the regular quantizer, written into the same slot
        k_f = k2.float()
        v_f = v2.float()
        pk, sk, _ = ops.quantize(k_f, dt, D)
        if self.asymmetric_v:
            v_min = v_f.min(dim=1, keepdim=True).values
            pv, sv, _ = ops.quantize(v_f - v_min, dt, D)
            self._zp[slot].copy_(v_min.squeeze(1))
        else:
            pv, sv, _ = ops.quantize(v_f, dt, D)
        self._kc[slot].copy_(pk.view(torch.uint8).reshape(-1))
        self._vc[slot].copy_(pv.view(torch.uint8).reshape(-1))
        self._ks[slot].copy_(sk)
        self._vs[slot].copy_(sv)

    def get(self) -> Tuple[Tensor, Tensor]:
        """The dequantized history (mxtorch.py:3069-3086): K and V as float32
        [B, H, T, D], oldest step first, V with its zero points added back."""
        if self._len == 0:
            raise RuntimeError("KV cache is empty")
        T, D, rows = self._len, self.head_dim, self._rows
        dev = self._kc.device
        dt = self.dtype
        if _fused_ok(dt, D):
            kind, var = ops._kind_variant(dt)
            outs = []
            for codes, scales, zp in ((self._kc, self._ks, None), (self._vc, self._vs, self._zp)):
                out = torch.empty(rows, T, D, dtype=torch.float32, device=dev)
                with L.on_device(dev):
                    rc = L.lib().mxk_kv_gather(codes.data_ptr(), scales.data_ptr(), L.ptr(zp), rows, D, kind,
                                               dt.bits, var, self._cap, self._start, T, out.data_ptr(),
                                               L.stream_of(out))
                L.check(rc, f"kv_gather({dt.name}, rows={rows}, steps={T})")
                outs.append(out)
            k_all, v_all = outs
        else:
            kq, vq = self.get_quantized()
            k_all = torch.stack([q.dequantize() for q in kq], dim=1)
            v_all = torch.stack([q.dequantize() for q in vq], dim=1)
            if self.asymmetric_v:
                v_all = v_all + self._zp.index_select(0, self._order().to(dev)).t().unsqueeze(-1)
        return k_all.reshape(-1, self.n_heads, T, D), v_all.reshape(-1, self.n_heads, T, D)

    def _views(self, codes: Tensor, scales: Tensor) -> List[mx_tensor]:
        dt, D, rows = self.dtype, self.head_dim, self._rows
        pdt = torch.int8 if dt.bits in (1, 2, 4, 8) else torch.int32
        out = []
        for s in self._order().tolist():
            out.append(mx_tensor(codes[s].view(pdt), scales[s], dt, torch.Size([rows, D]), rows * D, D))
        return out

    def get_quantized(self) -> Tuple[List[mx_tensor], List[mx_tensor]]:
        """Per-step quantized K and V slices, oldest first (mxtorch.py:3088-3090):
        mx_tensor views of the ring slots."""
        if self._len == 0:
            return [], []
        return self._views(self._kc, self._ks), self._views(self._vc, self._vs)

    def reset(self) -> None:
        """Forget every step and release the ring (mxtorch.py:3092-3096); the
        next request may have another batch size."""
        self._rows = None
        self._cap = self._start = self._len = 0
        self._kc = self._ks = self._vc = self._vs = self._zp = None

    @property
    def seq_len(self) -> int:
        return self._len

    def memory_bytes(self) -> int:
        """Bytes of the live steps' codes, scales and zero points, as the
        reference sums them per step (mxtorch.py:3102-3107)."""
        if self._len == 0:
            return 0
        per_step = 2 * (self._slot_bytes() + 4 * self._rows) + (4 * self._rows if self.asymmetric_v else 0)
        return self._len * per_step

    def compression_vs_fp16(self) -> float:
        T = self._len
        if T == 0:
            return 0.0
        return T * 2 * self.n_heads * self.head_dim * 2 / max(self.memory_bytes(), 1)

    def __repr__(self):
        return (f"kv_cache_quantizer(heads={self.n_heads}, dim={self.head_dim}, "
                f"dtype={self.dtype.name}, seq={self.seq_len}, "
                f"mem={self.memory_bytes() // 1024}KB)")
