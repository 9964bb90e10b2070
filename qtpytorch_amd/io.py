"""On-disk format of quantized models: save_quantized / load_quantized
(mxtorch.py:9860-10004).

The file is the reference's MX-native checkpoint, a torch.save'd dict:

    {"__mx_version__": 2,
     "<module path>.<attr>": {"dtype": name, "packed": CPU tensor, "scales": CPU tensor,
                               "shape": [..], "n": int, "block": int}, ...}

with the packed codes and scales byte for byte as in memory (mxtorch.py:
9886-9893).  Differences from the reference, on purpose:

  * entries of Hadamard ('h') tensors also hold "seed", the seed of the
    rotation their codes were made with, so that a checkpoint dequantizes
    with the same signs in any process (the reference re-derives the seed
    from the per-process salted hash(name), mxtorch.py:1584, 1723); an entry
    without it gets the default seed (ops.hadamard_seed);

  * mx_linear layers are saved under "<path>._mx_weight" / "<path>._mx_bias".
    The reference looks only for "weight"/"bias" attributes holding
    mx_tensors, so its save_quantized skips mx_linear's packed buffers
    (mxtorch.py:9867-9884); here they round-trip.
  * Loading uses torch.load(weights_only=True): the format holds only
    tensors, numbers, strings and lists, so nothing in the file is executed
    (the reference uses weights_only=False, mxtorch.py:9916).
  * A saved mx_linear comes back as an mx_linear in place of the model
    class's nn.Linear (same in/out features, the saved packed weight); other
    saved attributes are set as mx_tensors.  A plain state dict is loaded
    into the model and its nn.Linear layers matching the dtype patterns are
    converted with to_mx (the reference quantizes every matching parameter
    as is, mxtorch.py:9950-9999).
"""
from __future__ import annotations

import os
from typing import Dict, Optional, Union

import torch
import torch.nn as nn

from .dtypes import get_mx_dtype
from .nn import mx_linear, to_mx
from .tensor import mx_tensor

MX_VERSION = 2
_FLOAT_NAMES = ("float32", "fp32", "float", "float16", "bfloat16")


def _entry(t: mx_tensor) -> dict:
    e = {"dtype": t._mx_dtype.name, "packed": t._mx_packed.detach().cpu(),
         "scales": t._mx_scales.detach().cpu(), "shape": list(t._mx_orig_shape),
         "n": int(t._mx_n), "block": int(t._mx_block)}
    if t._mx_seed is not None:
        e["seed"] = int(t._mx_seed)
    return e


def _payload(p) -> Optional[mx_tensor]:
    if isinstance(p, mx_tensor):
        return p
    if isinstance(p, nn.Parameter) and isinstance(p.data, mx_tensor):
        return p.data
    return getattr(p, "_mx_payload", None) if p is not None else None


def save_quantized(model: nn.Module, path: str) -> str:
    """Write the packed codes and scales of every quantized tensor of `model`
    (mxtorch.py:9860-9898): mx_linear weights and biases, and "weight" /
    "bias" attributes of other modules that hold mx_tensors."""
    ckpt = {"__mx_version__": MX_VERSION}
    for full_name, module in model.named_modules():
        if isinstance(module, mx_linear):
            for attr in ("_mx_weight", "_mx_bias"):
                t = getattr(module, attr, None)
                if t is not None:
                    ckpt[f"{full_name}.{attr}"] = _entry(t)
            continue
        for attr in ("weight", "bias"):
            t = _payload(getattr(module, attr, None))
            if t is not None:
                ckpt[f"{full_name}.{attr}"] = _entry(t)
    torch.save(ckpt, path)
    return path


def _set_submodule(model: nn.Module, name: str, new: nn.Module) -> None:
    parent_name, _, leaf = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, leaf, new)


def load_quantized(checkpoint_path: str, model_class, dtype: Union[str, Dict[str, str]] = "int4d",
                   block_size: int = 128, model_kwargs: Optional[Dict] = None, device: str = "cpu") -> nn.Module:
    """Build model_class(**model_kwargs) and fill it from a checkpoint
    (mxtorch.py:9900-10004): an MX-native one restores the saved packed
    tensors unchanged; a plain state dict is loaded and its nn.Linear
    layers whose names match `dtype`'s patterns are quantized."""
    model = model_class(**(model_kwargs or {}))
    ckpt = torch.load(checkpoint_path, map_location="cpu", weights_only=True)
    dev = torch.device(device)
    if isinstance(ckpt, dict) and "__mx_version__" in ckpt:
        mods = dict(model.named_modules())
        linear_parts: Dict[str, Dict[str, mx_tensor]] = {}
        for key, entry in ckpt.items():
            if key == "__mx_version__":
                continue
            mod_name, _, attr = key.rpartition(".")
            if mod_name not in mods:
                continue
            t = mx_tensor(entry["packed"].to(dev), entry["scales"].to(dev), get_mx_dtype(entry["dtype"]),
                          torch.Size(entry["shape"]), int(entry["n"]), int(entry["block"]), seed=entry.get("seed"))
            if attr in ("_mx_weight", "_mx_bias"):
                linear_parts.setdefault(mod_name, {})[attr] = t
                continue
            mod = mods[mod_name]
            if attr in getattr(mod, "_parameters", {}):
                del mod._parameters[attr]
            setattr(mod, attr, t)
        for mod_name, parts in linear_parts.items():
            mod = mods[mod_name]
            w = parts.get("_mx_weight")
            if isinstance(mod, mx_linear):
                target = mod
            elif w is not None:
                in_f, out_f = (int(w._mx_orig_shape[0]), int(w._mx_orig_shape[1]))
                target = mx_linear.__new__(mx_linear)
                nn.Module.__init__(target)
                target.in_features, target.out_features = in_f, out_f
                target.mx_dtype, target.block, target.apply_bias = w._mx_dtype, w._mx_block, False
                target.register_buffer("_mx_weight", None)
                target.register_buffer("_mx_bias", None)
                if mod_name:
                    _set_submodule(model, mod_name, target)
                else:
                    model = target
            else:
                continue
            for attr, t in parts.items():
                setattr(target, attr, t)
        return model

    state = ckpt.get("state_dict") or ckpt.get("model") or ckpt if isinstance(ckpt, dict) else None
    if not isinstance(state, dict):
        raise ValueError(f"Cannot parse checkpoint at {checkpoint_path}")
    model.load_state_dict({k: v for k, v in state.items() if isinstance(v, torch.Tensor)}, strict=False)
    model = model.to(dev)
    dmap = {".*": dtype} if isinstance(dtype, str) else dict(dtype)
    dmap = {p: d for p, d in dmap.items() if d not in _FLOAT_NAMES}
    if dmap:
        model = to_mx(model, dmap, block_size)
    return model


def checkpoint_nbytes(path: str) -> int:
    return os.path.getsize(path)
