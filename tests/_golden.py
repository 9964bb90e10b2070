"""Loader for the committed golden vectors (tests/golden/fixtures.npz).

The vectors were written by tests/golden/gen_fixtures.py from the
reference's own CPU path; loading uses numpy without pickle support.
"""
import json
import os

import numpy as np
import torch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_Z = None
_J = None


def arrays():
    global _Z
    if _Z is None:
        _Z = np.load(os.path.join(HERE, "fixtures.npz"), allow_pickle=False)
    return _Z


def index():
    global _J
    if _J is None:
        with open(os.path.join(HERE, "fixtures.json")) as f:
            _J = json.load(f)
    return _J


def get(key) -> torch.Tensor:
    return torch.from_numpy(np.array(arrays()[key]))


def has(key) -> bool:
    return key in arrays().files


def input_tensor(name) -> torch.Tensor:
    """Golden input; bf16 inputs are stored as their int16 bit patterns."""
    case = next((c for c in index()["cases"] if c["kind"] == "input" and c["key"] == f"in/{name}"),
                {"dtype": "torch.float32"})
    t = get(f"in/{name}")
    if case["dtype"] == "torch.bfloat16":
        t = t.view(torch.bfloat16)
    return t


def cases(kind):
    return [c for c in index()["cases"] if c["kind"] == kind]


def nan_aware_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality of float32 tensors where every NaN matches any NaN
    (a NaN's payload and sign depend on the hardware that made it)."""
    a = a.contiguous().reshape(-1)
    b = b.contiguous().reshape(-1)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    na, nb = torch.isnan(a), torch.isnan(b)
    if not torch.equal(na, nb):
        return False
    return torch.equal(a[~na].view(torch.int32), b[~nb].view(torch.int32))


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality (tells -0.0 from 0.0)."""
    a = a.contiguous()
    b = b.contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype in (torch.float32,):
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)
