"""The Hadamard ('h') rotation seed (mxtorch.py:1723, 1584) is the same in
every process and travels with the codes.

The reference seeds the rotation with ``hash(name) % 2**31``, which Python
salts per process.  The package's default is the value that expression has
in a PYTHONHASHSEED=0 process (ops.hadamard_seed, computed without calling
hash()); these tests pin it to that expression evaluated in such a
subprocess, to the seeds recorded next to the golden vectors, and check that
processes with different salts agree on the seed and the sign vector.  The
mx_tensor and checkpoint plumbing of the seed is checked on CPU tensors
(no GPU compute)."""
import json
import os
import pickle
import subprocess
import sys

import torch
import torch.nn as nn

from oracle import mx_oracle as orc
from tests import _golden as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _h_names():
    from qtpytorch_amd import dtypes as D
    return [n for n, d in D._DTYPE_REGISTRY.items() if d.is_hadamard]


def test_seed_equals_hash_under_pythonhashseed_0():
    from qtpytorch_amd import ops
    names = _h_names()
    assert len(names) == 48
    for n in names:
        assert ops.hadamard_seed(n) == orc.reference_hadamard_seed(n), n


def test_seed_matches_golden_record():
    from qtpytorch_amd import ops
    rec = G.index()["hash_seed"]
    assert rec["PYTHONHASHSEED"] == "0"
    for n in ("int4dh", "int8dh", "float4dh"):
        assert ops.hadamard_seed(n) == rec[n]


def test_siphash_known_answer():
    """SipHash-2-4 test vector of the published reference implementation:
    key 00 01 .. 0f, message 00 01 .. 0e (15 bytes) -> a129ca6149be45e5."""
    from qtpytorch_amd import ops
    k0 = int.from_bytes(bytes(range(8)), "little")
    k1 = int.from_bytes(bytes(range(8, 16)), "little")
    assert ops._siphash24(bytes(range(15)), k0, k1) == 0xA129CA6149BE45E5
    assert ops._siphash24(b"", k0, k1) == 0x726FDB47DD0E0E31


def _seed_and_signs_in_subprocess(hashseed: str):
    code = ("import json, sys; sys.path.insert(0, %r)\n"
            "from qtpytorch_amd import ops\n"
            "out = {n: ops.hadamard_seed(n) for n in ('int4dh', 'int2dh', 'float8dh')}\n"
            "out['signs'] = ops.hadamard_signs(128, ops.hadamard_seed('int4dh'), 'cpu').tolist()\n"
            "out['salted'] = hash('int4dh') %% (2 ** 31)\n"
            "print(json.dumps(out))\n") % ROOT
    env = dict(os.environ, PYTHONHASHSEED=hashseed)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_seed_is_process_independent():
    a = _seed_and_signs_in_subprocess("1")
    b = _seed_and_signs_in_subprocess("987654")
    assert a["salted"] != b["salted"]            # the salted hash itself differs between them
    for k in ("int4dh", "int2dh", "float8dh", "signs"):
        assert a[k] == b[k], k
    assert a["signs"] == orc.hadamard_signs(128, orc.reference_hadamard_seed("int4dh")).tolist()


def _h_tensor(qa, seed=None):
    x = torch.randn(4, 128, generator=torch.Generator().manual_seed(3))
    s = orc.reference_hadamard_seed("int4dh") if seed is None else seed
    p, sc, n = orc.quantize(x, "int4dh", 128, seed=s)
    return qa.mx_tensor(p, sc, qa.get_mx_dtype("int4dh"), x.shape, n, 128, seed=seed)


def test_mx_tensor_carries_seed():
    import qtpytorch_amd as qa
    t = _h_tensor(qa)
    assert t._mx_seed == qa.ops.hadamard_seed("int4dh")
    u = _h_tensor(qa, seed=424242)
    assert u._mx_seed == 424242
    for v in (u.clone(), u.detach(), u.cpu(), u.reshape(-1), pickle.loads(pickle.dumps(u))):
        assert v._mx_seed == 424242
    names, meta = u.__tensor_flatten__()
    r = qa.mx_tensor.__tensor_unflatten__({k: getattr(u, k) for k in names}, meta, None, None)
    assert r._mx_seed == 424242
    base = qa.mx_tensor(u._mx_packed, u._mx_scales, qa.get_mx_dtype("int4d"), u._mx_orig_shape, u._mx_n, 128)
    assert base._mx_seed is None


class _Holder(nn.Module):
    def __init__(self):
        super().__init__()
        self.proj = nn.Linear(128, 4, bias=False)


def test_checkpoint_keeps_seed_across_processes(tmp_path):
    """save_quantized writes the seed of an 'h' tensor; load_quantized in a
    process with another hash salt restores it (and the same codes)."""
    import qtpytorch_amd as qa
    m = _Holder()
    del m.proj._parameters["weight"]
    m.proj.weight = _h_tensor(qa, seed=777)
    path = qa.save_quantized(m, str(tmp_path / "h.pt"))
    raw = torch.load(path, map_location="cpu", weights_only=True)
    assert raw["proj.weight"]["seed"] == 777 and raw["proj.weight"]["dtype"] == "int4dh"
    code = ("import sys, json; sys.path.insert(0, %r)\n"
            "import torch.nn as nn, qtpytorch_amd as qa\n"
            "class _Holder(nn.Module):\n"
            "    def __init__(self):\n"
            "        super().__init__(); self.proj = nn.Linear(128, 4, bias=False)\n"
            "m = qa.load_quantized(%r, _Holder)\n"
            "w = m.proj.weight\n"
            "print(json.dumps({'seed': w._mx_seed, 'packed': w._mx_packed.tolist()}))\n") % (ROOT, path)
    env = dict(os.environ, PYTHONHASHSEED="31337")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["seed"] == 777
    assert out["packed"] == m.proj.weight._mx_packed.tolist()
