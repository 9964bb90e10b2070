"""On-disk format (save_quantized / load_quantized, mxtorch.py:9860-10004) and
mx_tensor pickling (mxtorch.py:6418-6425), on the CPU: the packed codes and
scales must come back byte for byte.  The quantized tensors are built from
the oracle's quantizer (no GPU needed to move bytes)."""
import pickle

import torch
import torch.nn as nn

from oracle import mx_oracle as orc
from tests import _golden as G


def _mx(qa, x, name, block=128):
    p, s, n = orc.quantize(x, name, block)
    return qa.mx_tensor(p, s, qa.get_mx_dtype(name), x.shape, n, block)


def _mlp():
    torch.manual_seed(0)
    return nn.Sequential(nn.Linear(256, 128), nn.ReLU(), nn.Linear(128, 64, bias=False))


def _shell(qa, lin: nn.Linear, name: str):
    """An mx_linear holding the packed weight from_linear would store
    (quantize(weight.t()), mxtorch.py:7447), built without a GPU."""
    m = qa.mx_linear.__new__(qa.mx_linear)
    nn.Module.__init__(m)
    m.in_features, m.out_features = lin.in_features, lin.out_features
    m.mx_dtype, m.block, m.apply_bias = qa.get_mx_dtype(name), 128, False
    m._mx_weight = _mx(qa, lin.weight.data.t().contiguous(), name)
    m._mx_bias = _mx(qa, lin.bias.data, name) if lin.bias is not None else None
    return m


def _same(a, b):
    return (a._mx_dtype.name == b._mx_dtype.name and tuple(a._mx_orig_shape) == tuple(b._mx_orig_shape)
            and a._mx_n == b._mx_n and a._mx_block == b._mx_block
            and G.bits_equal(a._mx_packed.cpu(), b._mx_packed.cpu())
            and G.bits_equal(a._mx_scales.cpu(), b._mx_scales.cpu()))


def test_mx_linear_round_trip(tmp_path):
    import qtpytorch_amd as qa
    ref = _mlp()
    model = _mlp()
    model[0] = _shell(qa, ref[0], "int4d")
    model[2] = _shell(qa, ref[2], "int8d")
    path = qa.save_quantized(model, str(tmp_path / "m.pt"))
    raw = torch.load(path, map_location="cpu", weights_only=True)   # loads with the safe loader
    assert raw["__mx_version__"] == 2
    assert set(raw) == {"__mx_version__", "0._mx_weight", "0._mx_bias", "2._mx_weight"}
    assert raw["0._mx_weight"]["shape"] == [256, 128] and raw["0._mx_weight"]["dtype"] == "int4d"
    loaded = qa.load_quantized(path, _mlp)
    assert isinstance(loaded[0], qa.mx_linear) and isinstance(loaded[2], qa.mx_linear)
    assert isinstance(loaded[1], nn.ReLU)
    assert loaded[0].in_features == 256 and loaded[0].out_features == 128 and loaded[2]._mx_bias is None
    assert _same(loaded[0]._mx_weight, model[0]._mx_weight)
    assert _same(loaded[0]._mx_bias, model[0]._mx_bias)
    assert _same(loaded[2]._mx_weight, model[2]._mx_weight)
    # the file holds little more than the packed bytes and scales
    payload = sum(t.numel() * t.element_size() for e in raw.values() if isinstance(e, dict)
                  for t in (e["packed"], e["scales"]))
    assert qa.io.checkpoint_nbytes(path) < payload + 16384


class _WithMxAttr(nn.Module):
    def __init__(self):
        super().__init__()
        self.proj = nn.Linear(64, 32)


def test_weight_attribute_round_trip(tmp_path):
    """A module whose "weight" holds an mx_tensor (the attributes the
    reference saves, mxtorch.py:9867-9893)."""
    import qtpytorch_amd as qa
    m = _WithMxAttr()
    w = _mx(qa, torch.randn(32, 64), "float4d")
    del m.proj._parameters["weight"]
    m.proj.weight = w
    path = qa.save_quantized(m, str(tmp_path / "w.pt"))
    back = qa.load_quantized(path, _WithMxAttr)
    assert isinstance(back.proj.weight, qa.mx_tensor) and _same(back.proj.weight, w)


def test_mx_tensor_pickle_round_trip():
    import qtpytorch_amd as qa
    for name in ("int4d", "int3d", "float8d", "int16d"):
        t = _mx(qa, torch.randn(5, 300), name)
        back = pickle.loads(pickle.dumps(t))
        assert isinstance(back, qa.mx_tensor) and _same(back, t)
