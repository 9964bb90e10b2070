"""GPU round trip of the on-disk format (save_quantized / load_quantized,
mxtorch.py:9860-10004): packed bytes and forward outputs bitwise equal."""
import pytest
import torch

from tests import _golden as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qtpytorch_amd
    return qtpytorch_amd


def dev():
    return torch.device("cuda:0")


def _bits_eq(a, b):
    return G.bits_equal(a.detach().cpu(), b.detach().cpu())


class _MLP(torch.nn.Module):
    def __init__(self):
        super().__init__()
        torch.manual_seed(1)
        self.fc1 = torch.nn.Linear(512, 256)
        self.act = torch.nn.GELU()
        self.fc2 = torch.nn.Linear(256, 128, bias=False)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


def test_save_load_quantized_gpu(qa, tmp_path):
    """to_mx on the GPU, save_quantized, load_quantized back onto the GPU:
    the same packed bytes and the same forward output bit for bit; a plain
    state dict loaded with a dtype quantizes to the same bytes as to_mx."""
    x = torch.randn(16, 512, device=dev())
    model = qa.to_mx(_MLP().to(dev()), "int4d")
    y = model(x)
    path = qa.save_quantized(model, str(tmp_path / "q.pt"))
    back = qa.load_quantized(path, _MLP, device="cuda")
    assert isinstance(back.fc1, qa.mx_linear) and isinstance(back.fc2, qa.mx_linear)
    assert _bits_eq(back.fc1._mx_weight._mx_packed, model.fc1._mx_weight._mx_packed)
    assert _bits_eq(back(x), y)
    sd = str(tmp_path / "sd.pt")
    torch.save(_MLP().state_dict(), sd)
    from_sd = qa.load_quantized(sd, _MLP, dtype="int4d", device="cuda")
    assert _bits_eq(from_sd.fc1._mx_weight._mx_packed, model.fc1._mx_weight._mx_packed)
    assert _bits_eq(from_sd.fc2._mx_weight._mx_scales, model.fc2._mx_weight._mx_scales)
