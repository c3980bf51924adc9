"""reuse_mlp_temporary (grouped.py:18-36 counterpart): patching count,
idempotence, and the training-mode fallback to the original forward."""
import torch
from transformers import GemmaConfig
from transformers.models.gemma.modeling_gemma import GemmaMLP

from actune_amd.kernels.grouped import reuse_mlp_temporary


def _model():
    cfg = GemmaConfig(hidden_size=128, intermediate_size=256, hidden_activation="gelu_pytorch_tanh")
    return torch.nn.Sequential(GemmaMLP(cfg), torch.nn.Sequential(GemmaMLP(cfg)), torch.nn.Linear(128, 128))


def test_patches_every_gemma_mlp_once():
    model = _model()
    assert reuse_mlp_temporary(model) == 2
    assert reuse_mlp_temporary(model) == 0
    assert hasattr(model[0], "_group64_original_forward")


def test_grad_mode_uses_the_original_forward():
    model = _model()
    x = torch.randn(3, 128)
    want = model[0](x)
    reuse_mlp_temporary(model)
    with torch.enable_grad():
        got = model[0](x)
    assert torch.equal(got, want) and got.requires_grad
    with torch.no_grad():
        fused = model[0](x)  # CPU Linear children: the plain product path
    assert torch.allclose(fused, want.detach())
