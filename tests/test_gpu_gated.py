"""GPU parity of the gated-MLP quantizer (actune_quantize_gated) and of the
MLP forward built on it (gated_down_forward, the patched GemmaMLP forward).

Bar: codes and scales bit-exact against the group-64 quantizer run on the
product torch itself forms on the GPU (F.silu / F.gelu(approximate="tanh"),
then the product in the inputs' dtype): the quantizer is pinned to the
oracle elsewhere, so these tests pin the fused activation and product to
torch's own eager arithmetic. Every finite bf16 and f16 gate value is
checked in a group of its own (the group scale max|p| / 127 then fixes |p|
exactly, the code's sign its sign); fp32 on a large random sample.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from actune_amd import _native
from actune_amd.kernels.grouped import GroupedPaddedLinear, gated_down_forward, reuse_mlp_temporary
from actune_amd.layers import ResidentLinear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ACTS = {_native.ACT_SILU: F.silu, _native.ACT_GELU_TANH: lambda t: F.gelu(t, approximate="tanh")}


def _torch_codes(gate, up, act, A, scale=None):
    product = ACTS[act](gate)
    product.mul_(up)
    return _native.quantize_groups(product, A, input_scale=scale)


def _every_finite(dtype):
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    values = bits.view(dtype)
    return values[torch.isfinite(values)]


def _gated_in_calls(gate, up, act, A, rows):
    """quantize_gated over row slices of `rows` rows (all at once for None):
    at most 16384 groups per call take the quantizer's narrow geometry (2 or
    4 elements per lane), more take 8 per lane."""
    if rows is None:
        return _native.quantize_gated(gate, up, act, A)
    parts = [_native.quantize_gated(gate[i:i + rows], up[i:i + rows], act, A) for i in range(0, gate.shape[0], rows)]
    return torch.cat([p for p, _ in parts]), torch.cat([s for _, s in parts])


@pytest.mark.parametrize("rows", [None, 16384], ids=["wide", "narrow"])
@pytest.mark.parametrize("act", [_native.ACT_SILU, _native.ACT_GELU_TANH])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_every_gate_value_in_a_group_of_its_own(act, dtype, rows):
    """One group per finite gate value g = [g, 0 x 63] with up = 1: the scale
    of that group equals torch's for every value, so act(g) rounded to the
    dtype is torch's bit for bit wherever |act(g)| >= 127e-8 (below, the
    1e-8 floor of the scale hides it and the code is compared). In one call
    (8 elements per lane) and in calls of 16384 groups (2 per lane)."""
    values = _every_finite(dtype).to(DEV)
    gate = torch.zeros(values.numel(), 64, device=DEV, dtype=dtype)
    gate[:, 0] = values
    up = torch.ones_like(gate)
    got_p, got_s = _gated_in_calls(gate, up, act, 8, rows)
    want_p, want_s = _torch_codes(gate, up, act, 8)
    assert torch.equal(got_s, want_s)
    assert torch.equal(got_p, want_p)


@pytest.mark.parametrize("act", [_native.ACT_SILU, _native.ACT_GELU_TANH])
def test_fp32_gate_values_sampled(act):
    g = torch.Generator().manual_seed(act)
    values = torch.cat([torch.randn(1 << 20, generator=g) * s for s in (0.01, 1.0, 8.0, 100.0)])
    gate = torch.zeros(values.numel(), 64)
    gate[:, 0] = values
    gate = gate.to(DEV)
    up = torch.ones_like(gate)
    got = _native.quantize_gated(gate, up, act, 8)
    want = _torch_codes(gate, up, act, 8)
    assert torch.equal(got[1], want[1]) and torch.equal(got[0], want[0])


@pytest.mark.parametrize("act", [_native.ACT_SILU, _native.ACT_GELU_TANH])
@pytest.mark.parametrize("A", [8, 4, 2])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k", [(1, 1024), (50, 4096), (300, 16384), (7, 64), (3, 192), (16, 65536), (16385, 64)])
def test_products_equal_torch_then_quantizer(act, A, dtype, m, k):
    """Both lane geometries (narrow up to 16384 groups: the first, second,
    fourth to sixth shapes; 8 elements per lane above), ragged group counts
    (7, 9 and 16385 groups) and the channel-scale division."""
    g = torch.Generator().manual_seed(m + k + A)
    gate = (torch.randn(m, k, generator=g) * 3).to(dtype).to(DEV)
    up = torch.randn(m, k, generator=g).to(dtype).to(DEV)
    scale = torch.linspace(0.5, 2.0, k).to(dtype).to(DEV)
    for sd in (None, scale):
        got = _native.quantize_gated(gate, up, act, A, input_scale=sd)
        want = _torch_codes(gate, up, act, A, sd)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), sd is None


def test_rejects_bad_calls():
    gate = torch.randn(4, 128, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="up must match"):
        _native.quantize_gated(gate, gate[:, :64].contiguous(), _native.ACT_SILU, 4)
    with pytest.raises(ValueError, match="unknown gate activation"):
        _native.quantize_gated(gate, gate, 7, 4)
    lib = _native.lib()
    p = torch.empty(4, 64, dtype=torch.uint8, device=DEV)
    s = torch.empty(4, 2, device=DEV)
    assert lib.actune_quantize_gated(gate.data_ptr(), None, 0, 0, None, 4, 128, 4, p.data_ptr(), s.data_ptr(),
                                     None) != 0
    assert b"up operand" in lib.actune_last_error()


def _bank_linear(k, n, seed, assignments=None, scale=None):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(k, n, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
    lin = lin.to(DEV, torch.bfloat16)
    modes = assignments or {"q00": "w4a4", "q01": "w4a8", "q11": "w2a4", "q10": "w8a2"}
    clips = {m: None for m in set(modes.values())}
    if scale is not None:
        return ResidentLinear(lin, modes, clips, input_scale=scale)
    return GroupedPaddedLinear(lin, modes, "q11", clips)


@pytest.mark.parametrize("act_fn", [F.silu, torch.nn.SiLU(), torch.nn.GELU(approximate="tanh")])
@pytest.mark.parametrize("channel_scale", [False, True])
@pytest.mark.parametrize("m", [1, 50])
def test_gated_down_forward_equals_unfused(act_fn, channel_scale, m):
    """gated_down_forward on every precision profile (W2/W4/W8 x A2/A4/A8
    versions) equals act_fn(gate) * up fed to the module, bit for bit, and
    advances the module's counters like one call."""
    from actune_amd.precision import CONFIGURATIONS, precision_profile
    k, n = 4096, 1024
    scale = torch.linspace(0.5, 2.0, k) if channel_scale else None
    down = _bank_linear(k, n, seed=m + 3, scale=scale)
    g = torch.Generator().manual_seed(m)
    gate = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16).to(DEV)
    up = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    for q in CONFIGURATIONS:
        with precision_profile(q), torch.inference_mode():
            product = act_fn(gate)
            product.mul_(up)
            want = down(product)
            calls, elems = down.calls, down.input_elements
            got = gated_down_forward(down, gate, up, act_fn)
        assert torch.equal(got, want), q
        assert (down.calls, down.input_elements) == (calls + 1, elems + gate.numel())


def test_gated_down_forward_falls_back_where_it_cannot_fuse():
    """K padding (in_features 100), an activation the quantizer does not
    know, and a plain nn.Linear take the unfused calls."""
    gate = torch.randn(3, 100, device=DEV).to(torch.bfloat16)
    up = torch.randn(3, 100, device=DEV).to(torch.bfloat16)
    padded = _bank_linear(100, 64, seed=1)
    for down, act in ((padded, F.silu), (_bank_linear(128, 64, seed=2), torch.relu)):
        x, u = (gate, up) if down is padded else (torch.randn(3, 128, device=DEV).to(torch.bfloat16),) * 2
        with torch.inference_mode():
            product = act(x)
            product.mul_(u)
            assert torch.equal(gated_down_forward(down, x, u, act), down(product))
    plain = torch.nn.Linear(100, 64, device=DEV, dtype=torch.bfloat16)
    with torch.inference_mode():
        assert torch.equal(gated_down_forward(plain, gate, up, F.silu), plain(F.silu(gate) * up))


def test_patched_gemma_mlp_fuses_gelu_tanh_product(monkeypatch):
    """transformers' GemmaMLP (gelu_pytorch_tanh) patched by
    reuse_mlp_temporary: equal to the unpatched forward for every profile,
    and its down projection runs on the gated quantizer (in place of the
    activation, the product and the quantizer launches)."""
    from transformers import GemmaConfig
    from transformers.models.gemma.modeling_gemma import GemmaMLP
    from actune_amd.precision import CONFIGURATIONS, precision_profile
    cfg = GemmaConfig(hidden_size=1024, intermediate_size=4096, hidden_activation="gelu_pytorch_tanh")
    mlp = GemmaMLP(cfg).to(device=DEV, dtype=torch.bfloat16)
    modes = {"q00": "w4a4", "q01": "w2a4", "q11": "w2a4", "q10": "w4a8"}
    clips = {m: None for m in set(modes.values())}
    for name in ("gate_proj", "up_proj", "down_proj"):
        setattr(mlp, name, GroupedPaddedLinear(getattr(mlp, name), modes, "q11", clips))
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        want = {}
        for q in CONFIGURATIONS:
            with precision_profile(q):
                want[q] = mlp(x).clone()
        assert reuse_mlp_temporary(mlp) == 1
        for q in CONFIGURATIONS:
            with precision_profile(q):
                assert torch.equal(mlp(x), want[q]), q
        calls = []
        real = _native.quantize_gated
        monkeypatch.setattr(_native, "quantize_gated", lambda *a, **kw: calls.append(a[2]) or real(*a, **kw))
        with precision_profile("q00"):
            assert torch.equal(mlp(x), want["q00"])
    assert calls == [_native.ACT_GELU_TANH]
