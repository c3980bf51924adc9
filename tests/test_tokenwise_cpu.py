"""CPU tests of the tokenwise modules' install-time surface: buffer names,
layouts, dtypes and byte counts against the oracle's packers and codebooks
(the reference's own constructors, w4a8_triton.py:353-389,
w8a8_triton.py:93-112, w2a8_triton.py:128-170, wxa4_native.py:226-353),
argument checks and messages, replace helpers and the request-scoped
caches and counters."""
import numpy as np
import pytest
import torch

from actune_amd.kernels import tokenwise as T
from oracle import oracle as O


def _linear(n, k, bias=True, seed=0):
    torch.manual_seed(seed)
    return torch.nn.Linear(k, n, bias=bias, dtype=torch.bfloat16)


def _w(lin):
    return lin.weight.detach().float().numpy()


def test_w4a8_buffers_match_oracle_layout():
    lin = _linear(48, 256)
    mod = T.W4A8TritonLinear(lin)
    codes, scale = O.weight_codes(_w(lin), 4, 8)
    assert mod.packed_weight.dtype == torch.uint8 and tuple(mod.packed_weight.shape) == (128, 48)
    np.testing.assert_array_equal(mod.packed_weight.numpy(), O.pack_kmajor(codes, 4))
    np.testing.assert_array_equal(mod.weight_scale.numpy(), scale)
    assert mod.bias.dtype == torch.bfloat16 and torch.equal(mod.bias, lin.bias)
    assert mod.weight_quantizer == "rtn_per_output_row_v1" and mod.gemv_max_rows == 0
    clipped = T.W4A8TritonLinear(lin, weight_clip_ratios=0.9)
    c2, s2 = O.weight_codes(_w(lin), 4, 8, 0.9)
    np.testing.assert_array_equal(clipped.packed_weight.numpy(), O.pack_kmajor(c2, 4))
    np.testing.assert_array_equal(clipped.weight_scale.numpy(), s2)
    assert clipped.weight_quantizer == "awq_style_nested_clip_v1"


def test_w8a8_and_w2a8_buffers():
    lin = _linear(32, 256, bias=False)
    m8 = T.W8A8TritonLinear(lin)
    c8, s8 = O.weight_codes(_w(lin), 8, 8)
    assert m8.weight_int8.dtype == torch.int8 and tuple(m8.weight_int8.shape) == (256, 32)
    np.testing.assert_array_equal(m8.weight_int8.numpy(), O.pack_kmajor(c8, 8))
    np.testing.assert_array_equal(m8.weight_scale.numpy(), s8)
    assert m8.bias is None
    ratios = torch.linspace(0.5, 1.0, 32)
    m2 = T.W2A8TritonLinear(lin, weight_clip_ratios=ratios)
    c2, s2 = O.weight_codes(_w(lin), 2, 8, ratios.numpy())
    assert tuple(m2.packed_weight.shape) == (64, 32)
    np.testing.assert_array_equal(m2.packed_weight.numpy(), O.pack_kmajor(c2, 2))
    np.testing.assert_array_equal(m2.weight_scale.numpy(), s2)
    assert m2.weight_quantizer == "awq_style_joint_precision_lattice_clip_v1"


@pytest.mark.parametrize("cls,bits", [(T.W4A4NativeLinear, 4), (T.W2A4NativeLinear, 2)])
def test_native_a4_buffers(cls, bits):
    lin = _linear(40, 128)
    mod = cls(lin)
    codes, scale = O.weight_codes(_w(lin), bits, 4)
    np.testing.assert_array_equal(mod.packed_weight.numpy(), O.pack_rows(codes, bits))
    np.testing.assert_array_equal(mod.weight_scale.numpy(), scale)
    assert mod.bias.dtype == torch.float32 and torch.equal(mod.bias, lin.bias.float())
    assert mod.weight_bits == bits and mod.native_int4_tensor_core
    assert mod.activation_quantizer == "dynamic_per_row_s4_v1"
    nobias = cls(_linear(40, 128, bias=False))
    assert nobias.bias.numel() == 0 and nobias.bias.dtype == torch.float32


def test_w8a4_nested_buffers():
    lin = _linear(32, 256)
    mod = T.W8A4NativeLinear(lin)
    codes, scale = O.weight_codes(_w(lin), 8, 4)
    np.testing.assert_array_equal(mod.weight_int8.numpy(), O.pack_kmajor(codes, 8))
    np.testing.assert_array_equal(mod.weight_scale.numpy(), scale)
    assert mod.weight_bits == 8 and mod.a4_sign_extended_to_int8 and not mod.native_int4_tensor_core


@pytest.mark.parametrize("cls,k,msg", [
    (T.W4A8TritonLinear, 48, "divisible by 32"), (T.W8A8TritonLinear, 64, "divisible by 128"),
    (T.W2A8TritonLinear, 192, "divisible by 128"), (T.W4A4NativeLinear, 96, "divisible by 64"),
    (T.W8A4NativeLinear, 64, "divisible by 128"),
])
def test_in_features_checks(cls, k, msg):
    with pytest.raises(ValueError, match=msg):
        cls(_linear(16, k))


def test_forward_requires_cuda():
    for mod in (T.W4A8TritonLinear(_linear(16, 64)), T.W4A4NativeLinear(_linear(16, 64))):
        with pytest.raises(ValueError, match="CUDA"):
            mod(torch.zeros(1, 64, dtype=torch.bfloat16))


def test_replace_helpers():
    model = torch.nn.Sequential(torch.nn.Linear(128, 32), torch.nn.Sequential(torch.nn.Linear(128, 16)))
    n = T.replace_with_w8a8_triton_(model, lambda child, name: isinstance(child, torch.nn.Linear))
    assert n == 2 and isinstance(model[0], T.W8A8TritonLinear) and isinstance(model[1][0], T.W8A8TritonLinear)


def test_shared_cache_scope_and_counters():
    with T.shared_a8_cache_scope(enabled=False) as state:
        assert T.current_shared_a8_cache() is state and not state.enabled
        assert state.hits == state.misses == 0
    with T.decode_optimization_scope(enabled=False) as stats:
        assert not T.decode_enabled()
        assert set(stats.metrics()) == {"split_k_calls", "projection_groups", "projection_calls_fused",
                                        "partial_kernels", "reduction_kernels", "resident_quantization_kernels",
                                        "graph_replays", "graph_quantization_kernels"}
        with T.runtime_optimization_scope(dense_candidates=True):
            assert not T.decode_enabled() and T.dense_candidates_enabled()
        assert not T.dense_candidates_enabled()
    assert T.decode_enabled()
    with T.runtime_optimization_scope(dense_candidates=True) as rs:
        assert T.dense_candidates_enabled() and T.runtime_stats_dict(rs) == {
            "resident_a8_kernels": 0, "mlp_graph_replays": 0, "predecoded_r4_gemms": 0}
        with T.runtime_optimization_scope() as inner:
            assert T.dense_candidates_enabled() and inner is not rs  # None keeps the enclosing setting
    assert not T.dense_candidates_enabled()
    T.clear_shared_a8_cache()
    assert T.current_shared_a8_cache() is not None


def test_replace_is_all_or_nothing():
    """A selected layer the backend cannot take (in_features not a multiple
    of 32 for W4A8) makes the helper raise before anything is replaced."""
    model = torch.nn.Sequential(torch.nn.Linear(128, 32), torch.nn.Linear(100, 24))
    with pytest.raises(ValueError, match="divisible by 32"):
        T.replace_with_w4a8_triton_(model, lambda child, name: isinstance(child, torch.nn.Linear))
    assert all(type(m) is torch.nn.Linear for m in model)


def test_k_major_modules_take_any_output_width():
    """out_features need not be a multiple of 16 (the reference takes any):
    the buffers keep the reference's shapes; the kernels run on padded
    copies made at the first call."""
    model = torch.nn.Sequential(torch.nn.Linear(128, 32), torch.nn.Linear(128, 24))
    assert T.replace_with_w4a8_triton_(model, lambda child, name: isinstance(child, torch.nn.Linear)) == 2
    assert model[1].packed_weight.shape == (64, 24) and model[1].weight_scale.shape == (24,)
    for cls in (T.W8A8TritonLinear, T.W2A8TritonLinear, T.W8A4NativeLinear):
        mod = cls(torch.nn.Linear(128, 40))
        assert mod.out_features == 40 and mod.weight_scale.shape == (40,)


def test_decode_eligibility():
    x = torch.zeros(1, 4096, dtype=torch.bfloat16)
    assert not T.decode_eligible(x, k=4096)  # not on a GPU
    assert not T.decode_eligible(torch.zeros(2, 4096, dtype=torch.bfloat16), k=4096)
