"""Tokenwise (per-row) packed-integer linears on the HIP backend.

One module for the reference's tokenwise family, with its public names:

* ``W4A8TritonLinear``, the shared dynamic-A8 cache (``shared_a8_cache_scope``,
  ``clear_shared_a8_cache``, ``SharedA8CacheStats``) and
  ``replace_with_w4a8_triton_`` (actune/kernels/w4a8_triton.py:204-455);
* ``W8A8TritonLinear`` / ``replace_with_w8a8_triton_`` (w8a8_triton.py:90-170);
* ``W2A8TritonLinear`` / ``replace_with_w2a8_triton_`` (w2a8_triton.py:125-228);
* ``W2A4NativeLinear``, ``W4A4NativeLinear``, ``W8A4NativeLinear``
  (wxa4_native.py:223-391);
* the exact split-K decode surface: ``decode_optimization_scope``,
  ``DecodeStats``, ``decode_eligible``, ``decode_linear``, ``launch_decode``,
  ``launch_decode_group``, ``DecodeGraphPlan``, ``graph_decode_linear``,
  ``graph_plan_key``, ``decode_workspace_summary``
  (decode_w4a8_triton.py:113-480);
* ``runtime_optimization_scope`` / ``RuntimeStats`` / ``runtime_stats_dict``
  (runtime_options.py) and ``resident_a8_eligible`` / ``launch_resident_a8``
  (resident_a8_triton.py).

Buffers keep the reference's names, layouts, dtypes and byte counts
(``packed_weight`` K-major nibble pairs [K/2, N] for W4A8, ``weight_int8``
K-major [K, N] for W8A8 / W8A4, quarters [K/4, N] for W2A8, row-major packed
rows [N, K*W/8] for W4A4 / W2A4), so state dicts load unchanged. Weight codes
are computed as torch computes them on the device of the layer they are built
from (a GPU divides by the constants 7 and 127 through their fp32
reciprocals, w4a8_triton.py:33-36).

Every product call is the library's per-row quantizer
(actune_tokenwise_quantize) and its int8-MFMA GEMM (actune_tokenwise_linear);
the int32 accumulation is exact over all of K, split across workgroups where
the grid would otherwise be too small, so results never depend on the split.
"""
from __future__ import annotations

import threading
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import asdict, dataclass, field
from typing import Any, Iterator

import torch

from .. import _native
from . import quantizers

# ---------------------------------------------------------------- workspaces


def _workspace(owner, m, n, k, w_layout, a_layout, device):
    """The owner's split-K partial-sum workspace, grown when a call needs
    more; None when the call runs unsplit."""
    need = _native.tokenwise_workspace_bytes(m, n, k, w_layout, a_layout)
    if need == 0:
        return None
    ws = getattr(owner, "_tw_workspace", None)
    if ws is None or ws.numel() < need or ws.device != device:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        owner._tw_workspace = ws
    return ws


def _gemm(owner, activation, a_layout, scale, weight, w_layout, weight_scale, bias, n, k, epilogue, dtype):
    out = torch.empty((activation.shape[0], n), device=activation.device, dtype=dtype)
    ws = _workspace(owner, activation.shape[0], n, k, w_layout, a_layout, activation.device)
    return _native.tokenwise_linear(activation, a_layout, scale, weight, w_layout, weight_scale, bias, n, k,
                                    epilogue, out, workspace=ws)


def _pack_kmajor(codes, bits):
    """int8 codes [N, K] -> the K-major layouts (w4a8_triton.py:380-383,
    w2a8_triton.py:149-159; bits 8 is the transpose)."""
    if bits == 8:
        return codes.t().contiguous()
    per = 8 // bits
    part = codes.shape[1] // per
    mask = (1 << bits) - 1
    packed = torch.zeros(codes.shape[0], part, dtype=torch.int16, device=codes.device)
    for i in range(per):
        packed |= (codes[:, i * part:(i + 1) * part].to(torch.int16) & mask) << (i * bits)
    return packed.to(torch.uint8).t().contiguous()


def _pack_signed(values, bits):
    """Consecutive signed codes along K, row-major (wxa4_native.py:206-220)."""
    if bits not in (2, 4):
        raise ValueError("bits must be 2 or 4")
    per = 8 // bits
    fields = values.to(torch.int16).reshape(values.shape[0], -1, per) & ((1 << bits) - 1)
    packed = torch.zeros(fields.shape[:2], dtype=torch.int16, device=values.device)
    for j in range(per):
        packed |= fields[..., j] << (j * bits)
    return packed.to(torch.uint8).contiguous()


def _require_cuda(value, what):
    if not value.is_cuda:
        raise ValueError(f"{what} requires a CUDA input")


def _kmajor_width_ok(out_features):
    if out_features % 16:
        raise ValueError("K-major tokenwise weights need out_features divisible by 16 on this backend")


# ---------------------------------------------------------------- runtime options
_RUNTIME_ENABLED: ContextVar[bool] = ContextVar("vla_runtime_optimization_enabled", default=True)
_DENSE_CANDIDATES: ContextVar[bool] = ContextVar("vla_dense_runtime_candidates", default=False)
_RUNTIME_STATE: ContextVar[Any] = ContextVar("vla_runtime_optimization_stats", default=None)


@dataclass
class RuntimeStats:
    resident_a8_kernels: int = 0
    mlp_graph_replays: int = 0
    predecoded_r4_gemms: int = 0


@contextmanager
def runtime_optimization_scope(*, enabled=True, dense_candidates=None):
    """Request-local runtime switches and counters (runtime_options.py:20-35)."""
    dense_token = None if dense_candidates is None else _DENSE_CANDIDATES.set(dense_candidates)
    state = RuntimeStats()
    switch = _RUNTIME_ENABLED.set(enabled)
    token = _RUNTIME_STATE.set(state)
    try:
        yield state
    finally:
        _RUNTIME_STATE.reset(token)
        _RUNTIME_ENABLED.reset(switch)
        if dense_token is not None:
            _DENSE_CANDIDATES.reset(dense_token)


def runtime_stats_dict(state):
    return asdict(state)


# ---------------------------------------------------------------- decode switches and counters
_DECODE_ENABLED: ContextVar[bool] = ContextVar("vla_decode_optimization_enabled", default=True)


@dataclass
class DecodeStats:
    split_k_calls: int = 0
    projection_groups: int = 0
    projection_calls_fused: int = 0
    partial_kernels: int = 0
    reduction_kernels: int = 0
    resident_quantization_kernels: int = 0
    graph_replays: int = 0
    graph_quantization_kernels: int = 0
    pending: dict = field(default_factory=dict, repr=False)

    def metrics(self) -> dict:
        return {name: getattr(self, name) for name in (
            "split_k_calls", "projection_groups", "projection_calls_fused", "partial_kernels",
            "reduction_kernels", "resident_quantization_kernels", "graph_replays", "graph_quantization_kernels")}


_DECODE_STATE: ContextVar[DecodeStats | None] = ContextVar("vla_decode_state", default=None)


@contextmanager
def decode_optimization_scope(*, enabled: bool = True):
    """Bound decode fusion results and counters to one model forward
    (decode_w4a8_triton.py:278-289)."""
    state = DecodeStats()
    switch = _DECODE_ENABLED.set(enabled)
    token = _DECODE_STATE.set(state)
    try:
        yield state
    finally:
        state.pending.clear()
        _DECODE_STATE.reset(token)
        _DECODE_ENABLED.reset(switch)


def decode_eligible(value: torch.Tensor, *, k: int, n: int | None = None) -> bool:
    """Single-token bf16 calls take the split-K decode path. The reference
    restricts it to its measured shapes on one GPU generation
    (decode_w4a8_triton.py:297-309); here every shape the kernel takes
    qualifies (the split is chosen per shape)."""
    return (_DECODE_ENABLED.get() and value.is_cuda and value.dtype == torch.bfloat16 and value.numel() == k
            and value.shape[-1] == k and value.is_contiguous() and k % 64 == 0
            and (n is None or n % 16 == 0))


def resident_a8_eligible(value):
    """Opt-in dense candidate (resident_a8_triton.py:24-34): any contiguous
    bf16 activation on the GPU while the runtime switches allow it."""
    return (_DENSE_CANDIDATES.get() and _RUNTIME_ENABLED.get() and _DECODE_ENABLED.get() and value.is_cuda
            and value.dtype == torch.bfloat16 and value.dim() == 2 and value.is_contiguous())


def launch_resident_a8(value, activation, scale):
    """Per-row A8 quantization into caller-owned buffers (resident_a8_triton.py:37-42)."""
    _native.tokenwise_quantize(value, 8, activation, scale)
    state = _RUNTIME_STATE.get()
    if state is not None:
        state.resident_a8_kernels += 1


# ---------------------------------------------------------------- shared dynamic-A8 cache
class _SharedA8Entry:
    """One task-local dynamic-A8 result shared by sibling projections."""

    __slots__ = ("source", "in_features", "activation", "scale")

    def __init__(self, source, in_features, activation, scale):
        self.source = source
        self.in_features = in_features
        self.activation = activation
        self.scale = scale


class _A4Entry:
    __slots__ = ("source", "in_features", "packed", "scale")

    def __init__(self, source, in_features, packed, scale):
        self.source = source
        self.in_features = in_features
        self.packed = packed
        self.scale = scale


class SharedA8CacheStats:
    """Mutable statistics and one-entry workspace for a policy forward."""

    __slots__ = ("enabled", "entry", "a4_entry", "hits", "misses")

    def __init__(self, *, enabled: bool = True) -> None:
        self.enabled = enabled
        self.entry = None
        self.a4_entry = None
        self.hits = 0
        self.misses = 0


_SHARED_A8_STATE: ContextVar[SharedA8CacheStats | None] = ContextVar("vla_shared_dynamic_a8_state", default=None)


def clear_shared_a8_cache() -> None:
    """Drop the task-local sibling-projection activation cache."""
    state = _SHARED_A8_STATE.get()
    if state is None:
        _SHARED_A8_STATE.set(SharedA8CacheStats())
    else:
        state.entry = None
        state.a4_entry = None


@contextmanager
def shared_a8_cache_scope(*, enabled: bool = True) -> Iterator[SharedA8CacheStats]:
    """Bound cache lifetime to one policy forward and release its workspace."""
    state = SharedA8CacheStats(enabled=enabled)
    token = _SHARED_A8_STATE.set(state)
    try:
        yield state
    finally:
        _SHARED_A8_STATE.reset(token)


def _quantize_rows_shared(source, flat, *, in_features):
    """Quantize once and reuse for adjacent linears on the same tensor
    (w4a8_triton.py:270-325): per-row A8 depends only on the input and K,
    so q/k/v (or gate/up) share one quantizer launch whatever their weights."""
    if not source.is_cuda or flat.shape[-1] != in_features:
        raise ValueError("shared A8 quantization requires a CUDA input with matching K")
    state = _SHARED_A8_STATE.get()
    if state is None:
        state = SharedA8CacheStats()
        _SHARED_A8_STATE.set(state)
    entry = state.entry
    if (state.enabled and entry is not None and entry.source is source and entry.in_features == in_features
            and entry.activation.shape == flat.shape):
        state.hits += 1
        return entry.activation, entry.scale
    flat = flat.contiguous()
    activation, scale = _native.tokenwise_quantize(flat, 8)
    if resident_a8_eligible(flat):
        rstate = _RUNTIME_STATE.get()
        if rstate is not None:
            rstate.resident_a8_kernels += 1
    elif decode_eligible(flat, k=in_features):
        dstate = _DECODE_STATE.get()
        if dstate is not None:
            dstate.resident_quantization_kernels += 1
    state.misses += 1
    state.entry = _SharedA8Entry(source, in_features, activation, scale) if state.enabled else None
    return activation, scale


def _quantize_a4_shared(source, flat, *, in_features):
    """Per-row A4 codes (wxa4_native.py:123-160), reused inside an enabled
    shared-cache scope for the same source tensor."""
    if not source.is_cuda or flat.shape[-1] != in_features:
        raise ValueError("native A4 quantization requires a CUDA input with matching K")
    state = _SHARED_A8_STATE.get()
    entry = None if state is None else state.a4_entry
    if (entry is not None and entry.source is source and entry.in_features == in_features
            and entry.packed.shape[0] == flat.shape[0]):
        return entry.packed, entry.scale
    packed, scale = _native.tokenwise_quantize(flat.contiguous(), 4)
    if state is not None and state.enabled:
        state.a4_entry = _A4Entry(source, in_features, packed, scale)
    return packed, scale


# ---------------------------------------------------------------- A8 family
class _TokenwiseA8(torch.nn.Module):
    """Shared forward of the per-row A8 modules."""

    _layout = None
    _weight_name = None

    def _quantize(self, flat, *, source=None):
        if self.fused_quantization:
            return _quantize_rows_shared(flat if source is None else source, flat, in_features=self.in_features)
        return _native.tokenwise_quantize(flat.contiguous(), 8)

    def _fuses_rows(self, flat):
        """Two to eight 16-bit rows outside a shared-cache scope: the GEMM
        launch quantizes them itself (actune_tokenwise_linear_x), one launch
        fewer than the quantizer + GEMM pair, with the same codes and
        outputs. Inside an enabled scope the siblings share one quantizer
        launch instead."""
        state = _SHARED_A8_STATE.get()
        m = flat.shape[0]
        return (self.fused_quantization and 2 <= m <= 8 and flat.dtype in (torch.bfloat16, torch.float16)
                and self.in_features <= _native.tokenwise_fused_max_k(m)
                and (state is None or not state.enabled))

    def _linear(self, value):
        _require_cuda(value, type(self).__name__)
        original_shape = value.shape[:-1]
        flat = value.reshape(-1, self.in_features)
        if self._fuses_rows(flat):
            m = flat.shape[0]
            out = torch.empty((m, self.out_features), device=flat.device, dtype=value.dtype)
            scale = torch.empty(m, device=flat.device, dtype=torch.float32)
            ws = _workspace(self, m, self.out_features, self.in_features, self._layout, _native.TW_ACT_A8,
                            flat.device)
            _native.tokenwise_linear_x(flat.contiguous(), scale, getattr(self, self._weight_name), self._layout,
                                       self.weight_scale, self.bias, self.out_features, self.in_features,
                                       _native.TW_EPI_A8, out, workspace=ws)
            return out.reshape(*original_shape, self.out_features)
        activation, scale = self._quantize(flat, source=value)
        if self._layout == _native.TW_KMAJOR_W4 and decode_eligible(flat, k=self.in_features, n=self.out_features):
            state = _DECODE_STATE.get()
            if state is not None:
                state.split_k_calls += 1
                state.partial_kernels += 1
                state.reduction_kernels += 1
        output = _gemm(self, activation, _native.TW_ACT_A8, scale, getattr(self, self._weight_name), self._layout,
                       self.weight_scale, self.bias, self.out_features, self.in_features, _native.TW_EPI_A8,
                       value.dtype)
        return output.reshape(*original_shape, self.out_features)


class W4A8TritonLinear(_TokenwiseA8):
    """Inference-only linear with K-major packed symmetric INT4 weights and
    per-row dynamic INT8 activations (w4a8_triton.py:344-444)."""

    # the reference's GEMV program is kept behind a threshold for measurement
    # only; here one kernel serves every row count
    gemv_max_rows = 0
    _layout = _native.TW_KMAJOR_W4
    _weight_name = "packed_weight"

    def __init__(self, linear, fused_quantization=True, *, weight_clip_ratios=None):
        super().__init__()
        if linear.in_features % 32:
            raise ValueError("in_features must be divisible by 32")
        _kmajor_width_ok(linear.out_features)
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.fused_quantization = fused_quantization
        with torch.no_grad():
            weight = linear.weight.detach()
            quantized, scale = quantizers.symmetric_int4_quantize(weight, clip_ratios=weight_clip_ratios,
                                                                  gpu_division=weight.is_cuda)
            self.weight_quantizer = "rtn_per_output_row_v1" if weight_clip_ratios is None \
                else "awq_style_nested_clip_v1"
            packed = _pack_kmajor(quantized, 4)
        self.register_buffer("packed_weight", packed)
        self.register_buffer("weight_scale", scale.contiguous())
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().clone())

    def forward(self, value):
        if (self.fused_quantization and decode_eligible(value, k=self.in_features, n=self.out_features)
                and not torch.cuda.is_current_stream_capturing()):
            return graph_decode_linear(self, value, self.packed_weight, None, self.weight_scale, self.bias)
        return self._linear(value)


class W8A8TritonLinear(_TokenwiseA8):
    """Inference-only linear with K-major signed INT8 weights (w8a8_triton.py:90-157)."""

    _layout = _native.TW_KMAJOR_W8
    _weight_name = "weight_int8"

    def __init__(self, linear, fused_quantization=True):
        super().__init__()
        if linear.in_features % 128:
            raise ValueError("in_features must be divisible by 128")
        _kmajor_width_ok(linear.out_features)
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.fused_quantization = fused_quantization
        with torch.no_grad():
            weight = linear.weight.detach()
            quantized, scale = quantizers.weight_codes(weight, 8, 8, gpu_division=weight.is_cuda)
        self.register_buffer("weight_int8", quantized.t().contiguous())
        self.register_buffer("weight_scale", scale.contiguous())
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().clone())

    def forward(self, value):
        return self._linear(value)


class W2A8TritonLinear(_TokenwiseA8):
    """Inference-only linear with K-major packed signed INT2 weights (w2a8_triton.py:125-215)."""

    _layout = _native.TW_KMAJOR_W2
    _weight_name = "packed_weight"

    def __init__(self, linear, fused_quantization=True, *, weight_clip_ratios=None):
        super().__init__()
        if linear.in_features % 128:
            raise ValueError("in_features must be divisible by 128")
        _kmajor_width_ok(linear.out_features)
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.fused_quantization = fused_quantization
        with torch.no_grad():
            quantized, scale = quantizers.symmetric_int2_quantize(linear.weight, clip_ratios=weight_clip_ratios)
            packed = _pack_kmajor(quantized, 2)
        self.register_buffer("packed_weight", packed)
        self.register_buffer("weight_scale", scale.contiguous())
        self.weight_quantizer = "rtn_per_output_row_w2_v1" if weight_clip_ratios is None \
            else "awq_style_joint_precision_lattice_clip_v1"
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().clone())

    def forward(self, value):
        return self._linear(value)


def _replace(module, filter_fn, factory):
    replaced = 0
    for name, child in list(module.named_children()):
        if filter_fn(child, name):
            setattr(module, name, factory(child))
            replaced += 1
        else:
            replaced += _replace(child, filter_fn, factory)
    return replaced


def replace_with_w4a8_triton_(module, filter_fn) -> int:
    """Recursively replace eligible Linear children (w4a8_triton.py:447-455)."""
    return _replace(module, filter_fn, W4A8TritonLinear)


def replace_with_w8a8_triton_(module, filter_fn) -> int:
    return _replace(module, filter_fn, W8A8TritonLinear)


def replace_with_w2a8_triton_(module, filter_fn) -> int:
    return _replace(module, filter_fn, W2A8TritonLinear)


# ---------------------------------------------------------------- native A4 family
class _WxA4NativeLinear(torch.nn.Module):
    """W2A4 / W4A4 with row-major packed weights (wxa4_native.py:223-288)."""

    weight_bits: int

    def __init__(self, linear, *, weight_bits, weight_clip_ratios=None):
        super().__init__()
        if linear.in_features % 64:
            raise ValueError("native S4 MMA requires in_features divisible by 64")
        if weight_bits not in (2, 4):
            raise ValueError("weight_bits must be 2 or 4")
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.weight_bits = weight_bits
        with torch.no_grad():
            weight = linear.weight.detach()
            if weight_bits == 2:
                quantized, scale = quantizers.symmetric_int2_quantize(weight, clip_ratios=weight_clip_ratios)
            else:
                quantized, scale = quantizers.symmetric_int4_quantize(weight, clip_ratios=weight_clip_ratios,
                                                                      gpu_division=weight.is_cuda)
            packed = _pack_signed(quantized, weight_bits)
        self.register_buffer("packed_weight", packed)
        self.register_buffer("weight_scale", scale.contiguous())
        self.register_buffer("bias", torch.empty(0, dtype=torch.float32, device=linear.weight.device)
                             if linear.bias is None else linear.bias.detach().float().contiguous())
        self.weight_quantizer = f"rtn_per_output_row_w{weight_bits}_v1" if weight_clip_ratios is None \
            else "awq_style_joint_precision_lattice_clip_v1"
        self.activation_quantizer = "dynamic_per_row_s4_v1"
        self.compute_instruction = "v_mfma_i32_16x16x64_i8 (S4/S2 fields at the top of int8 lanes)"
        self.native_int4_tensor_core = True

    def forward(self, value):
        if not value.is_cuda:
            raise ValueError("native S4 MMA requires a CUDA input")
        original_shape = value.shape[:-1]
        flat = value.reshape(-1, self.in_features)
        packed, activation_scale = _quantize_a4_shared(value, flat, in_features=self.in_features)
        layout = _native.TW_ROWS_S4 if self.weight_bits == 4 else _native.TW_ROWS_S2
        output = _gemm(self, packed, _native.TW_ACT_A4, activation_scale, self.packed_weight, layout,
                       self.weight_scale, self.bias if self.bias.numel() else None, self.out_features,
                       self.in_features, _native.TW_EPI_A4, value.dtype)
        return output.reshape(*original_shape, self.out_features)


class W2A4NativeLinear(_WxA4NativeLinear):
    def __init__(self, linear, *, weight_clip_ratios=None):
        super().__init__(linear, weight_bits=2, weight_clip_ratios=weight_clip_ratios)


class W4A4NativeLinear(_WxA4NativeLinear):
    def __init__(self, linear, *, weight_clip_ratios=None):
        super().__init__(linear, weight_bits=4, weight_clip_ratios=weight_clip_ratios)


class W8A4NativeLinear(torch.nn.Module):
    """INT8 nested-R4 weights x A4 activations as one int8 GEMM
    (wxa4_native.py:315-391); the packed A4 codes are unpacked in the kernel."""

    def __init__(self, linear, *, weight_clip_ratios=None):
        super().__init__()
        if linear.in_features % 128:
            raise ValueError("W8A4 S8 MMA requires in_features divisible by 128")
        _kmajor_width_ok(linear.out_features)
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        with torch.no_grad():
            weight = linear.weight.detach()
            q8, scale = quantizers.weight_codes(weight, 8, 4, clip_ratios=weight_clip_ratios,
                                                gpu_division=weight.is_cuda)
        self.register_buffer("weight_int8", q8.t().contiguous())
        self.register_buffer("weight_scale", scale.contiguous())
        self.register_buffer("bias", torch.empty(0, dtype=torch.float32, device=linear.weight.device)
                             if linear.bias is None else linear.bias.detach().float().contiguous())
        self.weight_bits = 8
        self.weight_quantizer = "nested_signed_w8_rtn_v1" if weight_clip_ratios is None \
            else "awq_style_joint_precision_lattice_clip_v1"
        self.activation_quantizer = "dynamic_per_row_s4_v1"
        self.compute_instruction = "v_mfma_i32_16x16x64_i8 (A4 codes at the top of int8 lanes)"
        self.native_int4_tensor_core = False
        self.native_int8_tensor_core = True
        self.a4_sign_extended_to_int8 = True
        self.s4_mma_count_per_k_tile = 0

    def forward(self, value):
        if not value.is_cuda:
            raise ValueError("W8A4 integer MMA requires a CUDA input")
        original_shape = value.shape[:-1]
        flat = value.reshape(-1, self.in_features)
        packed, activation_scale = _quantize_a4_shared(value, flat, in_features=self.in_features)
        output = _gemm(self, packed, _native.TW_ACT_A4, activation_scale, self.weight_int8, _native.TW_KMAJOR_W8,
                       self.weight_scale, self.bias if self.bias.numel() else None, self.out_features,
                       self.in_features, _native.TW_EPI_A8, value.dtype)
        return output.reshape(*original_shape, self.out_features)


# ---------------------------------------------------------------- exact split-K decode
# longest row the GEMM launch quantizes itself (actune_tokenwise_linear_x)
_FUSED_MAX_K = 16384


class _WorkspaceOwner:
    pass


_LAUNCH_OWNER = _WorkspaceOwner()


def _decode_check_residual(residual):
    if residual is not None:
        raise NotImplementedError("the signed-R4 residual decode layout is not part of this backend")


def launch_decode(activation, packed, residual, activation_scale, weight_scale, bias, output, partial, *,
                  config=None):
    """Launch into caller-owned buffers (decode_w4a8_triton.py:113-149).
    ``partial`` is the caller's split-K workspace (any dtype, at least the
    bytes actune_tokenwise_workspace_bytes() asks for; nothing in it needs
    to start at any value). ``config`` is accepted for signature parity; the
    split is chosen per shape."""
    _decode_check_residual(residual)
    n = packed.shape[1]
    k = packed.shape[0] * 2
    m = activation.numel() // k
    need = _native.tokenwise_workspace_bytes(m, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    ws = None
    if need:
        ws = partial.view(-1).view(torch.uint8)
        if ws.numel() < need:
            raise ValueError(f"partial workspace too small: {need} bytes needed")
    return _native.tokenwise_linear(activation.reshape(m, k), _native.TW_ACT_A8, activation_scale.reshape(-1),
                                    packed, _native.TW_KMAJOR_W4, weight_scale, bias, n, k, _native.TW_EPI_A8,
                                    output.view(m, n), workspace=ws)


def launch_decode_group(activation, weights, residuals, activation_scale, scales, biases, outputs, partial, *,
                        splits=16, bn=128):
    """Two or three projections sharing one quantized activation
    (decode_w4a8_triton.py:205-239): one split-K launch per projection
    on the shared codes."""
    for r in residuals:
        _decode_check_residual(r)
    n = weights[0].shape[1]
    k = weights[0].shape[0] * 2
    ws = partial.view(-1).view(torch.uint8)
    need = _native.tokenwise_workspace_bytes(1, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    if need and ws.numel() < need:
        raise ValueError(f"partial workspace too small: {need} bytes needed")
    for w, s, b, o in zip(weights, scales, biases, outputs):
        _native.tokenwise_linear(activation.reshape(1, k), _native.TW_ACT_A8, activation_scale.reshape(-1), w,
                                 _native.TW_KMAJOR_W4, s, b, n, k, _native.TW_EPI_A8, o.view(1, n),
                                 workspace=ws if need else None)


def decode_linear(activation, packed, residual, activation_scale, weight_scale, bias, output):
    """One split-K decode into `output` (decode_w4a8_triton.py:312-323)."""
    _decode_check_residual(residual)
    n = packed.shape[1]
    k = packed.shape[0] * 2
    m = activation.numel() // k
    _native.tokenwise_linear(activation.reshape(m, k), _native.TW_ACT_A8, activation_scale.reshape(-1), packed,
                             _native.TW_KMAJOR_W4, weight_scale, bias, n, k, _native.TW_EPI_A8, output.view(m, n),
                             workspace=_workspace(_LAUNCH_OWNER, m, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8,
                                                  activation.device))
    state = _DECODE_STATE.get()
    if state is not None:
        state.split_k_calls += 1
        state.partial_kernels += 1
        state.reduction_kernels += 1


class DecodeGraphPlan:
    """Replay the fixed decode launch sequence (per-row quantizer, then one
    split-K GEMM per projection) from a hipGraph with private staging
    buffers; inputs are copied in and outputs cloned on every call
    (decode_w4a8_triton.py:326-425). Where the row fits it
    (in_features <= 16384), each projection's split GEMM quantizes the row
    itself (actune_tokenwise_linear_x): two launches per projection and no
    quantizer launch, with the same codes and outputs."""

    def __init__(self, value, weights, residuals, scales, biases):
        for r in residuals:
            _decode_check_residual(r)
        self.lock = threading.Lock()
        self.weights = tuple(weights)
        self.residuals = tuple(residuals)
        self.scales = tuple(scales)
        self.biases = tuple(biases)
        self.k = weights[0].shape[0] * 2
        self.n = weights[0].shape[1]
        self.groups = len(weights)
        dev = value.device
        self.fused = self.k <= _FUSED_MAX_K and value.dtype in (torch.bfloat16, torch.float16, torch.float32)
        self.input = torch.empty((1, self.k), device=dev, dtype=value.dtype)
        self.activation = None if self.fused else torch.empty_like(self.input, dtype=torch.int8)
        self.scale = torch.empty(1, device=dev, dtype=torch.float32)
        self.output = torch.empty((self.groups, self.n), device=dev, dtype=value.dtype)
        self.outputs = tuple(self.output[i:i + 1] for i in range(self.groups))
        need = _native.tokenwise_workspace_bytes(1, self.n, self.k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
        self.partial = torch.empty(max(need, 256) * self.groups, device=dev, dtype=torch.uint8)
        self._need = need
        self.graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device=dev)
        current = torch.cuda.current_stream(dev)
        stream.wait_stream(current)
        with torch.cuda.stream(stream):
            self.input.copy_(value.reshape(1, self.k))
            for _ in range(3):
                self._launch()
        current.wait_stream(stream)
        with torch.cuda.graph(self.graph, stream=stream):
            self._launch()
        current.wait_stream(stream)

    def _launch(self):
        if not self.fused:
            _native.tokenwise_quantize(self.input, 8, self.activation, self.scale)
        step = max(self._need, 256)
        for i in range(self.groups):
            ws = self.partial[i * step:(i + 1) * step] if self._need else None
            if self.fused:
                _native.tokenwise_linear_x(self.input, self.scale, self.weights[i], _native.TW_KMAJOR_W4,
                                           self.scales[i], self.biases[i], self.n, self.k, _native.TW_EPI_A8,
                                           self.outputs[i], workspace=ws)
            else:
                _native.tokenwise_linear(self.activation, _native.TW_ACT_A8, self.scale, self.weights[i],
                                         _native.TW_KMAJOR_W4, self.scales[i], self.biases[i], self.n, self.k,
                                         _native.TW_EPI_A8, self.outputs[i], workspace=ws)

    @property
    def workspace_bytes(self):
        return sum(t.numel() * t.element_size()
                   for t in (self.input, self.activation, self.scale, self.output, self.partial) if t is not None)

    def run(self, value):
        with self.lock:
            self.input.copy_(value.reshape(1, self.k))
            self.graph.replay()
            output = self.output.clone()
        state = _DECODE_STATE.get()
        if state is not None:
            state.graph_replays += 1
            state.graph_quantization_kernels += 1
            state.resident_quantization_kernels += 1
            state.partial_kernels += 1
            state.reduction_kernels += 1
            if self.groups == 1:
                state.split_k_calls += 1
            else:
                state.projection_groups += 1
                state.projection_calls_fused += self.groups
        return output


def _tensor_version(tensor):
    if tensor is None or tensor.is_inference():
        return None
    return tensor._version


def graph_plan_key(value, weights, residuals, scales, biases):
    return (torch.cuda.current_stream(value.device).cuda_stream,
            tuple((id(t), _tensor_version(t)) for t in (*weights, *residuals, *scales, *biases)))


def graph_decode_linear(owner, value, packed, residual, scale, bias):
    """Cached DecodeGraphPlan per (stream, tensor identities) on the owning
    module (decode_w4a8_triton.py:441-455)."""
    cache = getattr(owner, "_decode_graph_plans", None)
    if cache is None:
        cache = {}
        owner._decode_graph_plans = cache
    key = graph_plan_key(value, (packed,), (residual,), (scale,), (bias,))
    plan = cache.get(key)
    if plan is None:
        if len(cache) >= 8:
            cache.clear()
        plan = DecodeGraphPlan(value, (packed,), (residual,), (scale,), (bias,))
        cache[key] = plan
    return plan.run(value).reshape(*value.shape[:-1], packed.shape[1])


def decode_workspace_summary(module):
    """Count explicit persistent buffers after warm-up (decode_w4a8_triton.py:458-480)."""
    plans = {}
    mlp_plans = {}
    for child in module.modules():
        for plan in getattr(child, "_decode_graph_plans", {}).values():
            plans[id(plan)] = plan
        controller = getattr(child, "_decode_mlp_controller", None)
        if controller is not None:
            for plan in controller.plans.values():
                mlp_plans[id(plan)] = plan
        group = getattr(child, "_decode_projection_group", None)
        if group is not None:
            for plan in group.plans.values():
                plans[id(plan)] = plan
    return {
        "decode_graph_plan_count": len(plans),
        "mlp_graph_plan_count": len(mlp_plans),
        "mlp_graph_input_output_bytes": sum(t.numel() * t.element_size()
                                            for plan in mlp_plans.values() for t in (plan.input, plan.output)),
        "decode_graph_explicit_workspace_bytes": sum(plan.workspace_bytes for plan in plans.values()),
    }
