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
  (decode_w4a8_triton.py:113-480); sibling projections run as one GEMM
  launch plus one integer reduce (actune_tokenwise_linear_multi);
* ``runtime_optimization_scope`` / ``RuntimeStats`` / ``runtime_stats_dict``
  (runtime_options.py) and ``resident_a8_eligible`` / ``launch_resident_a8``
  (resident_a8_triton.py).

The request-scoped switches and counters live in two context variables of
this module (one immutable set of switches, one pair of counter objects),
read through ``decode_enabled()``, ``dense_candidates_enabled()`` and
``current_shared_a8_cache()``. Split-K partial sums get a fresh workspace
per call from the caching allocator (stream-ordered, and from the graph's
private pool under capture).

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
from collections import OrderedDict
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import asdict, dataclass
from typing import Iterator, NamedTuple

import torch

from .. import _native
from . import quantizers

# ---------------------------------------------------------------- request-scoped state
@dataclass(frozen=True)
class _Switches:
    """The request's tokenwise switches: ``runtime`` and ``dense`` belong to
    runtime_optimization_scope, ``decode`` to decode_optimization_scope.
    Replaced as a whole by each scope, so nested scopes restore cleanly."""

    runtime: bool = True
    dense: bool = False
    decode: bool = True


_SWITCHES: ContextVar[_Switches] = ContextVar("actune_tokenwise_switches", default=_Switches())
# (RuntimeStats or None, DecodeStats or None) of the innermost scopes
_COUNTERS: ContextVar[tuple] = ContextVar("actune_tokenwise_counters", default=(None, None))


@contextmanager
def _scoped(switches=None, runtime_stats=..., decode_stats=...):
    """Install new switches and / or counters for the body of a with-block."""
    old_rt, old_dec = _COUNTERS.get()
    counters = (old_rt if runtime_stats is ... else runtime_stats, old_dec if decode_stats is ... else decode_stats)
    tokens = [_COUNTERS.set(counters)]
    if switches is not None:
        tokens.append(_SWITCHES.set(switches))
    try:
        yield
    finally:
        for token in reversed(tokens):
            token.var.reset(token)


def _count(kind, **increments):
    """Add to the innermost scope's RuntimeStats (kind 0) or DecodeStats
    (kind 1), if a scope is open."""
    stats = _COUNTERS.get()[kind]
    if stats is not None:
        for name, value in increments.items():
            setattr(stats, name, getattr(stats, name) + value)


def decode_enabled() -> bool:
    """The decode switch of the innermost decode_optimization_scope (True
    outside any scope)."""
    return _SWITCHES.get().decode


def dense_candidates_enabled() -> bool:
    """The dense_candidates switch of the innermost runtime scope."""
    return _SWITCHES.get().dense


@dataclass
class RuntimeStats:
    """Counters of runtime_optimization_scope (runtime_options.py:13-17).
    resident_a8_kernels counts the dense-candidate row quantizations; this
    backend has no MLP graph controller and no pre-decoded R4 GEMM, so the
    other two stay 0 (the fields are kept for readers of the reference's
    dict)."""

    resident_a8_kernels: int = 0
    mlp_graph_replays: int = 0
    predecoded_r4_gemms: int = 0


@contextmanager
def runtime_optimization_scope(*, enabled=True, dense_candidates=None):
    """Request-local runtime switches with fresh counters; dense_candidates
    None keeps the enclosing setting (runtime_options.py:20-35)."""
    now = _SWITCHES.get()
    switches = _Switches(runtime=enabled, dense=now.dense if dense_candidates is None else bool(dense_candidates),
                         decode=now.decode)
    stats = RuntimeStats()
    with _scoped(switches, runtime_stats=stats):
        yield stats


def runtime_stats_dict(state):
    return asdict(state)


@dataclass
class DecodeStats:
    """Counters of one decode_optimization_scope (decode_w4a8_triton.py:242-257):
    every split decode linear (split_k_calls), every sibling group launched
    together (projection_groups, with its projections in
    projection_calls_fused), the split GEMM / integer reduce launches, the
    row quantizations on the decode path and the graph replays."""

    split_k_calls: int = 0
    projection_groups: int = 0
    projection_calls_fused: int = 0
    partial_kernels: int = 0
    reduction_kernels: int = 0
    resident_quantization_kernels: int = 0
    graph_replays: int = 0
    graph_quantization_kernels: int = 0

    def metrics(self) -> dict:
        return asdict(self)


@contextmanager
def decode_optimization_scope(*, enabled: bool = True):
    """Decode switch and fresh counters for one model forward."""
    now = _SWITCHES.get()
    stats = DecodeStats()
    with _scoped(_Switches(runtime=now.runtime, dense=now.dense, decode=enabled), decode_stats=stats):
        yield stats


def decode_eligible(value: torch.Tensor, *, k: int, n: int | None = None) -> bool:
    """Single-token bf16 calls take the split-K decode path. The reference
    restricts it to its measured shapes on one GPU generation
    (decode_w4a8_triton.py:297-309); here every shape the kernel takes
    qualifies (the split is chosen per shape)."""
    return (decode_enabled() and value.is_cuda and value.dtype == torch.bfloat16 and value.numel() == k
            and value.shape[-1] == k and value.is_contiguous() and k % 64 == 0
            and (n is None or n % 16 == 0))


def resident_a8_eligible(value):
    """Opt-in dense candidate (resident_a8_triton.py:24-34): any contiguous
    bf16 activation on the GPU while every switch allows it."""
    sw = _SWITCHES.get()
    return (sw.dense and sw.runtime and sw.decode and value.is_cuda and value.dtype == torch.bfloat16
            and value.dim() == 2 and value.is_contiguous())


def launch_resident_a8(value, activation, scale):
    """Per-row A8 quantization into caller-owned buffers (resident_a8_triton.py:37-42)."""
    _native.tokenwise_quantize(value, 8, activation, scale)
    _count(0, resident_a8_kernels=1)


# ---------------------------------------------------------------- split-K workspace and packing
def _split_workspace(m, n, k, w_layout, a_layout, device, targets=1):
    """A fresh workspace for one call's K-split partial sums (None when the
    call runs unsplit). Allocated per call from the caching allocator on the
    current stream: stream-ordered, and taken from the graph's private pool
    while a capture is recording, so no captured launch ever points at a
    buffer a later call could replace."""
    need = _native.tokenwise_workspace_bytes(m, n, k, w_layout, a_layout)
    if need == 0:
        return None
    return torch.empty(need * targets, dtype=torch.uint8, device=device)


def _gemm(activation, a_layout, scale, weight, w_layout, weight_scale, bias, n, k, epilogue, dtype):
    out = torch.empty((activation.shape[0], n), device=activation.device, dtype=dtype)
    ws = _split_workspace(activation.shape[0], n, k, w_layout, a_layout, activation.device)
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


def _kernel_operands(module, weight, bias):
    """(weight, weight_scale, bias, N) as a K-major GEMM launch takes them.
    The kernels read 16 output columns per 16-byte chunk of a K-major row, so
    a layer whose out_features is not a multiple of 16 (the reference takes
    any width, w4a8_triton.py:57-158) runs on copies of its weights, scale
    and bias zero-padded to the next multiple of 16; the caller keeps the
    first out_features columns of the result. The copies are made once per
    version of the buffers and held outside the module's buffers, so state
    dicts and storage counts stay the reference's (buffers that are
    inference tensors have no version counter, so theirs are remade on every
    call)."""
    n = module.out_features
    if n % 16 == 0:
        return weight, module.weight_scale, bias, n
    key = tuple(None if t is None else (t.data_ptr(), _version_of(t)) for t in (weight, module.weight_scale, bias))
    # inference tensors carry no version counter: their copies are remade on every call
    trackable = all(k is None or k[1] is not None for k in key)
    cached = module.__dict__.get("_padded_operands")
    if cached is None or cached[0] != key or not trackable:
        n16 = -(-n // 16) * 16

        def padded(t):
            if t is None:
                return None
            out = t.new_zeros(*t.shape[:-1], n16)
            out[..., :n] = t
            return out

        cached = (key, (padded(weight), padded(module.weight_scale), padded(bias), n16))
        module.__dict__["_padded_operands"] = cached
    return cached[1]


def _first_columns(out, n):
    """out [M, N'] cut to its first n columns (contiguous)."""
    return out if out.shape[1] == n else out[:, :n].contiguous()


# ---------------------------------------------------------------- shared per-row codes
class _Codes(NamedTuple):
    """Per-row codes of one input tensor at one width: what a later sibling
    on the same tensor may reuse while the tensor is unchanged and while the
    same stream capture (or none) is recording."""

    source: torch.Tensor
    version: int | None
    capture: int
    in_features: int
    codes: torch.Tensor
    scale: torch.Tensor


def _version_of(tensor):
    return None if tensor.is_inference() else tensor._version


class SharedA8CacheStats:
    """One forward's sibling-projection cache (w4a8_triton.py:227-237 names
    its fields): at most one input's per-row A8 codes and one input's A4
    codes (``entry`` / ``a4_entry``), reused by the next linears that read
    the very same tensor, unmodified, at the same K; ``hits`` / ``misses``
    count the A8 lookups."""

    __slots__ = ("enabled", "entry", "a4_entry", "hits", "misses")

    def __init__(self, *, enabled: bool = True) -> None:
        self.enabled = enabled
        self.entry = None
        self.a4_entry = None
        self.hits = 0
        self.misses = 0

    def lookup(self, slot, source, flat, in_features):
        held = getattr(self, slot)
        if (not self.enabled or held is None or held.source is not source or held.in_features != in_features
                or held.version != _version_of(source) or held.codes.shape[0] != flat.shape[0]
                or held.capture != _native.capture_id(flat.device)):
            return None
        return held

    def keep(self, slot, source, in_features, codes, scale):
        entry = _Codes(source, _version_of(source), _native.capture_id(codes.device), in_features, codes, scale)
        setattr(self, slot, entry if self.enabled else None)


_SHARED_A8: ContextVar[SharedA8CacheStats | None] = ContextVar("actune_tokenwise_shared_codes", default=None)


def current_shared_a8_cache():
    """The cache of the innermost shared_a8_cache_scope (None outside any)."""
    return _SHARED_A8.get()


def clear_shared_a8_cache() -> None:
    """Forget the codes held for sibling projections (a cache is opened for
    the current context if none is)."""
    state = _SHARED_A8.get()
    if state is None:
        _SHARED_A8.set(SharedA8CacheStats())
        return
    state.entry = state.a4_entry = None


@contextmanager
def shared_a8_cache_scope(*, enabled: bool = True) -> Iterator[SharedA8CacheStats]:
    """A fresh cache for the body (one model forward); its codes are dropped
    on exit."""
    state = SharedA8CacheStats(enabled=enabled)
    token = _SHARED_A8.set(state)
    try:
        yield state
    finally:
        _SHARED_A8.reset(token)


def _quantize_rows_shared(source, flat, *, in_features):
    """Per-row A8 codes of flat, reused from the cache when the previous
    quantization was of the same, unmodified source tensor: the codes depend
    only on the input and K, so q/k/v (or gate/up) share one quantizer launch
    whatever their weights (w4a8_triton.py:270-325)."""
    if not source.is_cuda or flat.shape[-1] != in_features:
        raise ValueError("shared A8 quantization requires a CUDA input with matching K")
    state = _SHARED_A8.get()
    if state is None:
        clear_shared_a8_cache()
        state = _SHARED_A8.get()
    held = state.lookup("entry", source, flat, in_features)
    if held is not None:
        state.hits += 1
        return held.codes, held.scale
    codes, scale = _native.tokenwise_quantize(flat.contiguous(), 8)
    if resident_a8_eligible(flat):
        _count(0, resident_a8_kernels=1)
    elif decode_eligible(flat, k=in_features):
        _count(1, resident_quantization_kernels=1)
    state.misses += 1
    state.keep("entry", source, in_features, codes, scale)
    return codes, scale


def _quantize_a4_shared(source, flat, *, in_features):
    """Per-row A4 codes (wxa4_native.py:123-160), reused inside a scope for
    the same unmodified source tensor."""
    if not source.is_cuda or flat.shape[-1] != in_features:
        raise ValueError("native A4 quantization requires a CUDA input with matching K")
    state = _SHARED_A8.get()
    held = None if state is None else state.lookup("a4_entry", source, flat, in_features)
    if held is not None:
        return held.codes, held.scale
    packed, scale = _native.tokenwise_quantize(flat.contiguous(), 4)
    if state is not None:
        state.keep("a4_entry", source, in_features, packed, scale)
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
        state = _SHARED_A8.get()
        m = flat.shape[0]
        return (self.fused_quantization and 2 <= m <= 8 and flat.dtype in (torch.bfloat16, torch.float16)
                and self.in_features <= _native.tokenwise_fused_max_k(m)
                and (state is None or not state.enabled))

    def _linear(self, value):
        _require_cuda(value, type(self).__name__)
        original_shape = value.shape[:-1]
        flat = value.reshape(-1, self.in_features)
        m = flat.shape[0]
        weight, wscale, bias, n = _kernel_operands(self, getattr(self, self._weight_name), self.bias)
        if self._fuses_rows(flat):
            out = torch.empty((m, n), device=flat.device, dtype=value.dtype)
            scale = torch.empty(m, device=flat.device, dtype=torch.float32)
            ws = _split_workspace(m, n, self.in_features, self._layout, _native.TW_ACT_A8, flat.device)
            _native.tokenwise_linear_x(flat.contiguous(), scale, weight, self._layout, wscale, bias, n,
                                       self.in_features, _native.TW_EPI_A8, out, workspace=ws)
            return _first_columns(out, self.out_features).reshape(*original_shape, self.out_features)
        activation, scale = self._quantize(flat, source=value)
        if self._layout == _native.TW_KMAJOR_W4 and decode_eligible(flat, k=self.in_features, n=self.out_features):
            _count_split_decode(1, self.out_features, self.in_features)
        output = _gemm(activation, _native.TW_ACT_A8, scale, weight, self._layout, wscale, bias, n,
                       self.in_features, _native.TW_EPI_A8, value.dtype)
        return _first_columns(output, self.out_features).reshape(*original_shape, self.out_features)


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


def _selected(module, filter_fn):
    """(parent, attribute, child) for every child the filter selects, in the
    reference's walk order: a selected child is not descended into."""
    for name, child in list(module.named_children()):
        if filter_fn(child, name):
            yield module, name, child
        else:
            yield from _selected(child, filter_fn)


def _replace(module, filter_fn, factory):
    """Build the replacement of every selected child first, then swap them
    in: a layer this backend cannot take (its constructor raises) leaves the
    model untouched instead of half replaced."""
    built = [(parent, name, factory(child)) for parent, name, child in _selected(module, filter_fn)]
    for parent, name, replacement in built:
        setattr(parent, name, replacement)
    return len(built)


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
        output = _gemm(packed, _native.TW_ACT_A4, activation_scale, self.packed_weight, layout,
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
        weight, wscale, bias, n = _kernel_operands(self, self.weight_int8, self.bias if self.bias.numel() else None)
        output = _gemm(packed, _native.TW_ACT_A4, activation_scale, weight, _native.TW_KMAJOR_W8, wscale, bias, n,
                       self.in_features, _native.TW_EPI_A8, value.dtype)
        return _first_columns(output, self.out_features).reshape(*original_shape, self.out_features)


# ---------------------------------------------------------------- exact split-K decode
# longest row a GEMM launch quantizes itself (actune_tokenwise_linear_x, one row)
_FUSED_MAX_K = 16384
# decode graph plans a module keeps (least recently used dropped first)
_PLANS_PER_MODULE = 4


def _decode_layout(residuals):
    """KMAJOR_W4, or KMAJOR_W4R4 when any projection carries a signed R4
    residual (decode_w4a8_triton.py:61-66): its weight code is the int8
    16 q4 + r4 and its epilogue scale ws / 16; a projection without a
    residual in the same launch computes as plain W4 (the reference's mixed
    W4/R4 group, :205-211)."""
    return _native.TW_KMAJOR_W4R4 if any(r is not None for r in residuals) else _native.TW_KMAJOR_W4


def _w4_shape(packed):
    """(N, K) of K-major nibble-pair weights [K/2, N]."""
    return packed.shape[1], packed.shape[0] * 2


def _count_split_decode(groups, n, k, layout=_native.TW_KMAJOR_W4):
    """DecodeStats of one decode of `groups` sibling projections on one row:
    the GEMM launch (a partial kernel) and, when the library splits K for
    this shape, the integer reduce."""
    split = _native.tokenwise_workspace_bytes(1, n, k, layout, _native.TW_ACT_A8) > 0
    kind = dict(split_k_calls=1) if groups == 1 else dict(projection_groups=1, projection_calls_fused=groups)
    _count(1, partial_kernels=1, reduction_kernels=int(split), **kind)


def _caller_workspace(partial, need):
    """The caller's partial-sum buffer as bytes (any dtype; its contents do
    not matter), or None when the call runs unsplit."""
    if not need:
        return None
    raw = partial.reshape(-1).view(torch.uint8)
    if raw.numel() < need:
        raise ValueError(f"partial workspace too small: {need} bytes needed")
    return raw


def launch_decode_group(activation, weights, residuals, activation_scale, scales, biases, outputs, partial, *,
                        splits=None, bn=None):
    """Decode of 1 to 4 sibling projections (K-major W4 weights, each with
    an optional signed R4 residual of the same packing) sharing one
    quantized row, into caller-owned buffers: ONE GEMM launch over every
    projection's column tiles and K splits, then one integer reduce for all
    of them (decode_w4a8_triton.py:150-239 launches the same pair).
    ``splits`` and ``bn`` are accepted for call compatibility: the library
    sizes the split per shape, and results do not depend on it. ``partial``:
    at least len(weights) x actune_tokenwise_workspace_bytes() bytes."""
    layout = _decode_layout(residuals)
    n, k = _w4_shape(weights[0])
    m = activation.numel() // k
    need = len(weights) * _native.tokenwise_workspace_bytes(m, n, k, layout, _native.TW_ACT_A8)
    targets = [(w, s, b, o.view(m, n)) for w, s, b, o in zip(weights, scales, biases, outputs)]
    return _native.tokenwise_linear_multi(targets, layout, n, k, _native.TW_EPI_A8,
                                          activation_scale.reshape(-1), codes=activation.reshape(m, k),
                                          workspace=_caller_workspace(partial, need),
                                          residuals=residuals if layout == _native.TW_KMAJOR_W4R4 else None)


def launch_decode(activation, packed, residual, activation_scale, weight_scale, bias, output, partial, *,
                  config=None):
    """One decode linear into caller-owned buffers (decode_w4a8_triton.py:113-149):
    the one-projection case of launch_decode_group. ``config`` is accepted
    for call compatibility (the split is chosen per shape)."""
    return launch_decode_group(activation, (packed,), (residual,), activation_scale, (weight_scale,), (bias,),
                               (output,), partial)[0]


def decode_linear(activation, packed, residual, activation_scale, weight_scale, bias, output):
    """One split-K decode into `output` with a per-call workspace
    (decode_w4a8_triton.py:312-323); a signed R4 residual goes through the
    multi-target entry point, the one that takes it."""
    layout = _decode_layout((residual,))
    n, k = _w4_shape(packed)
    m = activation.numel() // k
    work = _split_workspace(m, n, k, layout, _native.TW_ACT_A8, activation.device)
    if residual is None:
        _native.tokenwise_linear(activation.reshape(m, k), _native.TW_ACT_A8, activation_scale.reshape(-1), packed,
                                 layout, weight_scale, bias, n, k, _native.TW_EPI_A8, output.view(m, n),
                                 workspace=work)
    else:
        _native.tokenwise_linear_multi([(packed, weight_scale, bias, output.view(m, n))], layout, n, k,
                                       _native.TW_EPI_A8, activation_scale.reshape(-1),
                                       codes=activation.reshape(m, k), workspace=work, residuals=(residual,))
    _count_split_decode(1, n, k, layout)


def _record(issue, device):
    """A hipGraph of the launches `issue` makes: one eager pass on a side
    stream first (it runs every argument check outside the capture), then
    the capture on that stream; the current stream waits for both."""
    side = torch.cuda.Stream(device=device)
    current = torch.cuda.current_stream(device)
    side.wait_stream(current)
    with torch.cuda.stream(side):
        issue()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        issue()
    current.wait_stream(side)
    return graph


class DecodeGraphPlan:
    """A captured decode of 1 to 4 sibling projections of one row (K-major
    W4, each with an optional signed R4 residual). The contract is the
    reference's (decode_w4a8_triton.py:326-425): each run
    copies the row into the plan's staging buffer, replays, and returns the
    outputs [projections, N] as a fresh tensor, so callers never hold
    graph-owned memory. The graph holds two launches: the GEMM over every
    projection's tiles that quantizes the row itself (rows up to 16384
    long; longer rows add the quantizer launch first) and the integer reduce
    for all projections. Runs are serialised by a lock, since they share the
    staging buffers."""

    def __init__(self, value, weights, residuals, scales, biases):
        if not 1 <= len(weights) <= _native.MAX_TARGETS:
            raise ValueError(f"a decode plan takes 1 to {_native.MAX_TARGETS} projections")
        self.weights, self.residuals = tuple(weights), tuple(residuals)
        self.scales, self.biases = tuple(scales), tuple(biases)
        self.n, self.k = _w4_shape(self.weights[0])
        self.groups = len(self.weights)
        self.layout = _decode_layout(self.residuals)
        dev = value.device
        self.quantize_in_gemm = self.k <= _FUSED_MAX_K
        self.input = torch.empty((1, self.k), device=dev, dtype=value.dtype)
        self.activation = None if self.quantize_in_gemm else torch.empty((1, self.k), device=dev, dtype=torch.int8)
        self.scale = torch.empty(1, device=dev, dtype=torch.float32)
        self.output = torch.empty((self.groups, self.n), device=dev, dtype=value.dtype)
        need = self.groups * _native.tokenwise_workspace_bytes(1, self.n, self.k, self.layout, _native.TW_ACT_A8)
        self.partial = torch.empty(need, device=dev, dtype=torch.uint8) if need else None
        self.lock = threading.Lock()
        self.input.copy_(value.reshape(1, self.k))
        self.graph = _record(self._issue, dev)

    def _issue(self):
        targets = [(w, s, b, self.output[i:i + 1])
                   for i, (w, s, b) in enumerate(zip(self.weights, self.scales, self.biases))]
        residuals = self.residuals if self.layout == _native.TW_KMAJOR_W4R4 else None
        if self.quantize_in_gemm:
            _native.tokenwise_linear_multi(targets, self.layout, self.n, self.k, _native.TW_EPI_A8, self.scale,
                                           x=self.input, workspace=self.partial, residuals=residuals)
        else:
            _native.tokenwise_quantize(self.input, 8, self.activation, self.scale)
            _native.tokenwise_linear_multi(targets, self.layout, self.n, self.k, _native.TW_EPI_A8, self.scale,
                                           codes=self.activation, workspace=self.partial, residuals=residuals)

    @property
    def workspace_bytes(self):
        """Device bytes the plan holds outside the graph's own pool."""
        held = (self.input, self.activation, self.scale, self.output, self.partial)
        return sum(t.numel() * t.element_size() for t in held if t is not None)

    def run(self, value):
        with self.lock:
            self.input.copy_(value.reshape(1, self.k))
            self.graph.replay()
            result = self.output.clone()
        separate = int(not self.quantize_in_gemm)
        _count(1, graph_replays=1, graph_quantization_kernels=separate, resident_quantization_kernels=separate)
        _count_split_decode(self.groups, self.n, self.k, self.layout)
        return result


def graph_plan_key(value, weights, residuals, scales, biases):
    """What a captured plan depends on: the device and stream it replays on,
    the row dtype of its staging buffer, and the storage every captured
    launch reads (the graph holds addresses, so a weight written in place is
    still read correctly, while a weight moved to new storage needs a new
    plan)."""
    storage = tuple(None if t is None else t.data_ptr() for t in (*weights, *residuals, *scales, *biases))
    return (value.device, torch.cuda.current_stream(value.device).cuda_stream, value.dtype, storage)


def graph_decode_linear(owner, value, packed, residual, scale, bias):
    """Decode of one row through the owner's plan for this key, captured on
    first use; the owner keeps its most recently used plans
    (decode_w4a8_triton.py:441-455)."""
    plans = owner.__dict__.setdefault("_decode_graph_plans", OrderedDict())
    key = graph_plan_key(value, (packed,), (residual,), (scale,), (bias,))
    plan = plans.get(key)
    if plan is None:
        plan = DecodeGraphPlan(value, (packed,), (residual,), (scale,), (bias,))
        plans[key] = plan
        while len(plans) > _PLANS_PER_MODULE:
            plans.popitem(last=False)
    else:
        plans.move_to_end(key)
    return plan.run(value).reshape(*value.shape[:-1], packed.shape[1])


def decode_workspace_summary(module):
    """Plans and explicit device bytes of the decode graph plans held by
    `module` and its children, under the reference's keys
    (decode_w4a8_triton.py:458-480). This backend keeps no MLP graph plans:
    those two entries are 0."""
    plans = {id(plan): plan for child in module.modules()
             for plan in child.__dict__.get("_decode_graph_plans", {}).values()}
    return {"decode_graph_plan_count": len(plans), "mlp_graph_plan_count": 0, "mlp_graph_input_output_bytes": 0,
            "decode_graph_explicit_workspace_bytes": sum(plan.workspace_bytes for plan in plans.values())}
