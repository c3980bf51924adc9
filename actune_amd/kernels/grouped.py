"""Group-64 packed W{2,4,8} x A{2,4,8} linear modules on the HIP backend.

Same module surface as actune/kernels/grouped.py:108-167: ``pack_rows``,
``GroupedLinear`` (install-time weight codes + packed rows, forward = group-64
quantize + packed GEMM) and ``GroupedPaddedLinear`` (K padded to 128, one
backend per mode, dispatch on the active precision profile, per-call
counters). Buffers, dtypes and byte counts match the reference exactly, so
``install_bank``'s storage check and state dicts carry over unchanged.

The forward makes one library call, ``actune_grouped_forward``: the group-64
quantizer (with the channel-scale division fused in when a ResidentLinear
passes one) and the packed GEMM, both launched on the current HIP stream.
"""
from __future__ import annotations

import functools

from contextlib import contextmanager
from contextvars import ContextVar
from types import MethodType

import torch

from .. import _native
from ..precision import active_precision_profile
from .quantizers import weight_codes

CONFIG_AUTO = _native.CONFIG_AUTO


class SharedActivationCache:
    """Group-64 codes of the most recent input seen in one scope, keyed by
    the source tensor object (and its version counter), the activation width
    and the channel scale: linears that read the same x at the same width
    one after another (q/k/v, gate/up) then share one quantizer launch,
    whatever their weight widths.

    The scope also records, per call in order, which source it read (by
    order of first appearance), at which width and with which channel
    scale; ``sharing_plan()`` turns that record into one flag per call: True
    when another call of the pass reads the same input at the same width. A
    later pass of the same function (GraphReplay's warm-up and capture) can
    take that plan, so that an input only one linear reads is quantized
    inside that linear's GEMM launch."""

    __slots__ = ("enabled", "entries", "hits", "misses", "plan", "trace", "_sources")

    def __init__(self, *, enabled=True, plan=None):
        self.enabled = enabled
        self.entries = []
        self.hits = 0
        self.misses = 0
        self.plan = plan
        self.trace = []
        self._sources = []

    def record(self, source, width, scale):
        """Index of this call in the pass; notes what it reads."""
        for i, seen in enumerate(self._sources):
            if seen is source:
                break
        else:
            i = len(self._sources)
            self._sources.append(source)
        self.trace.append((i, width, None if scale is None else id(scale)))
        return len(self.trace) - 1

    def sharing_plan(self):
        """Per recorded call: True when another call reads the same input."""
        counts = {}
        for key in self.trace:
            counts[key] = counts.get(key, 0) + 1
        return tuple(counts[key] > 1 for key in self.trace)


# largest M at which a call inside an enabled shared scope still quantizes
# inside its GEMM when its forward would
_SHARED_FUSED_MAX_M = 8

_SHARED_GROUP_STATE: ContextVar[SharedActivationCache | None] = ContextVar("actune_shared_group64_codes",
                                                                           default=None)


@contextmanager
def shared_activation_scope(*, enabled=True, plan=None):
    """Bound the group-64 code cache to one forward (GraphReplay enters it
    with its shared_a8 flag, the reference's switch for shared activation
    quantization, graph.py:18-42). Outside a scope nothing is cached, so a
    tensor reused in place never sees stale codes. ``plan``: the
    sharing_plan() of an earlier pass of the same function."""
    state = SharedActivationCache(enabled=enabled, plan=plan)
    token = _SHARED_GROUP_STATE.set(state)
    try:
        yield state
    finally:
        _SHARED_GROUP_STATE.reset(token)


def _version(tensor):
    """In-place writes bump a tensor's version counter (shared with its
    views); inference tensors have none."""
    return None if tensor.is_inference() else tensor._version


def _shared_codes(state, source, flat, a, input_scale):
    """(packed, scales) of flat at width a from the scope's cache, quantizing
    on a miss. The cache holds the codes of ONE input (the most recent
    source, one entry per width and channel scale): a call on another
    tensor, on the same tensor after an in-place write, or under another
    stream capture (or none) drops them, so codes never outlive the values
    they were computed from, a captured launch never reads codes written
    outside its graph, and at most one input's codes stay alive."""
    stamp = (_version(source), _native.capture_id(flat.device))
    if state.entries and (state.entries[0][0] is not source or state.entries[0][1] != stamp):
        state.entries.clear()
    for _, _, shape, width, scale, packed, scales in state.entries:
        if shape == flat.shape and width == a and scale is input_scale:
            state.hits += 1
            return packed, scales
    packed, scales = _native.quantize_groups(flat, a, input_scale)
    state.misses += 1
    state.entries.append((source, stamp, flat.shape, a, input_scale, packed, scales))
    return packed, scales


def extension():
    """The native op object (reference: the JIT extension, grouped.py:97-105)."""
    return _native.extension()


def pack_rows(q, bits):
    """Pack int8 codes [N, K] into u8 [N, K*bits/8]: code k of a row sits in
    byte k*bits/8 at bit (k % (8/bits))*bits (grouped.py:108-111 layout)."""
    per = 8 // bits
    mask = (1 << bits) - 1
    fields = (q.to(torch.int32) & mask).reshape(q.shape[0], -1, per)
    packed = torch.zeros(fields.shape[:2], dtype=torch.int32, device=q.device)
    for j in range(per):
        packed |= fields[..., j] << (j * bits)
    return packed.to(torch.uint8).contiguous()


class GroupedLinear(torch.nn.Module):
    """One (W, A) version of a linear layer: packed weight codes + per-row
    scale (+ bias), forward through the HIP library."""

    def __init__(self, linear, w, a, ratios):
        super().__init__()
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.w, self.a = w, a
        if self.in_features % 64:
            raise ValueError("Grouped backend requires K divisible by 64")
        if w not in (2, 4, 8) or a not in (2, 4, 8):
            raise ValueError("Unsupported integer width")
        # codes as torch computes them where the layer lives (grouped.py:120
        # runs weight_codes on linear.weight's device): a CUDA layer divides
        # by 7 and 127 through their fp32 reciprocals, a CPU layer exactly
        codes, scale = weight_codes(linear.weight, w, a, clip_ratios=ratios,
                                    gpu_division=linear.weight.is_cuda)
        self.register_buffer("packed_weight", pack_rows(codes, w))
        self.register_buffer("weight_scale", scale.contiguous())
        bias = None
        if linear.bias is not None:
            bias = linear.bias.detach().clone()
            if a == 4:
                bias = bias.float()
        self.register_buffer("bias", bias)
        # kernel configuration id (ACTUNE_CONFIG_AUTO or a tuned id); not a buffer
        self.config = CONFIG_AUTO

    def forward(self, x, input_scale=None, source=None):
        """y = grouped linear of x (optionally x / input_scale, rounded to
        x's dtype, fused into the quantizer). Inside an enabled
        shared_activation_scope, calls whose GEMM takes the quantizer's codes
        reuse the codes of an earlier call on the same source tensor (source
        defaults to x) at the same width and channel scale."""
        if not x.is_cuda:
            raise ValueError("Grouped integer backend requires CUDA")
        flat = x.reshape(-1, self.in_features).contiguous()
        if input_scale is not None and input_scale.dtype != flat.dtype:
            flat = (flat / input_scale).contiguous()
            input_scale = None
            source = flat
        state = _SHARED_GROUP_STATE.get()
        m = flat.shape[0]
        if state is not None and state.enabled and m > 0:
            src = x if source is None else source
            call = state.record(src, self.a, input_scale)
            # Past _SHARED_FUSED_MAX_M tokens the codes are shared even where
            # the forward would quantize inside its GEMM: the in-launch
            # quantization then costs more than a GEMM on shared codes
            # (measured on MI355X at M = 50, 1024x1024: about 1.5 us per
            # linear). Without a plan the linears of a scope are taken to
            # read the same x; with one, an input no other call of the pass
            # reads at this width keeps the in-launch quantization.
            plan = state.plan
            shared = plan[call] if plan is not None and call < len(plan) else True
            if (m > _SHARED_FUSED_MAX_M and shared) or not _native.forward_fuses_quantizer(
                    m, self.out_features, self.in_features, self.w, self.a, flat.dtype, self.config):
                packed, scales = _shared_codes(state, src, flat, self.a, input_scale)
                # an automatic config resolves to the choice for packed codes
                out = _native.grouped_linear(packed, scales, self.packed_weight, self.weight_scale, self.bias,
                                             flat, self.w, self.a, self.config)
                return out.reshape(*x.shape[:-1], self.out_features)
        out = _native.grouped_forward(flat, self.packed_weight, self.weight_scale, self.bias,
                                      self.w, self.a, input_scale=input_scale, config=self.config)
        return out.reshape(*x.shape[:-1], self.out_features)


class GroupedPaddedLinear(torch.nn.Module):
    """Resident set of GroupedLinear versions of one layer; the active
    precision profile picks the version for each call."""

    def __init__(self, linear, assignments, initial, clips):
        super().__init__()
        logical = linear.in_features
        padded = -(-logical // 128) * 128
        if padded != logical:
            linear = _zero_padded(linear, padded)
        self.in_features = logical
        self.out_features = linear.out_features
        self.padding = padded - logical
        self.assignments = dict(assignments)
        self.default_profile = initial
        modes = sorted(set(self.assignments.values()))
        self.backends = torch.nn.ModuleDict(
            {mode: GroupedLinear(linear, int(mode[1]), int(mode[3]), clips[mode]) for mode in modes})
        self.register_buffer("_weight_dtype", torch.empty(0, device=linear.weight.device,
                                                          dtype=linear.weight.dtype))
        self.calls = 0
        self.input_elements = 0

    @property
    def weight(self):
        """Empty tensor of the weight dtype, for callers that sniff .weight.dtype."""
        return self._weight_dtype

    def active_backend(self):
        return self.backends[self.assignments[active_precision_profile() or self.default_profile]]

    def forward(self, x):
        return self._dispatch(x, None)

    def _dispatch(self, x, input_scale):
        self.calls += 1
        self.input_elements += x.numel()
        if not self.padding:
            return self.active_backend()(x, input_scale)
        source = x
        x = torch.nn.functional.pad(x, (0, self.padding))
        if input_scale is not None:
            input_scale = torch.nn.functional.pad(input_scale, (0, self.padding), value=1.0)
        backend = self.active_backend()
        if getattr(backend.forward, "__func__", None) is GroupedLinear.forward:
            # the padded copy is new on every call: key shared codes on the caller's tensor
            return backend(x, input_scale, source=source)
        return backend(x, input_scale)


def _zero_padded(linear, padded):
    """Copy of `linear` with zero weight columns up to `padded` inputs."""
    fc = torch.nn.Linear(padded, linear.out_features, bias=linear.bias is not None,
                         device=linear.weight.device, dtype=linear.weight.dtype)
    with torch.no_grad():
        fc.weight.zero_()
        fc.weight[:, :linear.in_features].copy_(linear.weight)
        if fc.bias is not None:
            fc.bias.copy_(linear.bias)
    return fc


def _gate_kind(act_fn):
    """The gated quantizer's code for an activation whose torch form it
    reproduces (SiLU; GELU with the tanh approximation, Gemma's
    gelu_pytorch_tanh), else None."""
    silu = (torch.nn.functional.silu, torch.nn.SiLU)
    if act_fn is silu[0] or type(act_fn) is silu[1] or type(act_fn).__name__ == "SiLUActivation":
        return _native.ACT_SILU
    if type(act_fn) is torch.nn.GELU and act_fn.approximate == "tanh":
        return _native.ACT_GELU_TANH
    inner = getattr(act_fn, "act", None)  # transformers' GELUTanh holds partial(gelu, approximate="tanh")
    if (type(act_fn).__name__ in ("GELUTanh", "PytorchGELUTanh") and isinstance(inner, functools.partial)
            and inner.func is torch.nn.functional.gelu and inner.keywords == {"approximate": "tanh"}):
        return _native.ACT_GELU_TANH
    return None


def gated_down_forward(down, gate, up, act_fn):
    """down(act_fn(gate) * up) for a gated MLP, the product formed in gate's
    dtype as torch forms it (act_fn(gate), then gate.mul_(up), grouped.py:
    22-25). Where down is a GroupedPaddedLinear (or ResidentLinear) without
    K padding whose active version is a GroupedLinear, and act_fn is one the
    gated quantizer knows, the activation and the product are formed inside
    down's quantizer launch (actune_quantize_gated: one launch in place of
    three) and down runs on its codes; the output is bit-identical to the
    unfused calls and down's calls / input_elements advance as for one call.
    Otherwise the unfused calls run."""
    kind = _gate_kind(act_fn)
    backend = down.active_backend() if isinstance(down, GroupedPaddedLinear) else None
    scale = getattr(down, "input_scale", None)
    fused = (kind is not None and backend is not None and not down.padding and gate.is_cuda
             and getattr(backend.forward, "__func__", None) is GroupedLinear.forward
             and gate.shape == up.shape and gate.dtype == up.dtype and gate.shape[-1] == down.in_features
             and gate.dtype in (torch.bfloat16, torch.float16, torch.float32)
             and (scale is None or scale.dtype == gate.dtype) and gate.numel() > 0)
    if not fused:
        product = act_fn(gate)
        product.mul_(up)
        return down(product)
    down.calls += 1
    down.input_elements += gate.numel()
    flat_gate = gate.reshape(-1, down.in_features).contiguous()
    flat_up = up.reshape(-1, down.in_features).contiguous()
    packed, scales = _native.quantize_gated(flat_gate, flat_up, kind, backend.a, input_scale=scale)
    out = _native.grouped_linear(packed, scales, backend.packed_weight, backend.weight_scale, backend.bias,
                                 flat_gate, backend.w, backend.a, backend.config)
    return out.reshape(*gate.shape[:-1], down.out_features)


def _inference_mlp(self, x):
    """GemmaMLP forward of the reference's patch (grouped.py:18-25): gate/up
    run as sibling projections (one launch when their activation widths
    match, else shared codes inside a shared_activation_scope), and the
    activation times up feeds the down projection through
    gated_down_forward (formed inside down's quantizer where it can be, else
    in the gate buffer as the reference reuses it); bit-identical to the
    unpatched forward."""
    if torch.is_grad_enabled():
        return self._group64_original_forward(x)
    gate_proj, up_proj = self.gate_proj, self.up_proj
    if isinstance(gate_proj, GroupedPaddedLinear) and isinstance(up_proj, GroupedPaddedLinear):
        gate, up = grouped_sibling_forward(x, [gate_proj, up_proj])
    else:
        gate, up = gate_proj(x), up_proj(x)
    return gated_down_forward(self.down_proj, gate, up, self.act_fn)


def reuse_mlp_temporary(model):
    """Patch every transformers GemmaMLP of `model` (once) with
    _inference_mlp; returns the number patched (grouped.py:28-36)."""
    from transformers.models.gemma.modeling_gemma import GemmaMLP
    count = 0
    for module in model.modules():
        if type(module) is GemmaMLP and not hasattr(module, "_group64_original_forward"):
            module._group64_original_forward = module.forward
            module.forward = MethodType(_inference_mlp, module)
            count += 1
    return count


def grouped_sibling_forward(x, modules):
    """Run GroupedPaddedLinear (or ResidentLinear) modules that read the same
    input x — sibling projections such as q/k/v or gate/up — and return their
    outputs in order.

    When every module's active backend has the same A, K, padding, bias
    dtype and input scale, all of them run in one actune_grouped_forward_multi
    call (up to 4 targets): one quantize + GEMM launch, also where their
    weight widths differ (q/k/v of a mixed-precision bank) and the decode
    kernel takes every width; otherwise each module runs on its own. Either
    way the outputs are bit-identical to calling the modules one by one, and each module's calls / input_elements counters
    advance exactly as for a separate call (BankRuntime.audit relies on them).
    """
    modules = list(modules)
    if not modules:
        return []
    backends = [m.active_backend() for m in modules]
    first, fb = modules[0], backends[0]
    scale = getattr(first, "input_scale", None)
    fusable = (
        x.is_cuda and 1 < len(modules) <= _native.MAX_TARGETS
        and all(getattr(b.forward, "__func__", None) is GroupedLinear.forward for b in backends)
        and all(m.in_features == first.in_features and m.padding == first.padding for m in modules)
        and all(b.a == fb.a for b in backends)
        and len({None if b.bias is None else b.bias.dtype for b in backends}) == 1
        and all(getattr(m, "input_scale", None) is scale for m in modules)
        and (scale is None or scale.dtype == x.dtype)
    )
    if not fusable:
        return [m(x) for m in modules]
    for m in modules:
        m.calls += 1
        m.input_elements += x.numel()
    if first.padding:
        x = torch.nn.functional.pad(x, (0, first.padding))
        if scale is not None:
            scale = torch.nn.functional.pad(scale, (0, first.padding), value=1.0)
    flat = x.reshape(-1, fb.in_features).contiguous()
    targets = [(b.packed_weight, b.weight_scale, b.bias, None, b.w) for b in backends]
    outs = _native.grouped_forward_multi(flat, targets, fb.w, fb.a, input_scale=scale, config=fb.config)
    return [o.reshape(*x.shape[:-1], m.out_features) for o, m in zip(outs, modules)]
