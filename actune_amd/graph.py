"""Shape- and precision-keyed HIP graph replay.

Same contract as actune/graph.py:6-95. One hipGraph (torch.cuda.CUDAGraph on
ROCm) is captured per (argument tree, tensor shapes/strides/dtypes/devices,
non-tensor reprs, every layer's active mode), up to ``max_graphs``; beyond
that calls run eagerly and are counted as fallbacks. Capture warms the
function twice on a side stream, records the per-layer ``calls`` /
``input_elements`` seen during capture and restores the live counters;
each replay copies the inputs into the captured static buffers, replays and
adds the recorded counts, so BankRuntime.audit sees the same numbers as
eager execution. The returned output is graph-owned (overwritten by the next
replay of the same graph).

Every launch of the grouped backend goes to the current stream through the
C ABI with no allocation or synchronisation inside, so it captures as is;
per-precision dispatch happens on the host, hence one graph per
configuration.
"""
from __future__ import annotations

from contextlib import contextmanager
from unittest.mock import patch

import torch
from torch.utils import _pytree as pytree

from .precision import active_precision_profile


def _literal(data):
    if isinstance(data, (bool, int, float)):
        return True
    return isinstance(data, (list, tuple)) and all(_literal(x) for x in data)


class GraphReplay:
    def __init__(self, function, layers, *, shared_a8=False, max_graphs=12):
        self.function = function
        self.layers = layers
        self.shared_a8 = shared_a8
        self.max_graphs = max_graphs
        self.graphs = {}
        self.enabled = False
        self.replays = 0
        self.fallbacks = 0
        self.constants = {}
        # per graph key: the group-64 sharing plan its capture followed
        self.sharing_plans = {}

    @contextmanager
    def scope(self, plan=None):
        """Serve small literal GPU constants built inside the function from a
        cache filled during warm-up (a fresh host->device copy cannot be
        captured); each use gets a clone because callers update in place.
        Also bounds the shared activation caches to the call (the tokenwise
        per-row codes, graph.py:18-42, and the group-64 codes), enabled when
        shared_a8 is set; yields the group-64 cache. ``plan``: the group-64
        sharing plan recorded by an earlier pass of the function."""
        make = torch.tensor

        def cached_tensor(data, *args, **kwargs):
            device = kwargs.get("device")
            on_gpu = device is not None and torch.device(device).type == "cuda"
            if not on_gpu or args or kwargs.get("requires_grad", False) or not _literal(data):
                return make(data, *args, **kwargs)
            key = (repr(data), repr(sorted(kwargs.items())))
            if key not in self.constants:
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError("Unwarmed CUDA constant in graph capture")
                self.constants[key] = make(data, **kwargs)
            return self.constants[key].clone()

        from .kernels.grouped import shared_activation_scope
        from .kernels.tokenwise import shared_a8_cache_scope
        with shared_a8_cache_scope(enabled=self.shared_a8), \
                shared_activation_scope(enabled=self.shared_a8, plan=plan) as group_codes, \
                patch.object(torch, "tensor", cached_tensor):
            yield group_codes

    def _key(self, leaves, spec):
        sig = []
        for leaf in leaves:
            if isinstance(leaf, torch.Tensor):
                sig.append((tuple(leaf.shape), tuple(leaf.stride()), str(leaf.dtype), str(leaf.device)))
            else:
                sig.append((type(leaf).__name__, repr(leaf)))
        profile = active_precision_profile()
        modes = tuple(m.assignments[profile or m.default_profile] for m in self.layers.values())
        return (str(spec), tuple(sig), modes)

    def _capture(self, leaves, spec):
        saved = {name: (m.calls, m.input_elements) for name, m in self.layers.items()}
        static = [x.clone() if isinstance(x, torch.Tensor) else x for x in leaves]
        args, kwargs = pytree.tree_unflatten(static, spec)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        # the first warm-up pass records which group-64 inputs several
        # linears share; the second pass and the capture follow that plan
        plan = None
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):
                with self.scope(plan) as group_codes:
                    self.function(*args, **kwargs)
                if plan is None:
                    plan = group_codes.sharing_plan()
        torch.cuda.current_stream().wait_stream(side)
        for m in self.layers.values():
            m.calls = m.input_elements = 0
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph), torch.inference_mode(), self.scope(plan):
            output = self.function(*args, **kwargs)
        self.sharing_plans[self._key(leaves, spec)] = plan
        counts = {name: (m.calls, m.input_elements) for name, m in self.layers.items()}
        for name, m in self.layers.items():
            m.calls, m.input_elements = saved[name]
        return graph, static, output, counts

    def __call__(self, *args, **kwargs):
        if not self.enabled:
            return self.function(*args, **kwargs)
        leaves, spec = pytree.tree_flatten((args, kwargs))
        key = self._key(leaves, spec)
        entry = self.graphs.get(key)
        if entry is None:
            if len(self.graphs) >= self.max_graphs:
                self.fallbacks += 1
                return self.function(*args, **kwargs)
            entry = self.graphs[key] = self._capture(leaves, spec)
        graph, static, output, counts = entry
        for src, dst in zip(leaves, static, strict=True):
            if isinstance(src, torch.Tensor):
                dst.copy_(src)
        graph.replay()
        for name, (calls, elements) in counts.items():
            self.layers[name].calls += calls
            self.layers[name].input_elements += elements
        self.replays += 1
        return output
