"""GPU tests of the Python module surface on the HIP path.

The modules (GroupedLinear, GroupedPaddedLinear, ResidentLinear, install_bank,
GraphReplay, the bit-exact tuner and sibling launches) are checked against the
CPU oracle (bit-exact bf16 in the library's canonical order) and against their
own eager execution. Shapes follow the reference's module tests
(tests/test_kernels.py:28-49, tests/test_method.py:92-124) and the
Gemma-300M-shaped action expert: width 1024, MLP 1024->4096->1024, 50-token
action chunks, q00/q01/q11/q10 switching under graph replay.
"""
import numpy as np
import pytest
import torch

from actune_amd import _native
from actune_amd.graph import GraphReplay
from actune_amd.kernels import tuning
from actune_amd.kernels.grouped import GroupedLinear, GroupedPaddedLinear, grouped_sibling_forward
from actune_amd.layers import ResidentLinear, install_bank, tensor_storage_bytes
from actune_amd.precision import CONFIGURATIONS, SharedBank, precision_profile
from oracle import oracle as O
from tests.helpers import PAIRS, bits, canonical_bounds, dtype_name, oracle_activation, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _linear(k, n, bias, seed, dtype=torch.bfloat16):
    _, w, b = seeded_inputs(1, k, n, seed=seed, dtype=dtype, bias=bias)
    lin = torch.nn.Linear(k, n, bias=bias, dtype=dtype)
    with torch.no_grad():
        lin.weight.copy_(w)
        if bias:
            lin.bias.copy_(b)
    return lin


def _oracle_module(backend, x_flat, input_scale=None):
    """Oracle output of one GroupedLinear on x_flat [M, K] (cpu)."""
    k = backend.in_features
    wc = O.unpack_rows(backend.packed_weight.cpu().numpy(), backend.w, k)
    ws = backend.weight_scale.cpu().numpy()
    bias = None if backend.bias is None else backend.bias.float().cpu().numpy()
    _, a_scales, a_codes = oracle_activation(x_flat, backend.a, input_scale)
    want = O.linear(a_codes, a_scales, wc, ws, bias, bounds=canonical_bounds(k // 64))
    return O.round_out(want, dtype_name(x_flat.dtype))


# ---------------------------------------------------------------- modules
@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("lead", [(1,), (2, 3), (4, 16)])
def test_grouped_linear_forward_matches_oracle(W, A, lead):
    k, n = 320, 72
    lin = _linear(k, n, True, seed=W * 3 + A)
    mod = GroupedLinear(lin, W, A, None).to(DEV)
    assert mod.bias.dtype == (torch.float32 if A == 4 else torch.bfloat16)
    g = torch.Generator().manual_seed(len(lead))
    x = torch.randn(*lead, k, generator=g).to(torch.bfloat16)
    out = mod(x.to(DEV))
    assert out.shape == (*lead, n) and out.dtype == torch.bfloat16
    want = _oracle_module(mod, x.reshape(-1, k))
    np.testing.assert_array_equal(bits(out.reshape(-1, n)), want)


def _torch_gpu_codes(v, W, A, ratio):
    """The weight codebook formulas of quantizers.py:23-94 evaluated inline by
    torch on the GPU (tensor / Python scalar is a reciprocal multiply there)."""
    amax = v.abs().amax(dim=1).clamp_min(1e-8)
    if ratio is not None and not (W == 8 and A != 4):
        amax = amax * ratio
    if W == 2:
        return (v / amax[:, None]).round().clamp(-2, 1).to(torch.int8), amax
    if W == 4 or A == 4:
        s4 = amax / 7.0
        q4 = (v / s4[:, None]).round().clamp(-8, 7).to(torch.int8)
        if W == 4:
            return q4, s4
        base = q4.to(torch.int16)
        res = (16.0 * (v / s4[:, None] - q4.float())).round().clamp(-8, 7).to(torch.int16)
        res = torch.minimum(torch.maximum(res, (-128 - 16 * base).clamp(min=-8)), (127 - 16 * base).clamp(max=7))
        return (16 * base + res).to(torch.int8), s4 / 16.0
    s = v.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    return (v / s[:, None]).round().clamp(-128, 127).to(torch.int8), s


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("ratio_kind", ["none", "scalar", "rows"])
def test_cuda_built_codes_follow_the_layer_device(W, A, ratio_kind):
    """grouped.py:120 computes weight_codes on the layer's device. A
    GroupedLinear built from a CUDA-resident layer therefore holds the codes
    torch-GPU computes (amax / 7.0 and / 127.0 as reciprocal multiplies,
    quantizers.py:38, 93): its packed_weight and weight_scale equal the
    oracle with gpu_division=True and the formulas evaluated inline by torch
    on the GPU, bit for bit. The same layer built on the CPU equals the IEEE
    oracle."""
    k, n = 512, 96
    lin = _linear(k, n, False, seed=40 + W * 3 + A)
    w_np = lin.weight.detach().float().numpy()
    ratio = {"none": None, "scalar": 0.9, "rows": torch.linspace(0.7, 1.0, n)}[ratio_kind]
    ratio_np = None if ratio is None else (ratio if isinstance(ratio, float) else ratio.numpy())
    cuda_lin = _linear(k, n, False, seed=40 + W * 3 + A).to(DEV)
    ratio_dev = ratio.to(DEV) if isinstance(ratio, torch.Tensor) else ratio
    mod = GroupedLinear(cuda_lin, W, A, ratio_dev)
    assert mod.packed_weight.is_cuda
    want_c, want_s = O.weight_codes(w_np, W, A, ratio_np, gpu_division=True)
    np.testing.assert_array_equal(mod.packed_weight.cpu().numpy(), O.pack_rows(want_c, W))
    np.testing.assert_array_equal(mod.weight_scale.cpu().numpy(), want_s)
    inline_c, inline_s = _torch_gpu_codes(cuda_lin.weight.detach().float(), W, A, ratio_dev)
    assert torch.equal(mod.weight_scale, inline_s)
    np.testing.assert_array_equal(O.unpack_rows(mod.packed_weight.cpu().numpy(), W, k), inline_c.cpu().numpy())
    host = GroupedLinear(lin, W, A, ratio)
    ieee_c, ieee_s = O.weight_codes(w_np, W, A, ratio_np)
    np.testing.assert_array_equal(host.packed_weight.numpy(), O.pack_rows(ieee_c, W))
    np.testing.assert_array_equal(host.weight_scale.numpy(), ieee_s)
    if W != 2:  # the two semantics really differ here (W2 divides by no constant)
        assert not np.array_equal(want_s, ieee_s)


def test_install_bank_on_cuda_model_uses_gpu_codes():
    """install_bank on a CUDA-resident model: every backend of every target
    holds the gpu_division codes of its (channel-scaled) weight."""
    model, bank, _ = _install(scales=True)
    source = Expert(0).to(DEV)
    for name in EXPERT:
        res = getattr(model, name)
        src = getattr(source, name).weight.detach()
        if res.input_scale is not None:
            src = src * res.input_scale[None, :]
        for mode, backend in res.backends.items():
            W, A = int(mode[1]), int(mode[3])
            c, s = O.weight_codes(src.float().cpu().numpy(), W, A, gpu_division=True)
            np.testing.assert_array_equal(backend.packed_weight.cpu().numpy(), O.pack_rows(c, W), err_msg=mode)
            np.testing.assert_array_equal(backend.weight_scale.cpu().numpy(), s, err_msg=mode)


def test_offset_views_compute_like_aligned_inputs():
    """A contiguous view at a 2-byte offset (x[:, 1:] of a [1, K + 1]
    tensor) is not 16-byte aligned: the group-64 and tokenwise modules copy
    it and compute what they compute for the same values aligned, as the
    reference's forward (grouped.py:129, .contiguous() keeps the view)
    computes any contiguous input."""
    from actune_amd.kernels import tokenwise as T
    k, n = 512, 64
    lin = _linear(k, n, False, seed=77)
    base = torch.randn(1, k + 1, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    view = base[:, 1:]
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    aligned = view.clone()
    for W, A in ((4, 8), (2, 4), (8, 2)):
        mod = GroupedLinear(lin, W, A, None).to(DEV)
        assert torch.equal(mod(view), mod(aligned))
    scale = torch.linspace(0.5, 2.0, k + 1).to(torch.bfloat16).to(DEV)[1:]
    r = ResidentLinear(lin, {q: "w4a8" for q in CONFIGURATIONS}, {"w4a8": None}, scale.cpu().clone()).to(DEV)
    assert torch.equal(r(view), r(aligned))
    tw = T.W4A8TritonLinear(lin.to(DEV))
    with T.decode_optimization_scope(enabled=False):
        assert torch.equal(tw(view), tw(aligned))
    assert torch.equal(tw(view), tw(aligned))  # the decode graph plan copies the row in


def test_grouped_linear_rejects_host_input():
    mod = GroupedLinear(_linear(64, 16, False, 1), 4, 8, None).to(DEV)
    with pytest.raises(ValueError, match="requires CUDA"):
        mod(torch.zeros(1, 64, dtype=torch.bfloat16))


def test_padded_linear_dispatch_on_gpu():
    """K = 100 pads to 128 with zero weight columns; each profile runs its own
    backend; counters count logical input elements."""
    lin = _linear(100, 40, True, seed=5)
    assign = {"q00": "w2a4", "q01": "w4a2", "q11": "w4a8", "q10": "w8a8"}
    clips = {"w2a4": None, "w4a2": 0.9, "w4a8": None, "w8a8": None}
    p = GroupedPaddedLinear(lin, assign, "q11", clips).to(DEV)
    x = torch.randn(7, 100, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    xp = torch.nn.functional.pad(x, (0, 28))
    for q in (None, *CONFIGURATIONS):
        mode = assign[q or "q11"]
        if q is None:
            out = p(x.to(DEV))
        else:
            with precision_profile(q):
                out = p(x.to(DEV))
        np.testing.assert_array_equal(bits(out), _oracle_module(p.backends[mode], xp), err_msg=str(q))
    assert p.calls == 5 and p.input_elements == 5 * 700


@pytest.mark.parametrize("m", [1, 3, 4, 5, 50])
@pytest.mark.parametrize("A", [2, 4, 8])
def test_resident_linear_fused_scale_equals_torch_division(m, A):
    """layers.py:41-42: forward quantizes x / input_scale rounded to x's
    dtype. The fused quantizer (M <= 4 inside the GEMM, standalone above)
    must equal quantizing torch's own division, and the oracle."""
    k, n = 256, 48
    lin = _linear(k, n, False, seed=m + A)
    scale = torch.linspace(0.25, 4.0, k).to(torch.bfloat16)
    r = ResidentLinear(lin, {q: f"w4a{A}" for q in CONFIGURATIONS}, {f"w4a{A}": None}, scale).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    out = r(x.to(DEV))
    divided = (x.to(DEV) / scale.to(DEV)).contiguous()
    plain = r.backends[f"w4a{A}"](divided)
    assert torch.equal(out, plain)
    np.testing.assert_array_equal(bits(out), _oracle_module(r.backends[f"w4a{A}"], x, scale))


def test_resident_linear_float_input_with_bf16_scale():
    """x in fp32 with a bf16 channel scale: the module divides in torch
    (fp32 result) and the fp32 quantizer path runs."""
    k, n = 128, 32
    lin = _linear(k, n, False, seed=2)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    r = ResidentLinear(lin, {q: "w8a8" for q in CONFIGURATIONS}, {"w8a8": None}, scale).to(DEV)
    x = torch.randn(3, k, generator=torch.Generator().manual_seed(3))
    out = r(x.to(DEV))
    assert out.dtype == torch.float32
    divided = (x.to(DEV) / scale.to(DEV)).cpu()  # the module's own torch division
    np.testing.assert_array_equal(bits(out), _oracle_module(r.backends["w8a8"], divided))


# ---------------------------------------------------------------- the expert bank
EXPERT = {  # Gemma-300M-shaped action expert, one block
    "q": (1024, 1024, True), "k": (256, 1024, True), "v": (256, 1024, True), "o": (1024, 1024, False),
    "gate": (4096, 1024, False), "up": (4096, 1024, False), "down": (1024, 4096, False),
}
FIXED = {"q": "w4a4", "k": "w8a4", "v": "w4a4", "o": "w2a4", "down": "w4a4"}
SWITCH = {"q00": ("w4a4", "w4a4"), "q01": ("w4a4", "w4a2"), "q11": ("w2a4", "w4a2"), "q10": ("w2a4", "w4a4")}


class Expert(torch.nn.Module):
    def __init__(self, seed=0):
        super().__init__()
        for i, (name, (n, k, bias)) in enumerate(EXPERT.items()):
            setattr(self, name, _linear(k, n, bias, seed=seed * 100 + i))

    def forward(self, x, fused_siblings=False):
        if fused_siblings:
            k, v = grouped_sibling_forward(x, [self.k, self.v])
            gate, up = grouped_sibling_forward(x, [self.gate, self.up])
        else:
            k, v = self.k(x), self.v(x)
            gate, up = self.gate(x), self.up(x)
        q = self.q(x)
        h = x + self.o(q * 0.5)
        h = h + self.down(torch.nn.functional.silu(gate) * up)
        return h, k, v


def _version_bytes(n, k, bias, mode):
    w, a = int(mode[1]), int(mode[3])
    return n * k * w // 8 + 4 * n + (0 if not bias else (4 * n if a == 4 else 2 * n))


def expert_bank(limit=1 << 30):
    configs = {}
    for q, (g, u) in SWITCH.items():
        configs[q] = dict(FIXED, gate=g, up=u)
    modes = [f"w{w}a{a}" for w in (2, 4, 8) for a in (2, 4, 8)]
    sizes = {name: {m: _version_bytes(n, k, b, m) for m in modes} for name, (n, k, b) in EXPERT.items()}
    return SharedBank(configurations=configs, shapes={n: [s[0], s[1]] for n, s in EXPERT.items()},
                      activation_elements={n: 50 * s[1] for n, s in EXPERT.items()},
                      shape_groups=[["q", "k", "v", "gate", "up"], ["o"], ["down"]],
                      version_bytes=sizes, budget="w4a4", storage_limit=limit)


def _install(tune=False, scales=False, seed=0):
    model = Expert(seed).to(DEV)
    bank = expert_bank()
    clips = {n: {m: None for m in {c[n] for c in bank.configurations.values()}} for n in bank.shapes}
    channel = None
    if scales:
        channel = {n: torch.linspace(0.5, 2.0, EXPERT[n][1]).to(torch.bfloat16) for n in ("q", "gate", "up")}
    runtime = install_bank(model, bank, clips, channel_scales=channel, tune=tune)
    return model, bank, runtime


def test_install_bank_holds_w2_w4_w8_and_switches():
    model, bank, runtime = _install()
    assert sorted(model.gate.backends) == ["w2a4", "w4a4"] and sorted(model.up.backends) == ["w4a2", "w4a4"]
    assert list(model.k.backends) == ["w8a4"] and list(model.o.backends) == ["w2a4"]
    resident = sum(tensor_storage_bytes(getattr(model, n)) for n in EXPERT)
    assert resident == bank.resident_bytes()
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    xd = x.to(DEV)
    for q in CONFIGURATIONS:
        runtime.before()
        with precision_profile(q):
            h, kk, vv = model(xd)
        metrics = runtime.audit(q)
        assert metrics["weight_bits"] <= 4 and metrics["activation_bits"] <= 4
        g_mode, u_mode = SWITCH[q]
        np.testing.assert_array_equal(bits(kk), _oracle_module(model.k.backends["w8a4"], x))
        gate = model.gate.backends[g_mode](xd)
        up = model.up.backends[u_mode](xd)
        np.testing.assert_array_equal(bits(gate), _oracle_module(model.gate.backends[g_mode], x), err_msg=q)
        np.testing.assert_array_equal(bits(up), _oracle_module(model.up.backends[u_mode], x), err_msg=q)


def _denoise(step, x, profiles, model, fused=False):
    """10 flow-matching steps: x <- x + dt * h(x) under a seeded per-call
    precision schedule, with eager work between the calls."""
    trace = []
    for i, q in enumerate(profiles):
        with precision_profile(q):
            h, kk, vv = step(x, fused)
        h = h.clone()
        trace.append((h, kk.clone(), vv.clone()))
        x = (x.float() + 0.1 * h.float()).to(torch.bfloat16)
    return x, trace


def _schedule(seed=1234, steps=10):
    g = np.random.default_rng(seed)
    return [CONFIGURATIONS[i] for i in g.integers(0, 4, steps)]


@pytest.mark.parametrize("fused,shared", [(False, False), (True, False), (False, True)])
def test_graph_replay_precision_schedule_matches_eager(fused, shared):
    """C5: 10 denoise steps over a 50-token chunk with q00/q01/q11/q10
    switching from a seeded schedule. Graph replays (one graph per active
    configuration) equal eager execution bit for bit, every replay, with eager
    work and synchronisations in between; counters match eager counts."""
    model, bank, runtime = _install()
    profiles = _schedule()
    assert len(set(profiles)) >= 3
    x0 = torch.randn(50, 1024, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(DEV)

    runtime.before()
    x_eager, eager = _denoise(model, x0, profiles, model, fused)
    eager_counts = {n: (m.calls, m.input_elements) for n, m in runtime.modules.items()}

    replay = GraphReplay(model, runtime.modules, shared_a8=shared)
    replay.enabled = True
    runtime.before()
    x_graph, graphed = _denoise(replay, x0, profiles, model, fused)
    torch.cuda.synchronize()
    assert len(replay.graphs) == len(set(profiles)) and replay.fallbacks == 0
    assert replay.replays == len(profiles)
    for i, (a, b) in enumerate(zip(eager, graphed)):
        for t_e, t_g in zip(a, b):
            assert torch.equal(t_e, t_g), (i, profiles[i])
    assert torch.equal(x_eager, x_graph)
    assert {n: (m.calls, m.input_elements) for n, m in runtime.modules.items()} == eager_counts
    if shared:
        # x is read by k, v, gate, up and q; o's and down's inputs by one linear each
        plans = list(replay.sharing_plans.values())
        assert len(plans) == len(set(profiles))
        assert all(len(p) == 7 and p[5:] == (False, False) and p[0] and p[1] for p in plans), plans
    for q in set(profiles):
        per_call = {n: 50 * EXPERT[n][1] for n in EXPERT}
        bank.check_request(q, per_call)


def test_shared_activation_scope_quantizes_once_per_width():
    """q/k/v/gate/up read the same x at M=50 (the GEMMs take the quantizer's
    codes): inside shared_activation_scope the A4 linears share one
    quantization (and an A2 sibling gets its own); outputs are bit-identical
    to the unshared forward."""
    from actune_amd.kernels.grouped import shared_activation_scope
    model, _, runtime = _install()
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    for q, (want_miss, want_hit) in {"q00": (3, 4), "q01": (4, 3)}.items():
        with precision_profile(q):
            plain = model(x)
            with shared_activation_scope() as state:
                shared = model(x)
        assert (state.misses, state.hits) == (want_miss, want_hit), (q, state.misses, state.hits)
        assert all(torch.equal(a, b) for a, b in zip(plain, shared))


def test_shared_activation_scope_drops_codes_of_mutated_or_older_inputs():
    """An input written in place between two linears (x.add_(), as a flow
    step's x += dt * v does) is quantized again, and the scope keeps the
    codes of one input only: a linear on another tensor in between drops
    them. Every output equals the unshared module on the same values."""
    from actune_amd.kernels.grouped import shared_activation_scope
    lin_a, lin_b = _linear(1024, 256, False, seed=61), _linear(1024, 128, False, seed=62)
    a = GroupedLinear(lin_a, 4, 4, None).to(DEV)
    b = GroupedLinear(lin_b, 8, 4, None).to(DEV)
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(DEV)
    other = torch.randn(50, 1024, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    x0 = x.clone()
    with shared_activation_scope() as state:
        y1 = a(x)
        x.add_(0.5)
        y2 = b(x)
        y3 = a(other)
        y4 = b(x)
        y5 = a(x)
    assert (state.misses, state.hits) == (4, 1), (state.misses, state.hits)
    assert len(state.entries) == 1
    assert torch.equal(y1, a(x0)) and torch.equal(y2, b(x)) and torch.equal(y3, a(other))
    assert torch.equal(y4, b(x)) and torch.equal(y5, a(x))


def test_graph_replay_limit_falls_back_to_eager():
    model, _, runtime = _install()
    replay = GraphReplay(model, runtime.modules, max_graphs=2)
    replay.enabled = True
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    outs = {}
    for q in CONFIGURATIONS + CONFIGURATIONS:
        with precision_profile(q):
            got = replay(x)[0].clone()
            want = model(x)[0]
        assert torch.equal(got, want), q
        outs.setdefault(q, got)
    assert len(replay.graphs) == 2 and replay.fallbacks == 4 and replay.replays == 4
    assert not torch.equal(outs["q00"], outs["q11"])  # the profiles really differ


def test_graph_replay_shared_a8_scope():
    """shared_a8=True binds the tokenwise shared-activation cache to each call
    (graph.py:18-42): inside the function the cache scope is enabled, and
    the replayed output of tokenwise siblings equals eager."""
    from actune_amd.kernels import tokenwise as T
    seen = []

    def fn(x):
        seen.append(T.current_shared_a8_cache().enabled)
        return x * 2

    for flag in (False, True):
        seen.clear()
        with GraphReplay(fn, {}, shared_a8=flag).scope():
            fn(torch.ones(2))
        assert seen == [flag]


def test_channel_scaled_bank_matches_eager_under_replay():
    model, _, runtime = _install(scales=True)
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    replay = GraphReplay(model, runtime.modules)
    replay.enabled = True
    for q in CONFIGURATIONS:
        with precision_profile(q):
            want = model(x)
            for _ in range(3):
                got = replay(x)
                torch.cuda.synchronize()
                assert all(torch.equal(a, b) for a, b in zip(want, got)), q
    # the folded scale really is used: q's input is x / scale
    scale = model.q.input_scale
    backend = model.q.backends["w4a4"]
    np.testing.assert_array_equal(bits(model.q(x)), _oracle_module(backend, x.cpu(), scale.cpu()))


# ---------------------------------------------------------------- tuner and siblings
def test_tuned_bank_is_bit_identical_to_untuned():
    tuning.TUNINGS.clear()
    tuned, _, _ = _install(tune=True)
    plain, _, _ = _install(tune=False)
    for m in (1, 8, 50, 300):
        x = torch.randn(m, 1024, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(DEV)
        for q in CONFIGURATIONS:
            with precision_profile(q):
                a, b = tuned(x), plain(x)
            assert all(torch.equal(s, t) for s, t in zip(a, b)), (m, q)
    assert tuning.TUNINGS
    for key, entry in tuning.TUNINGS.items():
        assert all(c["exact"] for c in entry["candidates"]), key
        assert _native.config_valid(entry["selected"], key[3])


def test_tuner_refuses_untuned_signature_in_capture():
    tuning.TUNINGS.clear()
    backend = GroupedLinear(_linear(128, 32, False, 3), 4, 8, None).to(DEV)
    x = torch.randn(2, 128).to(torch.bfloat16).to(DEV)
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="warmed before graph capture"):
        with torch.cuda.graph(graph):
            tuning.grouped_forward(backend, x)
    torch.cuda.synchronize()
    assert not tuning.TUNINGS


@pytest.mark.parametrize("m", [1, 4, 9, 50])
def test_sibling_forward_equals_separate_calls(m):
    model, _, runtime = _install()
    x = torch.randn(m, 1024, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(DEV)
    for q in CONFIGURATIONS:
        with precision_profile(q):
            runtime.before()
            sep = [model.k(x), model.v(x), model.gate(x), model.up(x), model.q(x)]
            sep_counts = {n: (mod.calls, mod.input_elements) for n, mod in runtime.modules.items()}
            runtime.before()
            kv = grouped_sibling_forward(x, [model.k, model.v])  # w8a4 + w4a4: one launch over both widths
            gu = grouped_sibling_forward(x, [model.gate, model.up])  # fused when (W, A) agree
            qq = grouped_sibling_forward(x, [model.q])
            counts = {n: (mod.calls, mod.input_elements) for n, mod in runtime.modules.items()}
        assert all(torch.equal(a, b) for a, b in zip(sep, kv + gu + qq)), q
        assert counts == sep_counts


def test_reuse_mlp_temporary_with_grouped_projections():
    """A GemmaMLP whose projections are GroupedPaddedLinear: the patched
    forward (gate/up as siblings, gate buffer reused for the product) equals
    the unpatched forward bit for bit, for matching and different gate/up
    versions, and under graph replay with the shared activation cache."""
    from transformers import GemmaConfig
    from transformers.models.gemma.modeling_gemma import GemmaMLP
    from actune_amd.kernels.grouped import reuse_mlp_temporary
    cfg = GemmaConfig(hidden_size=1024, intermediate_size=4096, hidden_activation="gelu_pytorch_tanh")
    mlp = GemmaMLP(cfg).to(device=DEV, dtype=torch.bfloat16)
    same = {q: "w4a4" for q in CONFIGURATIONS}
    mixed = {"q00": "w4a4", "q01": "w2a4", "q11": "w2a4", "q10": "w4a4"}
    clips = {m: None for m in ("w4a4", "w2a4")}
    mlp.gate_proj = GroupedPaddedLinear(mlp.gate_proj, mixed, "q11", clips)
    mlp.up_proj = GroupedPaddedLinear(mlp.up_proj, same, "q11", clips)
    mlp.down_proj = GroupedPaddedLinear(mlp.down_proj, same, "q11", clips)
    x = torch.randn(50, 1024, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        want = {q: _run_profile(mlp, x, q) for q in CONFIGURATIONS}
        assert reuse_mlp_temporary(mlp) == 1
        for q in CONFIGURATIONS:
            assert torch.equal(_run_profile(mlp, x, q), want[q]), q
        replay = GraphReplay(mlp, {"gate": mlp.gate_proj, "up": mlp.up_proj, "down": mlp.down_proj},
                             shared_a8=True)
        replay.enabled = True
        for q in CONFIGURATIONS + CONFIGURATIONS:
            with precision_profile(q):
                assert torch.equal(replay(x), want[q]), q


def _run_profile(module, x, q):
    with precision_profile(q):
        return module(x).clone()


# ---------------------------------------------------------------- C4: Gemma-2B-shaped W4A4 bank
GEMMA = {"q": (2048, 2048), "k": (256, 2048), "v": (256, 2048), "o": (2048, 2048),
         "gate": (16384, 2048), "up": (16384, 2048), "down": (2048, 16384)}
# fixed versions, and the two binary switchable matrices (q, gate) that move
# between W4A4 and W4A8; the A2 layers of the [M, 2048] shape group keep its
# element-weighted activation bits at 4 when both run at A8
GEMMA_FIXED = {"k": "w4a2", "v": "w4a2", "o": "w4a2", "up": "w4a2", "down": "w4a4"}
GEMMA_SWITCH = {"q00": ("w4a4", "w4a4"), "q01": ("w4a4", "w4a8"), "q11": ("w4a8", "w4a8"),
                "q10": ("w4a8", "w4a4")}


class GemmaBlock(torch.nn.Module):
    def __init__(self, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        for name, (n, k) in GEMMA.items():
            lin = torch.nn.Linear(k, n, bias=False, dtype=torch.bfloat16)
            with torch.no_grad():
                lin.weight.copy_((torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16))
            setattr(self, name, lin.to(DEV))

    def forward(self, x):
        q, k, v = self.q(x), self.k(x), self.v(x)
        h = x + self.o(q)
        return h + self.down(torch.nn.functional.silu(self.gate(h)) * self.up(h)), k, v


def gemma_bank():
    configs = {q: dict(GEMMA_FIXED, q=qm, gate=gm) for q, (qm, gm) in GEMMA_SWITCH.items()}
    modes = [f"w{w}a{a}" for w in (2, 4, 8) for a in (2, 4, 8)]
    sizes = {name: {m: n * k * int(m[1]) // 8 + 4 * n for m in modes} for name, (n, k) in GEMMA.items()}
    return SharedBank(configurations=configs, shapes={n: list(s) for n, s in GEMMA.items()},
                      activation_elements={n: 256 * s[1] for n, s in GEMMA.items()},
                      shape_groups=[["q", "k", "v", "o", "gate", "up"], ["down"]], version_bytes=sizes,
                      budget="w4a4", storage_limit=1 << 30)


@pytest.mark.parametrize("m", [256, 1])
def test_gemma_2b_w4a4_bank_against_oracle(m):
    """C4: a Gemma-2B-shaped block installed as a W4A4 shared bank whose two
    binary switchable matrices (q, gate) run W4A8 in three of the four
    configurations (balanced by A2 layers, precision.py:54-62). Under each
    configuration every linear equals the oracle on 64 sampled columns, the
    request passes the bank's audit, and a hipGraph replay equals eager."""
    model = GemmaBlock(4)
    bank = gemma_bank().validate()
    clips = {n: {md: None for md in {c[n] for c in bank.configurations.values()}} for n in bank.shapes}
    runtime = install_bank(model, bank, clips)
    x = torch.randn(m, 2048, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    xd = x.to(DEV)
    rng = np.random.default_rng(m)
    replay = GraphReplay(model, runtime.modules)
    replay.enabled = True
    for q in CONFIGURATIONS:
        runtime.before()
        with precision_profile(q):
            h_eager = model(xd)
            for name, (n, k) in GEMMA.items():
                layer = getattr(model, name)
                backend = layer.active_backend()
                assert f"w{backend.w}a{backend.a}" == bank.configurations[q][name]
                inp = x if k == 2048 else torch.randn(m, k, generator=torch.Generator().manual_seed(n)).to(
                    torch.bfloat16)
                out = layer(inp.to(DEV))
                cols = np.sort(rng.choice(n, size=min(64, n), replace=False))
                wc = O.unpack_rows(backend.packed_weight[torch.from_numpy(cols).to(DEV)].cpu().numpy(), backend.w, k)
                _, a_scales, a_codes = oracle_activation(inp, backend.a)
                want = O.linear(a_codes, a_scales, wc, backend.weight_scale.cpu().numpy()[cols], None,
                                bounds=canonical_bounds(k // 64))
                np.testing.assert_array_equal(bits(out)[:, cols], O.round_out(want, "bf16"), err_msg=f"{q} {name}")
            for _ in range(2):
                h_graph = replay(xd)
                torch.cuda.synchronize()
                assert all(torch.equal(a, b) for a, b in zip(h_eager, h_graph)), q
        metrics = bank.check_request(q, {n: m * GEMMA[n][1] for n in GEMMA})
        assert metrics["weight_bits"] == 4 and max(metrics["group_activation_bits"]) <= 4
