"""CPU tests of the Python surface: module buffers and byte counts, install-
time codebooks against the oracle, padding, dispatch, counters, bank rules
and install_bank's checks (the shapes of the reference's own tests,
tests/test_method.py:92-124 and tests/test_kernels.py:28-49)."""
import numpy as np
import pytest
import torch

from actune_amd.kernels import quantizers as Q
from actune_amd.kernels.grouped import GroupedLinear, GroupedPaddedLinear, pack_rows
from actune_amd.layers import BankRuntime, ResidentLinear, install_bank, tensor_storage_bytes
from actune_amd.precision import CONFIGURATIONS, SharedBank, active_precision_profile, pair, precision_profile
from oracle import oracle as O
from tests.helpers import PAIRS, seeded_inputs


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("ratios", [None, 0.9, "rows"])
def test_weight_codes_match_oracle(W, A, ratios):
    _, w, _ = seeded_inputs(1, 256, 40, seed=11 + W * 10 + A)
    if ratios == "rows":
        ratios = torch.linspace(0.7, 1.0, 40)
    codes, scale = Q.weight_codes(w, W, A, clip_ratios=ratios)
    want_c, want_s = O.weight_codes(w.float().numpy(), W, A,
                                    None if ratios is None else np.asarray(ratios, np.float32))
    np.testing.assert_array_equal(codes.numpy(), want_c)
    np.testing.assert_array_equal(scale.numpy(), want_s)


def test_weight_codes_edge_rows():
    w = torch.zeros(4, 128, dtype=torch.bfloat16)
    w[1, 3] = 1e-30  # below the 1e-8 floor
    w[2] = torch.linspace(-3, 3, 128)
    w[3, ::2] = -7.0
    for W, A in PAIRS:
        codes, scale = Q.weight_codes(w, W, A, clip_ratios=0.5)
        want_c, want_s = O.weight_codes(w.float().numpy(), W, A, 0.5)
        np.testing.assert_array_equal(codes.numpy(), want_c)
        np.testing.assert_array_equal(scale.numpy(), want_s)


def test_clip_ratio_messages():
    w = torch.ones(3, 64)
    with pytest.raises(ValueError, match="expected 3"):
        Q.weight_codes(w, 4, 8, clip_ratios=[0.5, 0.5])
    with pytest.raises(ValueError, match="finite"):
        Q.weight_codes(w, 2, 8, clip_ratios=float("inf"))
    with pytest.raises(ValueError, match=r"\(0, 1\]"):
        Q.weight_codes(w, 8, 4, clip_ratios=0.0)
    Q.weight_codes(w, 8, 8, clip_ratios=5.0)  # W8 with A != 4 ignores ratios entirely


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_rows_matches_oracle(bits):
    rng = np.random.default_rng(bits)
    lo = -(1 << (bits - 1))
    codes = rng.integers(lo, -lo, (7, 192)).astype(np.int8)
    np.testing.assert_array_equal(pack_rows(torch.from_numpy(codes), bits).numpy(), O.pack_rows(codes, bits))


@pytest.mark.parametrize("W,A", PAIRS)
def test_grouped_linear_buffers_and_bytes(W, A):
    lin = torch.nn.Linear(128, 48, bias=True, dtype=torch.bfloat16)
    g = GroupedLinear(lin, W, A, None)
    assert [n for n, _ in g.named_buffers()] == ["packed_weight", "weight_scale", "bias"]
    assert g.packed_weight.dtype == torch.uint8 and g.packed_weight.shape == (48, 128 * W // 8)
    assert g.weight_scale.dtype == torch.float32 and g.weight_scale.shape == (48,)
    assert g.bias.dtype == (torch.float32 if A == 4 else torch.bfloat16)
    bias_bytes = 48 * (4 if A == 4 else 2)
    assert tensor_storage_bytes(g) == 48 * 128 * W // 8 + 4 * 48 + bias_bytes
    codes, scale = O.weight_codes(lin.weight.float().detach().numpy(), W, A)
    np.testing.assert_array_equal(g.packed_weight.numpy(), O.pack_rows(codes, W))
    np.testing.assert_array_equal(g.weight_scale.numpy(), scale)
    with pytest.raises(ValueError, match="requires CUDA"):
        g(torch.zeros(1, 128, dtype=torch.bfloat16))


def test_grouped_linear_rejects_bad_shapes():
    with pytest.raises(ValueError, match="divisible by 64"):
        GroupedLinear(torch.nn.Linear(100, 8), 4, 8, None)
    with pytest.raises(ValueError, match="Unsupported integer width"):
        GroupedLinear(torch.nn.Linear(64, 8), 3, 8, None)


def test_padded_linear_pads_dispatches_and_counts():
    lin = torch.nn.Linear(100, 16, bias=False, dtype=torch.bfloat16)
    assign = {"q00": "w2a4", "q01": "w4a4", "q11": "w4a4", "q10": "w8a8"}
    clips = {"w2a4": None, "w4a4": 0.9, "w8a8": None}
    p = GroupedPaddedLinear(lin, assign, "q11", clips)
    assert p.in_features == 100 and p.padding == 28 and p.out_features == 16
    assert sorted(p.backends) == ["w2a4", "w4a4", "w8a8"]
    assert p.weight.dtype == torch.bfloat16 and p.weight.numel() == 0
    # padded weight columns are zero codes
    w4 = p.backends["w4a4"]
    codes = O.unpack_rows(w4.packed_weight.numpy(), 4, 128)
    assert not codes[:, 100:].any()
    seen = []
    for mode, backend in p.backends.items():
        backend.forward = (lambda mode: lambda x, s=None: seen.append((mode, tuple(x.shape))) or x)(mode)
    x = torch.zeros(3, 100, dtype=torch.bfloat16)
    p(x)
    with precision_profile("q00"):
        p(x)
    with precision_profile("q10"):
        p(x)
    assert seen == [("w4a4", (3, 128)), ("w2a4", (3, 128)), ("w8a8", (3, 128))]
    assert p.calls == 3 and p.input_elements == 900


def test_resident_linear_folds_scale():
    lin = torch.nn.Linear(128, 8, bias=False, dtype=torch.bfloat16)
    scale = torch.linspace(0.5, 2.0, 128).to(torch.bfloat16)
    r = ResidentLinear(lin, {q: "w8a8" for q in CONFIGURATIONS}, {"w8a8": None}, scale)
    folded = (lin.weight * scale[None, :]).float().detach().numpy()
    codes, s = O.weight_codes(folded, 8, 8)
    np.testing.assert_array_equal(r.backends["w8a8"].packed_weight.numpy(), O.pack_rows(codes, 8))
    assert r.default_profile == "q11" and r.input_scale.dtype == torch.bfloat16
    for bad in (torch.zeros(128), torch.ones(64), torch.full((128,), float("nan"))):
        with pytest.raises(ValueError, match="channel scale"):
            ResidentLinear(lin, {q: "w8a8" for q in CONFIGURATIONS}, {"w8a8": None}, bad)


def test_precision_profile_does_not_leak():
    assert active_precision_profile() is None
    with precision_profile("q00"):
        with precision_profile("q11"):
            assert active_precision_profile() == "q11"
        assert active_precision_profile() == "q00"
    assert active_precision_profile() is None
    with pytest.raises(ValueError, match="Unknown"):
        with precision_profile("q22"):
            pass
    assert pair("w4a8") == (4, 8)
    for bad in ("w3a8", "w4a", 48, "x4a8"):
        with pytest.raises(ValueError, match="invalid pi05 precision"):
            pair(bad)


def toy_bank(budget="w4a4", limit=10000):
    """8 layers [8, 128]; two binary switchable layers give four configs."""
    names = [str(i) for i in range(8)]
    base = "w4a4" if budget == "w4a4" else "w4a8"
    if budget == "w4a4":
        switch = {"q00": ("w4a4", "w4a4"), "q01": ("w4a4", "w4a2"), "q11": ("w2a4", "w4a2"), "q10": ("w2a4", "w4a4")}
    else:
        switch = {"q00": ("w4a8", "w4a8"), "q01": ("w4a8", "w2a8"), "q11": ("w2a8", "w2a8"), "q10": ("w2a8", "w4a8")}
    configs = {q: {n: base for n in names} for q in CONFIGURATIONS}
    for q, (m0, m1) in switch.items():
        configs[q]["0"], configs[q]["1"] = m0, m1
    modes = [f"w{w}a{a}" for w in (2, 4, 8) for a in (2, 4, 8)]
    sizes = {n: {m: 8 * 128 * int(m[1]) // 8 + 32 for m in modes} for n in names}
    return SharedBank(configurations=configs, shapes={n: [8, 128] for n in names},
                      activation_elements={n: 128 for n in names}, shape_groups=[names],
                      version_bytes=sizes, budget=budget, storage_limit=limit)


def test_shared_bank_rules():
    for budget in ("w4a4", "w4a8"):
        bank = toy_bank(budget).validate()
        full = sum(sum(bank.version_bytes[n][m] for n, m in c.items()) for c in bank.configurations.values())
        assert bank.resident_bytes() < full
        assert len({tuple(c.values()) for c in bank.configurations.values()}) == 4
    bank = toy_bank("w4a8")
    bank.storage_limit = bank.resident_bytes() - 1
    with pytest.raises(ValueError, match="resident"):
        bank.validate()
    with pytest.raises(ValueError, match="target"):
        bank.check_request("q11", {})
    bank = toy_bank()
    bank.configurations["q01"]["2"] = "w8a8"
    with pytest.raises(ValueError, match="two binary switchable"):
        bank.validate()
    bank = toy_bank()
    m = bank.metrics("q11")
    assert m["weight_bits"] == pytest.approx((6 * 4 + 2 + 4) / 8)
    assert m["activation_bits"] == pytest.approx((7 * 4 + 2) / 8)
    bank.configurations["q00"]["5"] = "w8a4"  # (7*4 + 8) / 8 = 4.5 weight bits
    with pytest.raises(ValueError, match="Active weight budget exceeds four bits"):
        bank.check_request("q00")
    bank.configurations["q00"]["5"] = "w2a8"  # (7*4 + 8) / 8 = 4.5 activation bits
    with pytest.raises(ValueError, match="Active activation budget exceeds four bits"):
        bank.check_request("q00")
    w4a8 = toy_bank("w4a8")
    w4a8.configurations["q10"]["4"] = "w4a4"
    with pytest.raises(ValueError, match="A8 on every target"):
        w4a8.check_request("q10")


def _toy_model():
    return torch.nn.Sequential(*[torch.nn.Linear(128, 8, bias=False, dtype=torch.bfloat16) for _ in range(8)])


def test_install_bank_swaps_and_checks_bytes():
    model = _toy_model()
    bank = toy_bank()
    clips = {n: {m: None for m in {c[n] for c in bank.configurations.values()}} for n in bank.shapes}
    runtime = install_bank(model, bank, clips)
    assert isinstance(runtime, BankRuntime)
    assert all(isinstance(model[i], ResidentLinear) for i in range(8))
    assert sorted(model[0].backends) == ["w2a4", "w4a4"] and sorted(model[1].backends) == ["w4a2", "w4a4"]
    for i in range(8):
        model[i].input_elements = 128
    assert runtime.audit("q11")["weight_bits"] <= 4
    runtime.before()
    assert all(model[i].calls == 0 and model[i].input_elements == 0 for i in range(8))

    bad = toy_bank()
    bad.version_bytes["3"]["w4a4"] += 1
    with pytest.raises(ValueError, match="storage differs"):
        install_bank(_toy_model(), bad, clips)
    small = toy_bank()
    small.storage_limit = small.resident_bytes()
    with pytest.raises(ValueError, match="exceeds storage budget"):
        scales = {n: torch.ones(128, dtype=torch.bfloat16) for n in small.shapes}
        install_bank(_toy_model(), small, clips, channel_scales=scales)
    wrong = _toy_model()
    wrong[2] = torch.nn.Linear(64, 8)
    with pytest.raises(ValueError, match="does not match the calibrated matrix: 2"):
        install_bank(wrong, toy_bank(), clips)
    assert isinstance(wrong[0], torch.nn.Linear)  # nothing replaced on failure


def test_shared_activation_sharing_plan():
    """The scope's record of one pass: a call is marked shared when another
    call of the pass reads the same tensor at the same width and channel
    scale (q/k/v and gate/up on x), and not when its input is read once (o
    on the attention output) or at a width no other call uses."""
    from actune_amd.kernels.grouped import SharedActivationCache, shared_activation_scope
    x, attn, mlp = torch.zeros(2), torch.zeros(2), torch.zeros(2)
    scale = torch.ones(2)
    state = SharedActivationCache()
    calls = [(x, 4, None), (x, 4, None), (x, 2, None), (attn, 4, None), (x, 4, None), (mlp, 4, None),
             (mlp, 4, scale), (mlp, 4, scale)]
    assert [state.record(*c) for c in calls] == list(range(len(calls)))
    assert state.sharing_plan() == (True, True, False, False, True, False, True, True)
    # a second pass of the same function reads fresh tensors in the same order
    again = SharedActivationCache(plan=state.sharing_plan())
    x2, attn2, mlp2 = torch.zeros(2), torch.zeros(2), torch.zeros(2)
    for src, w, sc in [(x2, 4, None), (x2, 4, None), (x2, 2, None), (attn2, 4, None), (x2, 4, None),
                       (mlp2, 4, None), (mlp2, 4, scale), (mlp2, 4, scale)]:
        again.record(src, w, sc)
    assert again.sharing_plan() == again.plan
    with shared_activation_scope(enabled=True, plan=(False,)) as st:
        assert st.plan == (False,) and st.enabled
