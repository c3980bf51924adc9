"""Install calibrated resident backends into an existing PyTorch model.

Same contract as actune/layers.py:9-91: ``tensor_storage_bytes``,
``ResidentLinear`` (optional channel-scale folding), ``BankRuntime``
(per-request counters and audit) and ``install_bank`` (validate, build,
byte-check, swap modules). The one behavioural difference is internal: the
runtime division ``x / input_scale`` is fused into the HIP quantizer (same
rounding: fp32 quotient rounded to x's dtype) instead of being a separate
elementwise launch.
"""
from __future__ import annotations

from types import MethodType

import torch

from .kernels.grouped import GroupedPaddedLinear


def tensor_storage_bytes(module):
    """Bytes of the distinct storages behind a module's parameters and buffers."""
    total = 0
    seen = set()
    for tensor in [*module.parameters(), *module.buffers()]:
        storage = tensor.untyped_storage()
        key = (tensor.device, storage.data_ptr())
        if key in seen:
            continue
        seen.add(key)
        total += storage.nbytes()
    return total


def _scaled_linear(linear, scale):
    """nn.Linear with weight * scale[None, :] in the weight dtype."""
    fc = torch.nn.Linear(linear.in_features, linear.out_features, bias=linear.bias is not None,
                         device=linear.weight.device, dtype=linear.weight.dtype)
    with torch.no_grad():
        fc.weight.copy_(linear.weight * scale[None, :])
        if linear.bias is not None:
            fc.bias.copy_(linear.bias)
    return fc


class ResidentLinear(GroupedPaddedLinear):
    """GroupedPaddedLinear whose input may be divided by a calibrated
    per-channel scale that was folded into the weights at install time."""

    def __init__(self, linear, assignments, clips, input_scale=None):
        scale = None
        if input_scale is not None:
            scale = torch.as_tensor(input_scale, device=linear.weight.device, dtype=linear.weight.dtype)
            valid = scale.shape == (linear.in_features,) and bool(torch.isfinite(scale).all()) \
                and bool((scale > 0).all())
            if not valid:
                raise ValueError("Invalid calibrated channel scale")
            linear = _scaled_linear(linear, scale)
        super().__init__(linear, assignments, "q11", clips)
        self.register_buffer("input_scale", scale)

    def forward(self, value):
        return self._dispatch(value, self.input_scale)


class BankRuntime:
    """Handle returned by install_bank: resets counters before a request and
    audits the executed activation elements after it."""

    def __init__(self, bank, modules):
        self.bank = bank
        self.modules = modules

    def before(self):
        for module in self.modules.values():
            module.calls = 0
            module.input_elements = 0

    def audit(self, configuration):
        executed = {name: module.input_elements for name, module in self.modules.items()}
        return self.bank.check_request(configuration, executed)


def install_bank(model, bank, clips, *, channel_scales=None, tune=False):
    """Replace every bank target of `model` with a ResidentLinear holding one
    group-64 backend per mode the bank's configurations use.

    Checks, before anything is modified: the bank is valid, every target is
    an nn.Linear of the calibrated [out, in] shape; then each backend's
    storage equals the bank's declared bytes and the total (channel scales
    included) fits the storage limit. tune=True routes backends through the
    bit-exact kernel-configuration selector.
    """
    bank.validate()
    scales = channel_scales or {}
    targets = {}
    for name in bank.shapes:
        module = model.get_submodule(name)
        if not isinstance(module, torch.nn.Linear) or \
                [module.out_features, module.in_features] != list(bank.shapes[name]):
            raise ValueError(f"Target does not match the calibrated matrix: {name}")
        targets[name] = module
    built = {}
    for name, linear in targets.items():
        assignment = {q: modes[name] for q, modes in bank.configurations.items()}
        resident = ResidentLinear(linear, assignment, clips[name], scales.get(name))
        for mode, backend in resident.backends.items():
            if tensor_storage_bytes(backend) != bank.version_bytes[name][mode]:
                raise ValueError(f"Loaded backend storage differs from calibration: {name}/{mode}")
            if tune:
                from .kernels.tuning import grouped_forward
                backend._untuned_forward = backend.forward
                backend.forward = MethodType(grouped_forward, backend)
        built[name] = resident
    if sum(tensor_storage_bytes(m) for m in built.values()) > bank.storage_limit:
        raise ValueError("Loaded bank, including channel scales, exceeds storage budget")
    for name, module in built.items():
        parent, _, child = name.rpartition(".")
        setattr(model.get_submodule(parent), child, module)
    return BankRuntime(bank, built)
