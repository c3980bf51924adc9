"""Request-scoped precision dispatch and shared resident-bank accounting.

Same contract as actune/precision.py:10-88 (the ContextVar-scoped profile and
SharedBank's budget rules and error messages), together with the two names
it depends on: CONFIGURATIONS (actune/tree.py:13) and pair()
(actune/_allocation/pi05_budget.py:19-22). The error messages are kept
verbatim because callers and tests match on them.
"""
from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
import math
import sys

CONFIGURATIONS = ("q00", "q01", "q11", "q10")
_WIDTHS = (2, 4, 8)
_EPS = 1e-12

_active = ContextVar("actune_precision_profile", default=None)


def pair(mode):
    """Split a 'w{W}a{A}' mode name into (W, A)."""
    ok = isinstance(mode, str) and len(mode) == 4 and mode[0] == "w" and mode[2] == "a"
    if ok and mode[1].isdigit() and mode[3].isdigit():
        w, a = int(mode[1]), int(mode[3])
        if w in _WIDTHS and a in _WIDTHS:
            return w, a
    raise ValueError(f"invalid pi05 precision: {mode}")


def active_precision_profile():
    """The configuration of the request being served, or None.

    When the reference's own ``actune.precision`` is loaded as a separate
    module (a deployment that changed its imports to this package but kept
    the reference Controller, whose runtime.py:9 binds the reference's
    ``precision_profile``), a configuration set there is honoured too, so
    dispatch never silently falls back to the default profile.
    """
    current = _active.get()
    if current is None:
        other = sys.modules.get("actune.precision")
        if other is not None and other is not sys.modules.get(__name__):
            getter = getattr(other, "active_precision_profile", None)
            if callable(getter):
                current = getter()
    return current


@contextmanager
def precision_profile(configuration):
    """Make `configuration` active for the enclosed block; nesting restores."""
    if configuration not in CONFIGURATIONS:
        raise ValueError("Unknown ActTune configuration")
    token = _active.set(configuration)
    try:
        yield
    finally:
        _active.reset(token)


def _weighted_mean(pairs):
    """sum(weight * value) / sum(weight) over (weight, value) pairs."""
    num = den = 0
    for weight, value in pairs:
        num += weight * value
        den += weight
    return num / den


@dataclass
class SharedBank:
    """Four precision configurations over one resident set of weight versions.

    configurations: {q: {layer: mode}}; shapes: {layer: [out, in]};
    activation_elements: {layer: elements per request}; shape_groups: lists
    of layers that execute with the same activation shape; version_bytes:
    {layer: {mode: bytes}}; budget: 'w4a4' or 'w4a8'; storage_limit: bytes.
    """
    configurations: dict
    shapes: dict
    activation_elements: dict
    shape_groups: list
    version_bytes: dict
    budget: str
    storage_limit: int

    def _versions(self):
        return {name: {cfg[name] for cfg in self.configurations.values()} for name in self.shapes}

    def resident_bytes(self):
        """Bytes of every version any configuration uses, each counted once."""
        return sum(self.version_bytes[name][mode]
                   for name, modes in self._versions().items() for mode in modes)

    def metrics(self, configuration, activation_elements=None):
        """Parameter-weighted weight bits, element-weighted activation bits,
        and activation bits per shape group for one configuration."""
        modes = self.configurations[configuration]
        counts = self.activation_elements if activation_elements is None else activation_elements
        positive = all(type(v) is int and v > 0 for v in counts.values())
        if set(counts) != set(self.shapes) or not positive:
            raise ValueError("Every target must execute with a positive activation-element count")
        bits = {name: pair(mode) for name, mode in modes.items()}
        weight_bits = _weighted_mean((math.prod(self.shapes[n]), bits[n][0]) for n in bits)
        act_bits = _weighted_mean((counts[n], bits[n][1]) for n in bits)
        group_bits = [_weighted_mean((counts[n], bits[n][1]) for n in group) for group in self.shape_groups]
        return dict(weight_bits=weight_bits, activation_bits=act_bits, group_activation_bits=group_bits)

    def check_request(self, configuration, counts=None):
        """Raise if one request under `configuration` breaks the budget."""
        m = self.metrics(configuration, counts)
        if m["weight_bits"] > 4 + _EPS:
            raise ValueError("Active weight budget exceeds four bits")
        if self.budget == "w4a4":
            if max([m["activation_bits"], *m["group_activation_bits"]]) > 4 + _EPS:
                raise ValueError("Active activation budget exceeds four bits")
        elif self.budget == "w4a8":
            if any(pair(mode)[1] != 8 for mode in self.configurations[configuration].values()):
                raise ValueError("W4A8 requires A8 on every target")
        return m

    def validate(self):
        """Check the bank's structure and every configuration; returns self."""
        if self.budget not in ("w4a4", "w4a8") or set(self.configurations) != set(CONFIGURATIONS):
            raise ValueError("Expected a W4A4/W4A8 bank with four configurations")
        for shape in self.shapes.values():
            if len(shape) != 2 or not all(type(v) is int and v > 0 for v in shape):
                raise ValueError("Invalid matrix shapes")
        if not self.shapes:
            raise ValueError("Invalid matrix shapes")
        members = sorted(name for group in self.shape_groups for name in group)
        if members != sorted(self.shapes) or not all(self.shape_groups):
            raise ValueError("Invocation-shape groups must partition the targeted layers")
        if any(set(cfg) != set(self.shapes) for cfg in self.configurations.values()):
            raise ValueError("Configuration coverage differs from targeted layers")
        versions = self._versions()
        switchable = sorted(len(v) for v in versions.values() if len(v) > 1)
        if switchable != [2, 2]:
            raise ValueError("Paper bank requires exactly two binary switchable matrices")
        order = sorted(self.shapes)
        if len({tuple(cfg[n] for n in order) for cfg in self.configurations.values()}) != 4:
            raise ValueError("Configurations must realize all four alternatives")
        for name, modes in versions.items():
            for mode in modes:
                pair(mode)
                size = self.version_bytes[name][mode]
                if type(size) is not int or size <= 0:
                    raise ValueError("Version storage must include packed weights, scales and bias")
        for configuration in CONFIGURATIONS:
            self.check_request(configuration)
        if self.storage_limit <= 0 or self.resident_bytes() > self.storage_limit:
            raise ValueError("All resident versions together exceed storage budget")
        return self
