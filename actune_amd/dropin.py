"""Serve the reference's ``actune.*`` import paths from this package.

A deployment of the reference (zanehpn/Actune) imports its hot-path modules
by their ``actune`` names: ``from actune import Controller`` pulls in
``actune/runtime.py``, which binds ``precision_profile`` from
``actune.precision`` (runtime.py:9, used at :78), and the integration example
then imports ``install_bank`` from ``actune.layers`` (examples/integrate.py:8-9).
For the Controller's ``precision_profile(cfg)`` to select the resident
version that this package's modules dispatch on, both names must resolve to
the SAME module object, before the reference package itself is imported.

``install()`` puts a finder at the front of ``sys.meta_path`` that answers
each aliased ``actune.<name>`` with the already-imported module of this
package, so the reference package's own relative imports (``from .precision
import precision_profile``) land on it as well. Everything else under
``actune`` (controller, tree, features, device, allocation) still comes from
the reference installation. Call it before anything imports ``actune``:

    import actune_amd.dropin
    actune_amd.dropin.install()
    from actune import Controller, Prediction        # reference control plane
    from actune.layers import install_bank           # this package
"""
from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

# reference module path -> module of this package that replaces it
ALIASES = {
    "actune.precision": "actune_amd.precision",
    "actune.layers": "actune_amd.layers",
    "actune.graph": "actune_amd.graph",
    "actune.kernels.grouped": "actune_amd.kernels.grouped",
    "actune.kernels.quantizers": "actune_amd.kernels.quantizers",
    "actune.kernels.tuning": "actune_amd.kernels.tuning",
    # the tokenwise family: one module serves the five reference modules
    "actune.kernels.w4a8_triton": "actune_amd.kernels.tokenwise",
    "actune.kernels.w8a8_triton": "actune_amd.kernels.tokenwise",
    "actune.kernels.w2a8_triton": "actune_amd.kernels.tokenwise",
    "actune.kernels.wxa4_native": "actune_amd.kernels.tokenwise",
    "actune.kernels.decode_w4a8_triton": "actune_amd.kernels.tokenwise",
    "actune.kernels.resident_a8_triton": "actune_amd.kernels.tokenwise",
    "actune.kernels.runtime_options": "actune_amd.kernels.tokenwise",
}


class _AliasLoader(importlib.abc.Loader):
    """Hands the import system an existing module object under a second name."""

    def __init__(self, target: str):
        self.target = target
        self._spec = None

    def create_module(self, spec):
        module = importlib.import_module(self.target)
        self._spec = module.__spec__
        return module

    def exec_module(self, module):
        # the import machinery stamped the alias spec on the shared module;
        # give it back its own, so reload() and pickling keep working
        if self._spec is not None:
            module.__spec__ = self._spec


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        if fullname not in ALIASES:
            return None
        return importlib.util.spec_from_loader(fullname, _AliasLoader(ALIASES[fullname]))


_FINDER = _AliasFinder()


def install() -> None:
    """Route the aliased ``actune.*`` imports to this package (idempotent).

    Raises RuntimeError if one of them was already imported from elsewhere:
    the reference's ``precision_profile`` would then already be bound to a
    different ContextVar, which is exactly the silent mismatch this prevents.
    """
    clashes = [name for name, target in ALIASES.items()
               if name in sys.modules and sys.modules[name] is not sys.modules.get(target)]
    if clashes:
        raise RuntimeError("install() must run before these modules are imported: " + ", ".join(sorted(clashes)))
    if _FINDER not in sys.meta_path:
        sys.meta_path.insert(0, _FINDER)


def uninstall() -> None:
    """Remove the finder (modules already imported under alias names stay)."""
    if _FINDER in sys.meta_path:
        sys.meta_path.remove(_FINDER)
