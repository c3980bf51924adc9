"""CPU tests of the drop-in import paths (actune_amd.dropin).

A stand-in ``actune`` package plays the reference installation: its
``__init__`` imports ``runtime`` (the Controller), whose module binds
``precision_profile`` from ``.precision`` exactly as actune/runtime.py:9 does,
and the caller then imports ``install_bank`` from ``actune.layers`` in the
order of examples/integrate.py:8-9. The reference's own ``layers`` and
``kernels.grouped`` are stand-ins that fail if they are ever imported.
"""
import subprocess
import sys
import textwrap
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

STANDIN = {
    "actune/__init__.py": "from .runtime import Controller, Prediction\n",
    "actune/runtime.py": textwrap.dedent("""
        from .precision import precision_profile

        class Prediction:
            pass

        class Controller:
            def __init__(self, policy):
                self.policy = policy

            def predict(self, observation, configuration):
                with precision_profile(configuration):
                    return self.policy(observation, configuration)
    """),
    "actune/precision.py": textwrap.dedent("""
        from contextlib import contextmanager
        from contextvars import ContextVar
        _active = ContextVar("reference_profile", default=None)

        def active_precision_profile():
            return _active.get()

        @contextmanager
        def precision_profile(configuration):
            token = _active.set(configuration)
            try:
                yield
            finally:
                _active.reset(token)
    """),
    "actune/layers.py": "raise ImportError('the reference layers module was imported')\n",
    "actune/kernels/__init__.py": "",
    "actune/kernels/grouped.py": "raise ImportError('the reference grouped module was imported')\n",
}

# A GroupedPaddedLinear whose q00 and q11 versions differ; the Controller
# serves one request under q00 and one under q11 and reports which backend
# the module would dispatch to.
CHECK = textwrap.dedent("""
    import torch
    {prologue}
    from actune import Controller
    from {layers} import install_bank
    from {grouped} import GroupedPaddedLinear
    import actune_amd.layers, actune_amd.precision

    lin = torch.nn.Linear(128, 16, bias=False)
    assign = {{"q00": "w2a4", "q01": "w4a8", "q11": "w4a8", "q10": "w4a8"}}
    m = GroupedPaddedLinear(lin, assign, "q11", {{"w2a4": None, "w4a8": None}})
    ctl = Controller(lambda obs, cfg: (m.active_backend().w, m.active_backend().a))
    assert ctl.predict(None, "q00") == (2, 4), ctl.predict(None, "q00")
    assert ctl.predict(None, "q11") == (4, 8)
    assert m.active_backend() is m.backends["w4a8"]  # outside a request: the default profile
    print("ALIASED", __import__("sys").modules["actune.precision"] is actune_amd.precision,
          install_bank is actune_amd.layers.install_bank)
""")


def _run(tmp_path, prologue, layers, grouped):
    for rel, text in STANDIN.items():
        path = tmp_path / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text)
    code = CHECK.format(prologue=prologue, layers=layers, grouped=grouped)
    env = {"PYTHONPATH": f"{tmp_path}:{ROOT}", "PATH": "/usr/bin:/bin"}
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    return res.stdout


def test_alias_recipe_serves_reference_import_paths(tmp_path):
    """The drop-in recipe: dropin.install() first, then the reference's own
    import order; actune.precision, actune.layers and actune.kernels.grouped
    are this package's modules and the Controller's precision_profile drives
    dispatch."""
    out = _run(tmp_path, "import actune_amd.dropin; actune_amd.dropin.install()",
               "actune.layers", "actune.kernels.grouped")
    assert "ALIASED True True" in out


def test_changed_imports_with_reference_controller(tmp_path):
    """Without the alias (imports changed to actune_amd, Controller still the
    reference's): the reference ContextVar is honoured, so q00 still reaches
    the module instead of silently running the default q11."""
    out = _run(tmp_path, "", "actune_amd.layers", "actune_amd.kernels.grouped")
    assert "ALIASED False True" in out


def test_install_refuses_after_reference_import(tmp_path):
    for rel, text in STANDIN.items():
        path = tmp_path / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text)
    code = ("import actune, actune_amd.dropin\n"
            "try:\n    actune_amd.dropin.install()\nexcept RuntimeError as e:\n    print('REFUSED', e)\n")
    env = {"PYTHONPATH": f"{tmp_path}:{ROOT}", "PATH": "/usr/bin:/bin"}
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    assert "REFUSED" in res.stdout and "actune.precision" in res.stdout


def test_alias_serves_tokenwise_modules(tmp_path):
    """The tokenwise family's five reference module paths resolve to the one
    tokenwise module of this package after install()."""
    for rel, text in STANDIN.items():
        path = tmp_path / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text)
    code = textwrap.dedent("""
        import actune_amd.dropin
        actune_amd.dropin.install()
        import actune
        from actune.kernels.w4a8_triton import W4A8TritonLinear, shared_a8_cache_scope
        from actune.kernels.w8a8_triton import W8A8TritonLinear
        from actune.kernels.w2a8_triton import W2A8TritonLinear
        from actune.kernels.wxa4_native import W4A4NativeLinear, W2A4NativeLinear, W8A4NativeLinear
        from actune.kernels.decode_w4a8_triton import decode_optimization_scope, DecodeGraphPlan
        from actune.kernels.runtime_options import runtime_optimization_scope
        import actune_amd.kernels.tokenwise as T
        assert W4A8TritonLinear is T.W4A8TritonLinear and W8A4NativeLinear is T.W8A4NativeLinear
        assert decode_optimization_scope is T.decode_optimization_scope
        print("TOKENWISE OK")
    """)
    env = {"PYTHONPATH": f"{tmp_path}:{ROOT}", "PATH": "/usr/bin:/bin"}
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    assert "TOKENWISE OK" in res.stdout
