"""Builds libactune_hip.so in-tree with hipcc for gfx950.

Usage: ``python -m actune_amd.build [--incremental]`` (or
``__graft_entry__.build()``, which always compiles everything).
Objects go to ``actune_amd/_build/``, the library to ``actune_amd/lib/``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libactune_hip.so"
SOURCES = ["api.hip", "quantize.hip", "gemm_smallm.hip", "gemm_tiled.hip", "gemm_stream.hip", "gemm_prefill.hip", "gemm_decode.hip",
           "gemm_decode_mixed.hip", "noalloc.hip", "tokenwise.hip"]
# diagnostic library of register-resident compute ceilings, timed by bench.py
CEILING_SOURCE = "ceiling.hip"
CEILING_LIB = LIB_DIR / "libactune_ceiling.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # every FMA in the kernels is an explicit fmaf: no contraction
        "-ffp-contract=off",
        # packed fp32 VALU ops are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in VGPRs: the fp32 epilogue reads them without
        # v_accvgpr_read copies
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    ]


def _includes(path: Path, seen: set) -> None:
    """Adds path and every local header it includes (transitively) to seen."""
    if path in seen or not path.exists():
        return
    seen.add(path)
    for line in path.read_text().splitlines():
        line = line.strip()
        if line.startswith("#include \""):
            _includes((path.parent / line.split('"')[1]).resolve(), seen)


def _stale(src: str, out: Path) -> bool:
    """True when `out` is missing or older than the source, a header it
    includes, or this build script."""
    if not out.exists():
        return True
    deps = {Path(__file__)}
    _includes((CSRC / src).resolve(), deps)
    return any(d.stat().st_mtime > out.stat().st_mtime for d in deps)


def _compile(src: str, incremental: bool = False) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    if incremental and not _stale(src, out):
        return out
    cmd = [hipcc(), *flags(), "-c", str(CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return out


def build(verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every source (or, incremental, only the out-of-date ones) and
    link the library."""
    OBJ.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as pool:
        objs = list(pool.map(lambda src: _compile(src, incremental), SOURCES + [CEILING_SOURCE]))
    for lib, parts in ((LIB, objs[:-1]), (CEILING_LIB, objs[-1:])):
        tmp = lib.with_suffix(".so.tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, parts)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        os.replace(tmp, lib)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
