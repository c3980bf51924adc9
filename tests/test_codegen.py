"""Checks on the device code of the built library (our own build): no packed
fp32 VALU instructions (the library is compiled with packed-fp32-ops off)
and every kernel is gfx950 code."""
import shutil
import subprocess
from pathlib import Path

import pytest

from actune_amd import _native

LLVM = Path("/opt/rocm/llvm/bin")


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    objdump = LLVM / "llvm-objdump"
    if not objdump.exists():
        pytest.skip("llvm-objdump not available")
    work = tmp_path_factory.mktemp("codeobj")
    lib = work / "lib.so"
    shutil.copy(_native.LIB_PATH, lib)
    subprocess.run([str(objdump), "--offloading", str(lib)], check=True, capture_output=True, cwd=work)
    bundles = sorted(work.glob("lib.so.*gfx950*"))
    assert bundles, "no gfx950 code object in the library"
    text = []
    for b in bundles:
        res = subprocess.run([str(objdump), "-d", str(b)], check=True, capture_output=True, text=True)
        text.append(res.stdout)
    return "\n".join(text)


def test_no_packed_fp32_instructions(device_asm):
    for op in ("v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32"):
        assert op not in device_asm, op


def test_kernels_use_int8_mfma(device_asm):
    assert "v_mfma_i32_16x16x64_i8" in device_asm
    assert "buffer_load_dwordx4" in device_asm
