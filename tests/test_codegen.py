"""Checks on the device code of the built library (our own build): no packed
fp32 VALU instructions (the library is compiled with packed-fp32-ops off),
every kernel is gfx950 code, and no VALU instruction touches an MFMA result
register before the MFMA's wait states have passed on every control-flow
path."""
import collections
import re
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


# ---------------------------------------------------------------- MFMA result hazard
# A VALU instruction that reads or writes a VGPR written by an int8 MFMA must
# issue at least MFMA_WAIT wait states after it (every instruction counts one,
# s_nop N counts N + 1). In straight-line code the compiler never leaves fewer
# than 8 here; across a branch its wait states have been seen missing (the
# read then sees the register's old value), so the check follows every
# control-flow path backwards from each VALU instruction.
MFMA_WAIT = 8
_INS = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):")
_FN = re.compile(r"^([0-9a-f]+) <(.+)>:$")
_TGT = re.compile(r"<(.+)\+0x([0-9a-f]+)>\s*$")
_END_FLOW = ("s_branch", "s_endpgm", "s_setpc_b64")


def _vgprs(tok):
    m = re.fullmatch(r"v(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    return set(range(int(m.group(1)), int(m.group(2)) + 1)) if m else set()


def _operands(args):
    toks = [x.strip() for x in args.split(",") if x.strip()]
    dest = _vgprs(toks[0].split()[0]) if toks else set()
    srcs = set()
    for x in toks[1:]:
        srcs |= _vgprs(x.split()[0])
    return dest, srcs


def _functions(text):
    fns, cur, base = {}, None, 0
    for line in text.splitlines():
        m = _FN.match(line.strip())
        if m:
            cur, base = m.group(2), int(m.group(1), 16)
            fns[cur] = []
            continue
        m = _INS.match(line)
        if m and cur:
            t = _TGT.search(line)
            fns[cur].append((int(m.group(3), 16) - base, m.group(1), m.group(2),
                             int(t.group(2), 16) if t and t.group(1) == cur else None))
    return fns


def _mfma_hazards(ins):
    index = {a: k for k, (a, *_rest) in enumerate(ins)}
    preds = collections.defaultdict(list)
    for k, (_a, op, _args, t) in enumerate(ins):
        if k + 1 < len(ins) and op not in _END_FLOW:
            preds[k + 1].append(k)
        if t is not None and (op.startswith("s_cbranch") or op == "s_branch") and t in index:
            preds[index[t]].append(k)
    found = []
    for k, (a, op, args, _t) in enumerate(ins):
        if not op.startswith("v_") or op.startswith("v_mfma"):
            continue
        dest, srcs = _operands(args)
        touched = dest | srcs
        if not touched:
            continue
        stack, seen = [(p, 0) for p in preds[k]], set()
        while stack:
            j, ws = stack.pop()
            if ws >= MFMA_WAIT or (j, ws) in seen:
                continue
            seen.add((j, ws))
            _a2, op2, args2, _t2 = ins[j]
            if op2.startswith("v_mfma") and _operands(args2)[0] & touched:
                found.append((hex(a), op, args, ws))
                break
            step = int(args2.split()[0], 0) + 1 if op2 == "s_nop" else 1
            stack.extend((p, ws + step) for p in preds[j])
    return found


def test_mfma_results_wait_on_every_path(device_asm):
    fns = _functions(device_asm)
    assert any(any(op.startswith("v_mfma") for _a, op, _x, _t in ins) for ins in fns.values())
    bad = {name: h[:3] for name, ins in fns.items() if (h := _mfma_hazards(ins))}
    assert not bad, f"VALU access to an MFMA result before {MFMA_WAIT} wait states: {bad}"


# ---------------------------------------------------------------- M0 and LDS DMA
def test_m0_is_only_set_for_lds_dma(device_asm):
    """The tokenwise ring kernel issues its LDS-DMA loads from inline asm
    that sets M0 (the LDS base of the load) itself. The compiler reserves M0
    and does not expect the asm to change it, so the shipped code must use
    M0 nowhere else: every reference to m0 is that s_mov, followed by the
    one wait state and the load, and every LDS-DMA load has its own M0 set
    right before it."""
    fns = _functions(device_asm)
    loads = 0
    for name, ins in fns.items():
        for k, (_a, op, args, _t) in enumerate(ins):
            if re.search(r"\bm0\b", args):
                assert op == "s_mov_b32" and args.startswith("m0,"), (name, op, args)
                assert k + 2 < len(ins) and ins[k + 1][1] == "s_nop" and ins[k + 2][1] == "buffer_load_dwordx4" \
                    and ins[k + 2][2].endswith(" lds"), (name, ins[k:k + 3])
            if op.startswith("buffer_load") and args.endswith(" lds"):
                loads += 1
                assert k >= 2 and ins[k - 2][1] == "s_mov_b32" and ins[k - 2][2].startswith("m0,"), (name, op, args)
    assert loads > 0, "no LDS-DMA loads in the library"
