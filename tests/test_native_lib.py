"""CPU checks of the C ABI library: it loads without a GPU, exports every
symbol include/actune_hip.h declares, passes its host layout self-test and
rejects bad arguments before launching anything."""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

from actune_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "actune_hip.h"


def declared_functions():
    text = HEADER.read_text()
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(actune_[a-z_0-9]+)\s*\(", text, re.M)
    assert names, "no declarations found"
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    names = declared_functions()
    assert {"actune_quantize_groups", "actune_grouped_linear", "actune_grouped_forward",
            "actune_grouped_dots_i32", "actune_version", "actune_last_error"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name


def test_ceiling_library_loads_and_rejects_bad_arguments():
    """The diagnostic ceiling library (timed by bench.py) is built beside the
    main one; it checks its arguments before launching anything."""
    from actune_amd import build
    lib = ctypes.CDLL(str(build.CEILING_LIB))
    lib.actune_ceiling_macs_per_iter.restype = ctypes.c_long
    lib.actune_ceiling_macs_per_iter.argtypes = [ctypes.c_int]
    assert lib.actune_ceiling_words() == 48
    assert [lib.actune_ceiling_macs_per_iter(k) for k in range(9)] == \
        [4 * 65536] * 4 + [8 * 65536] + [4 * 65536] * 2 + [8 * 65536] * 2
    assert lib.actune_ceiling_macs_per_iter(9) == -1
    lib.actune_ceiling_run.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p]
    assert lib.actune_ceiling_run(0, None, None, 1, 1, None) == -1
    buf = ctypes.create_string_buffer(16)
    assert lib.actune_ceiling_run(9, buf, buf, 1, 1, None) == -1     # unknown kind
    assert lib.actune_ceiling_run(0, buf, buf, 0, 1, None) == -1     # no workgroups
    # the decode load floor checks its problems, wave count, row split and sink
    f = lib.actune_ceiling_decode_floor
    f.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int64,
                  ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    w = (ctypes.c_void_p * 1)(ctypes.addressof(buf))
    n = (ctypes.c_int64 * 1)(4096)
    sink = ctypes.create_string_buffer(4)
    assert f(w, n, 0, 2048, 4, 0, sink, 1 << 20, None) == -1          # no problem
    assert f(w, n, 1, 2048, 6, 0, sink, 1 << 20, None) == -1          # 6 waves
    assert f(w, n, 1, 2048 * 9, 4, 0, sink, 1 << 20, None) == -1      # 9 slots per wave
    assert f(w, n, 1, 2048, 4, 0, sink, 100, None) == -1              # sink too small
    assert f(w, n, 1, 1 << 20, 4, 0, sink, 1 << 30, None) == -1       # buffer past 2 GiB


def test_version_and_layout_selftest():
    assert "gfx950" in _native.version()
    assert _native.lib().actune_layout_selftest() == 0


def test_config_table():
    n = _native.num_configs()
    assert n == 17
    assert _native.config_valid(0, 64) and not _native.config_valid(0, 65)
    assert all(_native.config_valid(c, 4096) for c in range(3, 7))
    assert all(_native.config_valid(c, 1) and _native.config_valid(c, 4096) for c in range(10, 14))
    assert all(_native.config_valid(c, 1024) and not _native.config_valid(c, 1025) for c in range(14, 17))
    assert _native.config_valid(9, 16) and not _native.config_valid(9, 17)
    assert not _native.config_valid(n, 1) and not _native.config_valid(-2, 1)
    for m in (1, 8, 16, 17, 50, 512):
        c = _native.default_config(m, 4096, 4096, 4, 8)
        assert _native.config_valid(c, m)
    # fused decode: the fewest waves whose load ring holds a wave's K-range
    assert _native.default_config(1, 4096, 4096, 4, 8) == 14
    assert _native.default_config(4, 4096, 4096, 4, 8) == 15   # 4 tokens x 16 groups exceed the x passes
    assert _native.default_config(1, 4096, 11008, 4, 8) == 16
    assert _native.default_config(1, 4096, 4096, 8, 8) == 15   # W8: 8 groups per ring
    assert _native.default_config(1, 1024, 4096, 4, 8) == 14   # narrow N, one token: fewest waves that fit
    # waves past the nonempty canonical chunks (ceil(K/256) quads) get no work
    assert _native.default_config(1, 256, 2048, 4, 4) == 14
    assert _native.default_config(2, 256, 2048, 4, 4) == 15    # 8 quads: at most 8 waves
    assert _native.default_config(8, 256, 2048, 4, 4) == 15
    assert _native.default_config(8, 256, 1024, 4, 4) == 14    # 4 quads: 4 waves
    assert _native.default_config(8, 2048, 2048, 4, 4) == 15
    assert _native.default_config(1, 4096, 65536, 4, 8) == 2   # no decode config fits
    # M = 8: 16 waves quantize x in the launch, up to four row tiles sharing a
    # workgroup; for K = 11008 no wave count both fits its ring and quantizes
    # its range, so 16 waves take the quantizer's codes
    assert _native.default_config(8, 4096, 4096, 4, 8) == 16
    assert _native.default_config(8, 11008, 4096, 4, 8) == 16
    assert _native.default_config(8, 4096, 11008, 4, 8) == 16
    # very wide N: in-launch quantization too heavy even shared by four tiles,
    # so 8 waves take the codes
    assert _native.default_config(8, 22016, 4096, 4, 8) == 15
    # M = 3..4, wide N: 16 waves and four row tiles per workgroup below 1024
    # row tiles, 8 waves and two tiles from there on (M = 2: 4 waves, one
    # tile per workgroup, below 1024 row tiles)
    assert _native.default_config(3, 11008, 4096, 4, 8) == 16
    assert _native.default_config(4, 12288, 4096, 4, 8) == 16
    assert _native.default_config(4, 22016, 4096, 4, 8) == 15
    assert _native.default_config(2, 4096, 4096, 4, 8) == 14  # narrow N: as for M = 1
    assert _native.default_config(2, 11008, 4096, 4, 8) == 14  # two tokens: one tile per workgroup
    assert _native.default_config(2, 22016, 4096, 4, 8) == 15
    # M = 9..16: the quantizer's codes (16-token tile); 16 waves and shared
    # row tiles below 1024 row tiles, 8 waves from there on and for narrow N;
    # K = 11008 fits no wave count at 16 tokens: the streaming kernel
    assert _native.default_config(16, 12288, 4096, 4, 8) == 16
    assert _native.default_config(12, 22016, 4096, 4, 8) == 15
    assert _native.default_config(16, 4096, 4096, 4, 8) == 15
    assert _native.default_config(16, 4096, 11008, 4, 8) == 9
    # M = 17..64 (16-token blocks): the Gemma-300M expert shapes at M = 50
    assert _native.default_config(50, 4096, 1024, 4, 4) == 14
    assert _native.default_config(50, 1024, 4096, 8, 4) == 15
    assert _native.default_config(50, 4096, 4096, 4, 4) == 16
    # wide N at K = 1024 (4 quads): 4 waves, where 16 would leave 12 idle
    assert _native.default_config(17, 8192, 1024, 4, 4) == 14
    assert _native.default_config(8, 8192, 1024, 2, 4) == 14
    assert _native.default_config(4, 8192, 1024, 4, 4) == 14
    import torch
    # from 1024 row tiles above 16 tokens: 16 waves for K >= 4096, 4 below
    assert _native.default_config(32, 22016, 4096, 4, 8) == 16
    assert _native.default_config(50, 22016, 4096, 8, 8) == 16
    assert _native.default_config(50, 32768, 2048, 4, 4) == 14
    assert _native.default_config(24, 16384, 2048, 4, 4) == 14
    # W8 at 2-4 tokens takes at most 8 waves; W2 at K >= 4096 takes 16
    assert _native.default_config(2, 1024, 4096, 8, 4) == 15
    assert _native.default_config(4, 1024, 1024, 8, 8) == 14
    assert _native.default_config(3, 1024, 4096, 2, 8) == 16
    assert _native.default_config(2, 4096, 4096, 2, 4) == 16
    assert _native.default_config(4, 2048, 4096, 2, 2) == 16
    assert _native.default_config(2, 4096, 2048, 2, 4) == 14
    # W8 4096x4096 at 13-16 tokens: 8 waves on codes; 16 waves in the launch at 9-12, on codes from 17
    assert _native.default_config(13, 4096, 4096, 8, 4) == 15
    assert _native.default_config(16, 4096, 4096, 8, 8) == 15
    assert _native.default_config(10, 4096, 4096, 8, 8) == 16
    assert _native.default_config(17, 4096, 4096, 8, 8) == 16
    # narrow W8 at 5-8 tokens: 8 waves with x quantized in the launch; W4 keeps 16
    assert _native.default_config(5, 4096, 4096, 8, 8) == 15
    assert _native.default_config(8, 1024, 4096, 8, 4) == 15
    assert _native.forward_fuses_quantizer(8, 1024, 4096, 8, 4, torch.bfloat16)
    assert _native.default_config(8, 4096, 4096, 4, 8) == 16
    assert _native.default_config(8, 4096, 8192, 8, 8) == 16  # 8 waves do not hold K = 8192 of W8
    # in-launch quantization with 8-token tiles up to 300 group-rows per SIMD
    # (W4A8 22016x4096: 215 at M = 5, 344 at M = 8)
    assert _native.forward_fuses_quantizer(5, 22016, 4096, 4, 8, torch.bfloat16)
    assert not _native.forward_fuses_quantizer(8, 22016, 4096, 4, 8, torch.bfloat16)
    # in-launch quantization with 16-token blocks up to 200 group-rows per SIMD
    bf16 = torch.bfloat16
    assert _native.forward_fuses_quantizer(50, 8192, 1024, 4, 4, bf16)      # 200
    assert not _native.forward_fuses_quantizer(64, 8192, 1024, 4, 4, bf16)  # 256
    assert _native.forward_fuses_quantizer(50, 2048, 2048, 4, 4, bf16, 15)
    assert _native.default_config(65, 4096, 4096, 4, 8) not in (14, 15, 16)  # 192 prefill tiles
    # above 64 tokens, narrow problems (at most 128 tiles of 64x32, K <= 4096)
    # run the decode kernel in 16-token blocks
    assert _native.default_config(256, 256, 2048, 4, 4) == 15
    assert _native.default_config(128, 1024, 1024, 4, 4) == 14
    assert _native.default_config(256, 512, 4096, 8, 8) == 16
    assert _native.default_config(96, 2048, 16384, 4, 4) == 13  # K above 4096
    # prefill: 64x32 tiles below two 64x64 tiles per CU, 64x64 below four,
    # 128x64 from four for W <= 4 (W8 keeps 64x64), the tiled kernel from eight
    assert _native.default_config(256, 2048, 2048, 4, 4) == 13
    assert _native.default_config(512, 4096, 4096, 4, 8) == 12
    assert _native.default_config(256, 16384, 2048, 4, 4) == 10
    assert _native.default_config(512, 11008, 4096, 2, 8) == 10
    assert _native.default_config(512, 11008, 4096, 8, 8) == 12
    assert _native.default_config(2048, 4096, 4096, 4, 8) == 3


def _err():
    return _native.lib().actune_last_error().decode()


@pytest.mark.parametrize("args,msg", [
    (dict(A=3), "Unsupported integer width"),
    (dict(K=100), "K divisible by 64"),
    (dict(dt=7), "dtype"),
])
def test_quantize_rejects_bad_arguments(args, msg):
    p = dict(x=None, dt=0, sc=None, M=4, K=128, A=8)
    p.update(args)
    rc = _native.lib().actune_quantize_groups(p["x"], p["dt"], p["sc"], p["M"], p["K"], p["A"], None, None, None)
    assert rc == 1 and msg in _err()


@pytest.mark.parametrize("args,msg", [
    (dict(W=5), "Unsupported integer width"),
    (dict(K=96), "invalid dimensions"),
    (dict(N=0), "invalid dimensions"),
    (dict(config=0, M=65), "M <= 64"),
    (dict(config=14, M=1025), "M <= 1024"),
    (dict(config=99), "invalid configuration"),
    (dict(out_dt=9), "dtype"),
    (dict(M=4), "null pointer"),
])
def test_linear_rejects_bad_arguments(args, msg):
    p = dict(M=4, N=32, K=128, W=4, A=8, config=3, out_dt=0)
    p.update(args)
    rc = _native.lib().actune_grouped_linear(None, None, None, None, None, 2, None, p["out_dt"],
                                             p["M"], p["N"], p["K"], p["W"], p["A"], p["config"], None)
    assert rc == 1 and msg in _err()


def test_auto_config_with_invalid_arguments_reports_them():
    """ACTUNE_CONFIG_AUTO with a width or dimension no call takes used to run
    the config selection on it first (a division by the weight width: the
    process died of SIGFPE); the call now names the bad argument."""
    lib = _native.lib()
    for W in (0, 16):
        rc = lib.actune_grouped_linear(None, None, None, None, None, 2, None, 0, 4, 32, 128, W, 8, -1, None)
        assert rc == 1 and "Unsupported integer width" in _err()
    rc = lib.actune_grouped_forward(None, 0, None, None, None, None, None, None, 2, None, 4, 0, 128, 4, 8, -1, None)
    assert rc == 1 and "invalid dimensions" in _err()
    assert _native.default_config(4, 4096, 4096, 0, 8) == -1
    assert _native.default_config(4, 4096, 100, 4, 8) == -1


def test_entry_points_survive_argument_fuzz():
    """tests/abi_fuzz.py in a child process: every entry point, NULL buffers,
    edge-case and invalid arguments; each call returns a status (OK only for
    an empty call) and none crashes."""
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "abi_fuzz.py"), str(_native.LIB_PATH), "3000"],
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, (res.returncode, res.stdout[-2000:], res.stderr[-2000:])


def test_zero_rows_is_a_no_op_without_a_gpu():
    lib = _native.lib()
    assert lib.actune_grouped_linear(None, None, None, None, None, 2, None, 0, 0, 32, 128, 4, 8, -1, None) == 0
    assert lib.actune_quantize_groups(None, 0, None, 0, 128, 8, None, None, None) == 0


def test_streaming_config_reports_its_own_limit():
    rc = _native.lib().actune_grouped_linear(None, None, None, None, None, 2, None, 0, 17, 32, 128, 4, 8, 8, None)
    assert rc == 1 and "M <= 16" in _err()


def test_tokenwise_split_rule():
    """Tokenwise GEMM K splits, read from the workspace the library asks for
    (S x M x N int32 when S > 1). Ring GEMM (M > 32): the split doubles while
    the 64 x 128 grid has fewer workgroups than the 256 CUs and the partials
    stay within 8 MiB, each split keeping 4 K-steps below 128 workgroups and
    16 from there. M <= 32: the fewest splits whose ranges fit the entry
    loads."""
    a8, w4, w2 = _native.TW_ACT_A8, _native.TW_KMAJOR_W4, _native.TW_KMAJOR_W2

    def split_of(m, n, k, wl=w4):
        need = _native.tokenwise_workspace_bytes(m, n, k, wl, a8)
        assert need % (m * n * 4) == 0
        return max(1, need // (m * n * 4))

    assert split_of(512, 4096, 4096) == 1    # 256 workgroups
    assert split_of(256, 4096, 4096) == 2    # 128 workgroups, 64 K-steps
    assert split_of(128, 4096, 11008) == 4   # 64 workgroups, 172 K-steps, 8 MiB of partials
    assert split_of(64, 4096, 4096) == 4     # a third doubling would leave 8 K-steps
    assert split_of(128, 4096, 4096, w2) == 2  # 32 K-steps of 128
    assert split_of(320, 4096, 4096) == 1    # two splits would hold 10 MiB of partials
    assert split_of(64, 512, 4096) == 16     # 4 workgroups: down to 4 K-steps
    # M <= 32: the fewest splits whose ranges fit the 8 K-steps a workgroup
    # loads at entry (4 for the int8 K-major layout)
    assert split_of(1, 4096, 4096) == 8
    assert split_of(8, 4096, 11008) == 22
    assert split_of(1, 256, 2048) == 4
    assert split_of(1, 4096, 4096, _native.TW_KMAJOR_W8) == 16
    assert split_of(32, 128, 512) == 1       # one workgroup range: no reduce


@pytest.mark.parametrize("M", range(1, 17))
def test_decode_row_division_is_exact_over_its_range(M):
    """gemm_decode divides group-row indices r = group * M + token by M as
    (r * ceil(2^16 / M)) >> 16 (launch.hpp, LinearArgs::m_div); decode_fits
    keeps r below 16 groups x 16 tokens. Exact over that range for every M of
    a 16-token block and for every ragged tail, and the stated first failure
    (r = 4694 at M = 15) is where the identity r * e < 2^16 says."""
    d = (65536 + M - 1) // M
    assert all((r * d) >> 16 == r // M for r in range(256))
    e = d * M - 65536
    bad = [r for r in range(1 << 16) if (r * d) >> 16 != r // M]
    if e == 0:
        assert not bad
    else:
        assert bad and bad[0] >= 65536 // e
    if M == 15:
        assert bad[0] == 4694
