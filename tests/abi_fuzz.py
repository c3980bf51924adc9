"""Argument fuzz of the C ABI, run as a child process by
tests/test_native_lib.py (a crash then fails that test instead of ending
the test session).

Every entry point is called with NULL buffers over edge-case dimensions,
widths, dtypes, layouts and configs, including values no call accepts.
Each call must return a status code, and ACTUNE_OK only where the call is
empty (M == 0). No GPU is needed: nothing valid ever reaches a launch.

Usage: python tests/abi_fuzz.py LIBRARY CALLS
"""
import ctypes
import random
import sys

P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64


class Target(ctypes.Structure):  # actune_linear_target
    _fields_ = [("w", P), ("w_scale", P), ("bias", P), ("out", P), ("N", L), ("W", ctypes.c_int32)]


class TwTarget(ctypes.Structure):  # actune_tw_target
    _fields_ = [("w", P), ("r", P), ("w_scale", P), ("bias", P), ("out", P)]


SIGNATURES = {
    "actune_quantize_groups": [P, I, P, L, L, I, P, P, P],
    "actune_quantize_gated": [P, P, I, I, P, L, L, I, P, P, P],
    "actune_grouped_linear": [P, P, P, P, P, I, P, I, L, L, L, I, I, I, P],
    "actune_grouped_forward": [P, I, P, P, P, P, P, P, I, P, L, L, L, I, I, I, P],
    "actune_grouped_forward_multi": [P, I, P, P, P, ctypes.POINTER(Target), I, I, L, L, I, I, I, P],
    "actune_grouped_forward_noalloc": [P, I, P, P, P, P, I, P, L, L, L, I, I, I, P],
    "actune_grouped_dots_i32": [P, P, L, L, L, I, I, I, P, P],
    "actune_forward_fuses_quantizer": [L, L, L, I, I, I, I],
    "actune_default_config": [L, L, L, I, I],
    "actune_config_valid": [I, L],
    "actune_tokenwise_quantize": [P, I, L, L, I, P, P, P],
    "actune_tokenwise_workspace_bytes": [L, L, L, I, I],
    "actune_tokenwise_linear": [P, I, P, P, I, P, P, I, P, I, L, L, L, I, P, L, P],
    "actune_tokenwise_linear_x": [P, I, P, P, I, P, P, I, P, I, L, L, L, I, P, L, P],
    "actune_tokenwise_linear_multi": [P, I, P, I, P, I, ctypes.POINTER(TwTarget), I, I, I, L, L, L, I, P, L, P],
}

MS = [-1, 0, 1, 2, 8, 17, 64, 65, 512, 1024, 1025, 2**31, 2**40]
NS = [-1, 0, 1, 16, 42, 4096, 2**31, 2**40]
KS = [-64, 0, 1, 64, 100, 128, 4096, 11008, 65536, 2**31, 2**40]
WIDTHS = [-1, 0, 1, 2, 3, 4, 8, 16]
CODES = [-2, -1, 0, 1, 2, 3, 5, 6, 99]
CONFIGS = [-2, -1, 0, 3, 9, 10, 14, 16, 17]


def main(path, calls):
    lib = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        getattr(lib, name).argtypes = args
    lib.actune_tokenwise_workspace_bytes.restype = L
    rng = random.Random(0)
    bad = []

    def status(name, rc, m):
        if rc not in (0, 1, 2) or (rc == 0 and m != 0):
            bad.append((name, rc, m))

    for _ in range(calls):
        m, n, k = rng.choice(MS), rng.choice(NS), rng.choice(KS)
        w, a = rng.choice(WIDTHS), rng.choice(WIDTHS)
        dt, dt2, cfg = rng.choice(CODES), rng.choice(CODES), rng.choice(CONFIGS)
        lay, lay2 = rng.choice(CODES), rng.choice(CODES)
        ws = rng.choice([0, -1, 1 << 20])
        nt = rng.choice([-1, 0, 1, 3, 4, 5])
        targets = (Target * 5)(*[Target(None, None, None, None, rng.choice(NS), rng.choice(WIDTHS))
                                 for _ in range(5)])
        tw_targets = (TwTarget * 5)()
        status("quantize_groups", lib.actune_quantize_groups(None, dt, None, m, k, a, None, None, None), m)
        status("quantize_gated", lib.actune_quantize_gated(None, None, dt, lay, None, m, k, a, None, None, None), m)
        status("grouped_linear", lib.actune_grouped_linear(None, None, None, None, None, dt, None, dt2,
                                                           m, n, k, w, a, cfg, None), m)
        status("grouped_forward", lib.actune_grouped_forward(None, dt, None, None, None, None, None, None, dt2,
                                                             None, m, n, k, w, a, cfg, None), m)
        status("grouped_forward_multi", lib.actune_grouped_forward_multi(
            None, dt, None, None, None, targets if nt >= 0 else None, nt, dt2, m, k, w, a, cfg, None), m)
        status("grouped_forward_noalloc", lib.actune_grouped_forward_noalloc(
            None, dt, None, None, None, None, dt2, None, m, n, k, w, a, cfg, None), m)
        status("grouped_dots_i32", lib.actune_grouped_dots_i32(None, None, m, n, k, w, a, cfg, None, None), m)
        lib.actune_forward_fuses_quantizer(m, n, k, w, a, dt, cfg)
        lib.actune_default_config(m, n, k, w, a)
        lib.actune_config_valid(cfg, m)
        status("tokenwise_quantize", lib.actune_tokenwise_quantize(None, dt, m, k, a, None, None, None), m)
        lib.actune_tokenwise_workspace_bytes(m, n, k, lay, lay2)
        status("tokenwise_linear", lib.actune_tokenwise_linear(None, lay2, None, None, lay, None, None, dt, None,
                                                               dt2, m, n, k, cfg, None, ws, None), m)
        status("tokenwise_linear_x", lib.actune_tokenwise_linear_x(None, dt, None, None, lay, None, None, dt, None,
                                                                   dt2, m, n, k, cfg, None, ws, None), m)
        status("tokenwise_linear_multi", lib.actune_tokenwise_linear_multi(
            None, lay2, None, dt, None, lay, tw_targets if nt >= 0 else None, nt, dt, dt2, m, n, k, cfg, None,
            ws, None), m)
    for b in bad[:20]:
        print("bad", b)
    print(f"{calls} rounds, {len(bad)} bad")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1], int(sys.argv[2])))
