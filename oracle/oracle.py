"""CPU oracle for the group-64 packed-integer linear path (TEST INFRASTRUCTURE).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker. The product
package ``actune_amd`` never imports it; a product path that fell back to it
would be a CPU fallback, which the product forbids.

Arithmetic lives in ``grouped_oracle.c`` (plain C, built with
``-ffp-contract=off`` so every FMA is an explicit ``fmaf``); this module wraps
it with numpy arrays and adds the vectorised byte helpers. Each function names
the reference lines (zanehpn/Actune) it restates:

* ``quantize_groups``  actune/calibration.py:7-16 and kernels/grouped.py:55-71,
  with the channel-scale division of layers.py:40-42 folded in.
* ``weight_codes``     actune/kernels/quantizers.py:4-94.
* ``pack_rows`` / ``unpack_rows``  kernels/grouped.py:67-71, 83-88, 108-111.
* ``group_dots``       kernels/grouped.py:89, grouped_native.cu:70-74.
* ``group_epilogue``   kernels/grouped.py:90-94, grouped_native.cu:75, 85.
* ``activation_dequant`` / ``reference_float_linear``  calibration.py:7-16 and
  tests/test_kernels.py:42-44 (the reference's float dequant-then-matmul).
* ``tw_*`` / ``pack_kmajor`` / ``unpack_kmajor``  the tokenwise family
  (w4a8_triton.py, w8a8_triton.py, w2a8_triton.py, wxa4_native.py).
* ``nested_r4_codes``  decode_w4a8_triton.py:61-66 (signed-R4 residual codes).

Pinning: every function is checked against known answers fixed by the
mathematics (exactly representable ties, hand-derived codes and bytes,
brute-force integer dots, exact-rational FMA cases): the group-64 functions
in ``tests/test_oracle.py``, the tokenwise ones in
``tests/test_oracle_tokenwise.py``.
"""
from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libgrouped_oracle.so"
_LIB = None

DTYPES = {"bf16": 0, "f16": 1, "f32": 2}
_P = ctypes.c_void_p
_I = ctypes.c_int64


def build() -> Path:
    """Compile the C oracle in place (gcc, via oracle/Makefile)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        so = ctypes.CDLL(str(_LIB_PATH))
        so.oracle_quantize_groups.argtypes = [_P, ctypes.c_int, _P, _I, _I, ctypes.c_int, _P, _P, _P]
        so.oracle_weight_codes.argtypes = [_P, _I, _I, ctypes.c_int, ctypes.c_int, _P, _P, _P]
        so.oracle_pack_rows.argtypes = [_P, _I, _I, ctypes.c_int, _P]
        so.oracle_unpack_rows.argtypes = [_P, _I, _I, ctypes.c_int, _P]
        so.oracle_group_dots.argtypes = [_P, _P, _I, _I, _I, _P, _I, _P, _I, _P]
        so.oracle_group_epilogue.argtypes = [_P, _P, _P, _P, _I, _P, _I, _P, _I, _P, _I, _P]
        so.oracle_round_out.argtypes = [_P, _I, ctypes.c_int, _P]
        so.oracle_round_out.restype = None
        so.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        so.oracle_f32_to_bf16.restype = ctypes.c_uint16
        so.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        so.oracle_f16_to_f32.restype = ctypes.c_float
        so.oracle_weight_codes_recip.argtypes = [_P, _I, _I, ctypes.c_int, ctypes.c_int, _P, _P, _P]
        so.oracle_tw_recip.argtypes = [ctypes.c_int]
        so.oracle_tw_recip.restype = ctypes.c_float
        so.oracle_tw_quantize_rows.argtypes = [_P, ctypes.c_int, _I, _I, ctypes.c_int, _P, _P]
        so.oracle_tw_epilogue.argtypes = [_P, _I, _I, _P, _P, _P, ctypes.c_int, _P]
        _LIB = so
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- dtype bits
def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(bits):
    """The C oracle's f16 -> f32 widening (used for f16 activations and
    channel scales), element by element."""
    b = np.asarray(bits, dtype=np.uint16).reshape(-1)
    f = lib().oracle_f16_to_f32
    return np.array([f(int(v)) for v in b], dtype=np.float32).reshape(np.shape(bits))


def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def round_out(values_f32, dtype="bf16"):
    """fp32 -> bf16/f16 bit patterns, RNE (the kernels' final cast)."""
    v = _c(values_f32, np.float32)
    if dtype == "f32":
        return v.copy()
    out = np.empty(v.shape, dtype=np.uint16)
    lib().oracle_round_out(_ptr(v), v.size, DTYPES[dtype], _ptr(out))
    return out


# ---------------------------------------------------------------- quantizer
def quantize_groups(x, A, dtype="bf16", input_scale=None):
    """Group-64 activation codes. x: [M,K] bit patterns (uint16) for bf16/f16,
    float32 for f32. Returns (packed u8 [M,K*A/8], scales f32 [M,K/64],
    codes int8 [M,K])."""
    store = np.float32 if dtype == "f32" else np.uint16
    x = _c(x, store)
    M, K = x.shape
    if A not in (2, 4, 8) or K % 64:
        raise ValueError("Unsupported activation width or unaligned input")
    sc = None if input_scale is None else _c(input_scale, store)
    packed = np.empty((M, K * A // 8), np.uint8)
    scales = np.empty((M, K // 64), np.float32)
    codes = np.empty((M, K), np.int8)
    rc = lib().oracle_quantize_groups(_ptr(x), DTYPES[dtype], _ptr(sc), M, K, A,
                                      _ptr(packed), _ptr(scales), _ptr(codes))
    if rc:
        raise ValueError("oracle_quantize_groups rejected its arguments")
    return packed, scales, codes


def activation_dequant(x_f32, A):
    """codes * scale in fp32 (calibration.activation_reference restated)."""
    x = _c(x_f32, np.float32)
    M, K = x.shape
    _, s, c = quantize_groups(x, A, dtype="f32")
    return (c.astype(np.float32).reshape(M, K // 64, 64) * s[:, :, None]).reshape(M, K)


# ---------------------------------------------------------------- weights
def validate_clip_ratios(clip_ratios, out_features):
    """quantizers.py:4-21: scalar or per-row ratios in (0, 1]."""
    ratio = np.asarray(clip_ratios, dtype=np.float32).reshape(-1)
    if ratio.size == 1:
        ratio = np.full(out_features, ratio[0], np.float32)
    if ratio.size != out_features:
        raise ValueError(f"expected {out_features} AWQ-style clip ratios, got {ratio.size}")
    if not np.isfinite(ratio).all():
        raise ValueError("AWQ-style clip ratios must be finite")
    if bool(((ratio <= 0.0) | (ratio > 1.0)).any()):
        raise ValueError("AWQ-style clip ratios must lie in (0, 1]")
    return np.ascontiguousarray(ratio)


def weight_codes(w_f32, W, A, clip_ratios=None, gpu_division=False):
    """Per-row weight codebook (quantizers.py:83-94) on the fp32 weight image.
    gpu_division: the divisions by the constants 7 and 127 as torch performs
    them on a GPU-resident weight (multiply by the fp32 reciprocal) instead of
    the IEEE quotient torch-CPU computes. Returns (codes int8 [N,K], scale f32 [N])."""
    w = _c(w_f32, np.float32)
    N, K = w.shape
    ratios = None
    if clip_ratios is not None and not (W == 8 and A != 4):
        ratios = validate_clip_ratios(clip_ratios, N)
    codes = np.empty((N, K), np.int8)
    scale = np.empty(N, np.float32)
    fn = lib().oracle_weight_codes_recip if gpu_division else lib().oracle_weight_codes
    if fn(_ptr(w), N, K, W, A, _ptr(ratios), _ptr(codes), _ptr(scale)):
        raise ValueError("Unsupported integer width")
    return codes, scale


# ---------------------------------------------------------------- packing
def pack_rows(codes, bits):
    c = _c(codes, np.int8)
    R, K = c.shape
    out = np.empty((R, K * bits // 8), np.uint8)
    if lib().oracle_pack_rows(_ptr(c), R, K, bits, _ptr(out)):
        raise ValueError("bad packing width")
    return out


def unpack_rows(packed, bits, K):
    p = _c(packed, np.uint8)
    R = p.shape[0]
    out = np.empty((R, K), np.int8)
    if lib().oracle_unpack_rows(_ptr(p), R, K, bits, _ptr(out)):
        raise ValueError("bad packing width")
    return out


# ---------------------------------------------------------------- GEMM
def group_dots(a_codes, w_codes, rows=None, cols=None):
    """Exact int32 dots [len(rows), len(cols), G]."""
    a = _c(a_codes, np.int8)
    w = _c(w_codes, np.int8)
    M, K = a.shape
    N = w.shape[0]
    r = None if rows is None else _c(rows, np.int64)
    c = None if cols is None else _c(cols, np.int64)
    nr = M if r is None else r.size
    nc = N if c is None else c.size
    out = np.empty((nr, nc, K // 64), np.int32)
    if lib().oracle_group_dots(_ptr(a), _ptr(w), M, N, K, _ptr(r), nr, _ptr(c), nc, _ptr(out)):
        raise ValueError("K must be a multiple of 64")
    return out


def group_epilogue(dots, a_scales, w_scale, bias=None, rows=None, cols=None, bounds=None):
    """fp32 epilogue with the given chunk bounds (None = sequential)."""
    d = _c(dots, np.int32)
    nr, nc, G = d.shape
    s = _c(a_scales, np.float32)
    ws = _c(w_scale, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    r = None if rows is None else _c(rows, np.int64)
    c = None if cols is None else _c(cols, np.int64)
    bd = None if bounds is None else _c(bounds, np.int64)
    out = np.empty((nr, nc), np.float32)
    rc = lib().oracle_group_epilogue(_ptr(d), _ptr(s), _ptr(ws), _ptr(b), G, _ptr(r), nr, _ptr(c), nc,
                                     _ptr(bd), 0 if bd is None else bd.size - 1, _ptr(out))
    if rc:
        raise ValueError("bad reduction bounds")
    return out


def linear(a_codes, a_scales, w_codes, w_scale, bias=None, bounds=None, rows=None, cols=None):
    """fp32 output of the grouped linear in the given reduction order."""
    d = group_dots(a_codes, w_codes, rows, cols)
    return group_epilogue(d, a_scales, w_scale, bias, rows, cols, bounds)


def reference_float_linear(x_f32, A, w_codes, w_scale, bias=None):
    """The reference test's float criterion (tests/test_kernels.py:42-44):
    F.linear(activation_reference(x, A), q.float() * scale[:, None], bias)."""
    xq = activation_dequant(x_f32, A).astype(np.float64)
    wf = (w_codes.astype(np.float32) * _c(w_scale, np.float32)[:, None]).astype(np.float64)
    y = xq @ wf.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y.astype(np.float32)


# ---------------------------------------------------------------- orders
def chunk_bounds(G, steps_groups, chunks):
    """Group boundaries of ``chunks`` contiguous K-chunks made of whole steps
    of ``steps_groups`` groups: chunk c covers steps
    [floor(c*S/chunks), floor((c+1)*S/chunks)), S = ceil(G/steps_groups),
    clipped to G. Empty chunks are kept (they contribute +0)."""
    S = math.ceil(G / steps_groups)
    b = [min(G, (c * S // chunks) * steps_groups) for c in range(chunks)] + [G]
    return np.asarray(b, np.int64)


# ---------------------------------------------------------------- tokenwise family
# Per-row (tokenwise) quantization with full-K int32 accumulation:
# actune/kernels/w4a8_triton.py, w8a8_triton.py, w2a8_triton.py,
# decode_w4a8_triton.py and wxa4_native.py (arithmetic in tokenwise_oracle.c).

def tw_recip(p):
    """The fp32 reciprocal 1/p the reference's per-row quantizers multiply by."""
    return np.float32(lib().oracle_tw_recip(int(p)))


def tw_quantize_rows(x, bits, dtype="bf16"):
    """Per-row dynamic A8 (bits 8) or A4 (bits 4) codes and scales
    (w4a8_triton.py:161-201, wxa4_native.py:28-65). x: [M, K] bit patterns
    (uint16) for bf16/f16, float32 for f32. Returns (codes int8 [M, K],
    scales f32 [M])."""
    store = np.float32 if dtype == "f32" else np.uint16
    x = _c(x, store)
    M, K = x.shape
    codes = np.empty((M, K), np.int8)
    scales = np.empty(M, np.float32)
    if lib().oracle_tw_quantize_rows(_ptr(x), DTYPES[dtype], M, K, bits, _ptr(codes), _ptr(scales)):
        raise ValueError("bad per-row quantizer arguments")
    return codes, scales


def tw_dots(a_codes, w_codes):
    """Exact full-K int32 dots acc[m, n] = sum_k a[m, k] * w[n, k] (int64
    brute force, checked to fit int32)."""
    acc = a_codes.astype(np.int64) @ w_codes.astype(np.int64).T
    if np.abs(acc).max(initial=0) >= 2**31:
        raise OverflowError("accumulator exceeds int32")
    return acc.astype(np.int32)


def tw_epilogue(acc, a_scales, w_scale, bias=None, mode=0):
    """fp32 output from int32 accumulators: mode 0 = the A8 family's
    (acc * as) * ws (+ bias), mode 1 = the native A4 kernels' acc * (as * ws)
    (+ bias); see tokenwise_oracle.c."""
    acc = _c(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    if lib().oracle_tw_epilogue(_ptr(acc), M, N, _ptr(_c(a_scales, np.float32)), _ptr(_c(w_scale, np.float32)),
                                _ptr(b), mode, _ptr(out)):
        raise ValueError("bad epilogue mode")
    return out


def pack_kmajor(codes, bits):
    """The tokenwise family's K-major weight layouts (int8 codes [N, K]):
    bits 8: int8 [K, N] (w8a8_triton.py:106, wxa4_native.py:334);
    bits 4: u8 [K/2, N], byte j of column n = code j (low nibble) and code
            j + K/2 (high nibble) (w4a8_triton.py:380-383);
    bits 2: u8 [K/4, N], byte j = codes j, j + K/4, j + K/2, j + 3K/4 at bits
            0, 2, 4, 6 (w2a8_triton.py:149-159)."""
    c = _c(codes, np.int8)
    N, K = c.shape
    if bits == 8:
        return np.ascontiguousarray(c.T)
    per = 8 // bits
    part = K // per
    fields = [(c[:, i * part:(i + 1) * part].astype(np.int16) & ((1 << bits) - 1)) << (i * bits)
              for i in range(per)]
    packed = np.zeros((N, part), np.int16)
    for f in fields:
        packed |= f
    return np.ascontiguousarray(packed.astype(np.uint8).T)


def nested_r4_codes(q4, r4):
    """The W4R4 decode's int8 weight codes from signed q4 and r4 codes (each
    int8 in [-8, 7], any shape): 16 q4 + r4 formed in int16 and narrowed to
    8 bits by two's-complement wrap (decode_w4a8_triton.py:61-66), so the
    pair (-8, r < 0) wraps to 128 + r. The matching epilogue is mode 0 with
    the weight scale divided by 16 (:103-104)."""
    q = _c(q4, np.int8).astype(np.int16)
    r = _c(r4, np.int8).astype(np.int16)
    if q.shape != r.shape or q.min(initial=0) < -8 or q.max(initial=0) > 7 or r.min(initial=0) < -8 \
            or r.max(initial=0) > 7:
        raise ValueError("q4 and r4 are signed 4-bit codes of one shape")
    return (q * 16 + r).astype(np.uint16).astype(np.uint8).view(np.int8)


def unpack_kmajor(packed, bits, K):
    """Inverse of pack_kmajor: int8 codes [N, K]."""
    p = _c(packed, np.uint8 if bits != 8 else np.int8)
    if bits == 8:
        return np.ascontiguousarray(p.T.astype(np.int8))
    per = 8 // bits
    half = 1 << (bits - 1)
    cols = []
    for i in range(per):
        u = ((p.T.astype(np.int16) >> (i * bits)) & ((1 << bits) - 1))
        cols.append(((u ^ half) - half).astype(np.int8))
    return np.ascontiguousarray(np.concatenate(cols, axis=1))
