"""ctypes binding of libactune_hip.so (include/actune_hip.h).

The library is the only compute path of this package: there is no Python or
CPU fallback. Loading fails loudly when the library is missing, and every
call raises on a non-zero status with the library's error message.

The wrappers take torch tensors (device memory and the current stream come
from PyTorch-ROCm) and reproduce the reference's argument checks and
messages (actune/kernels/grouped_native.cu:92-105, grouped.py:118-119, 128).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libactune_hip.so"
_LIB = None

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
CONFIG_AUTO = -1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
MAX_TARGETS = 4


class _Target(ctypes.Structure):
    """actune_linear_target"""
    _fields_ = [("w", _P), ("w_scale", _P), ("bias", _P), ("out", _P), ("N", _I64), ("W", ctypes.c_int32)]


class _TwTarget(ctypes.Structure):
    """actune_tw_target"""
    _fields_ = [("w", _P), ("r", _P), ("w_scale", _P), ("bias", _P), ("out", _P)]


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m actune_amd.build` "
                "(the group-64 backend has no fallback path)")
        so = ctypes.CDLL(str(LIB_PATH))
        so.actune_version.restype = ctypes.c_char_p
        so.actune_last_error.restype = ctypes.c_char_p
        so.actune_quantize_groups.argtypes = [_P, _I, _P, _I64, _I64, _I, _P, _P, _P]
        so.actune_quantize_gated.argtypes = [_P, _P, _I, _I, _P, _I64, _I64, _I, _P, _P, _P]
        so.actune_grouped_linear.argtypes = [_P, _P, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I, _I, _I, _P]
        so.actune_grouped_forward.argtypes = [_P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64,
                                              _I, _I, _I, _P]
        so.actune_grouped_forward_multi.argtypes = [_P, _I, _P, _P, _P, ctypes.POINTER(_Target), _I, _I,
                                                    _I64, _I64, _I, _I, _I, _P]
        so.actune_grouped_dots_i32.argtypes = [_P, _P, _I64, _I64, _I64, _I, _I, _I, _P, _P]
        so.actune_tokenwise_quantize.argtypes = [_P, _I, _I64, _I64, _I, _P, _P, _P]
        so.actune_tokenwise_workspace_bytes.argtypes = [_I64, _I64, _I64, _I, _I]
        so.actune_tokenwise_workspace_bytes.restype = _I64
        so.actune_tokenwise_linear.argtypes = [_P, _I, _P, _P, _I, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I, _P,
                                               _I64, _P]
        so.actune_tokenwise_linear_x.argtypes = [_P, _I, _P, _P, _I, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I,
                                                 _P, _I64, _P]
        so.actune_tokenwise_linear_multi.argtypes = [_P, _I, _P, _I, _P, _I, ctypes.POINTER(_TwTarget), _I, _I, _I,
                                                     _I64, _I64, _I64, _I, _P, _I64, _P]
        so.actune_forward_fuses_quantizer.argtypes = [_I64, _I64, _I64, _I, _I, _I, _I]
        so.actune_config_valid.argtypes = [_I, _I64]
        so.actune_default_config.argtypes = [_I64, _I64, _I64, _I, _I]
        _LIB = so
    return _LIB


def _check(rc: int) -> None:
    if rc:
        msg = lib().actune_last_error().decode()
        raise RuntimeError(msg) if rc == 2 else ValueError(msg)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_HIP = None


def capture_id(device=None) -> int:
    """Id of the stream capture the current stream of `device` is recording
    (hipStreamGetCaptureInfo), 0 when it records none. Caches of device
    tensors use it so that a captured launch never reads a tensor written
    outside its graph, nor an eager call one written only at replay."""
    global _HIP
    if not torch.cuda.is_current_stream_capturing():
        return 0
    if _HIP is None:
        # resolved through the library's handle: the HIP runtime it (and
        # torch) run on, not a second copy
        fn = lib().hipStreamGetCaptureInfo
        fn.argtypes = [_P, ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_ulonglong)]
        _HIP = fn
    status, ident = _I(0), ctypes.c_ulonglong(0)
    rc = _HIP(_stream(device), ctypes.byref(status), ctypes.byref(ident))
    if rc != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed ({rc})")
    return int(ident.value) if status.value == 1 else 0


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype not in DTYPE_CODES:
        raise ValueError(f"unsupported dtype {t.dtype}")
    return DTYPE_CODES[t.dtype]


def _bias_code(bias) -> int:
    """dtype code of a bias (2 when there is none); the reference op accepts
    floating biases only (grouped_native.cu:97)."""
    if bias is None:
        return 2
    if bias.dtype not in DTYPE_CODES:
        raise RuntimeError("float scales/bias required")
    return DTYPE_CODES[bias.dtype]


def _check_buffer(t, name, shape, dtype, device):
    """A caller-supplied buffer must be a contiguous tensor of exactly this
    shape and dtype on the operation's device: the C ABI takes raw pointers
    and cannot check sizes itself."""
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise RuntimeError(f"{name} must be a contiguous {list(shape)} tensor, got {list(t.shape)}")


def _check_weights(w, ws, bias, k, W):
    """Packed weights u8 [N, K*W/8], float32 scale [N], optional bias [N]."""
    if w.dtype != torch.uint8:
        raise RuntimeError("packed uint8 required")
    if ws.dtype != torch.float32:
        raise RuntimeError("float scales/bias required")
    if w.dim() != 2 or w.size(1) != k * W // 8:
        raise RuntimeError("packed shape mismatch")
    if not (w.is_contiguous() and ws.is_contiguous() and (bias is None or bias.is_contiguous())):
        raise RuntimeError("contiguous operands required")
    n = w.size(0)
    if ws.numel() != n:
        raise RuntimeError("scale shape mismatch")
    if bias is not None and bias.numel() != n:
        raise RuntimeError("bias shape mismatch")
    _bias_code(bias)
    return n


def _check_widths(W, A):
    if W not in (2, 4, 8) or A not in (2, 4, 8):
        raise ValueError("Unsupported integer width")


def _check_flat(flat):
    if flat.dim() != 2 or not flat.is_contiguous():
        raise RuntimeError("contiguous [M, K] input required")
    _dtype_code(flat)


def _aligned16(t):
    """t itself when its data is 16-byte aligned (the kernels read rows with
    16-byte loads), else an aligned copy: a contiguous view at an odd offset
    (x[:, 1:].reshape(...) style) computes as the reference does."""
    if t is None or t.data_ptr() % 16 == 0:
        return t
    return t.clone()


def version() -> str:
    return lib().actune_version().decode()


def num_configs() -> int:
    return lib().actune_num_configs()


def config_valid(config: int, m: int) -> bool:
    return bool(lib().actune_config_valid(config, m))


def default_config(m: int, n: int, k: int, w: int, a: int) -> int:
    return lib().actune_default_config(m, n, k, w, a)


def forward_fuses_quantizer(m, n, k, w, a, dtype, config=CONFIG_AUTO) -> bool:
    """Whether grouped_forward quantizes x inside its GEMM launch."""
    rc = lib().actune_forward_fuses_quantizer(m, n, k, w, a, DTYPE_CODES[dtype], config)
    if rc < 0:
        raise ValueError(lib().actune_last_error().decode())
    return bool(rc)


def _require_cuda(*tensors):
    if not all(t.is_cuda for t in tensors if t is not None):
        raise RuntimeError("CUDA required")
    dev = tensors[0].device
    if any(t is not None and t.device != dev for t in tensors):
        raise RuntimeError("device mismatch")


def _check_input_scale(input_scale, x):
    if input_scale is not None and (input_scale.dtype != x.dtype or input_scale.numel() != x.shape[-1]
                                    or not input_scale.is_contiguous()):
        raise RuntimeError("input_scale must be a contiguous [K] tensor of the input dtype")


def _act_buffers(packed, scales, m, k, a, device):
    """Packed activations u8 [M, K*A/8] and scales f32 [M, K/64]: allocated
    here, or checked when the caller passes them."""
    if packed is None:
        packed = torch.empty((m, k * a // 8), device=device, dtype=torch.uint8)
    if scales is None:
        scales = torch.empty((m, k // 64), device=device, dtype=torch.float32)
    _check_buffer(packed, "packed", (m, k * a // 8), torch.uint8, device)
    _check_buffer(scales, "scales", (m, k // 64), torch.float32, device)
    return packed, scales


def quantize_groups(x: torch.Tensor, a: int, input_scale: torch.Tensor | None = None,
                    packed: torch.Tensor | None = None, scales: torch.Tensor | None = None):
    """Group-64 quantize a contiguous [M, K] tensor; returns (packed, scales)."""
    _require_cuda(x, input_scale, packed, scales)
    _check_widths(8, a)
    _check_flat(x)
    m, k = x.shape
    _check_input_scale(input_scale, x)
    x, input_scale = _aligned16(x), _aligned16(input_scale)
    packed, scales = _act_buffers(packed, scales, m, k, a, x.device)
    _check(lib().actune_quantize_groups(_ptr(x), _dtype_code(x), _ptr(input_scale), m, k, a,
                                        _ptr(packed), _ptr(scales), _stream(x.device)))
    return packed, scales


ACT_SILU, ACT_GELU_TANH = 0, 1


def quantize_gated(gate: torch.Tensor, up: torch.Tensor, act: int, a: int, input_scale: torch.Tensor | None = None,
                   packed: torch.Tensor | None = None, scales: torch.Tensor | None = None):
    """Group-64 codes of p = act(gate) * up (ACT_SILU or ACT_GELU_TANH, p
    formed in the inputs' dtype as torch forms it) through
    actune_quantize_gated: equal to quantize_groups on a tensor holding p.
    gate, up: contiguous [M, K] of one dtype. Returns (packed, scales)."""
    _require_cuda(gate, up, input_scale, packed, scales)
    _check_widths(8, a)
    _check_flat(gate)
    if up.shape != gate.shape or up.dtype != gate.dtype or not up.is_contiguous():
        raise RuntimeError("up must match gate (contiguous [M, K], same dtype)")
    if act not in (ACT_SILU, ACT_GELU_TANH):
        raise ValueError("unknown gate activation")
    m, k = gate.shape
    _check_input_scale(input_scale, gate)
    gate, up, input_scale = _aligned16(gate), _aligned16(up), _aligned16(input_scale)
    packed, scales = _act_buffers(packed, scales, m, k, a, gate.device)
    _check(lib().actune_quantize_gated(_ptr(gate), _ptr(up), _dtype_code(gate), act, _ptr(input_scale), m, k, a,
                                       _ptr(packed), _ptr(scales), _stream(gate.device)))
    return packed, scales


def _check_linear_operands(a, as_, w, ws, bias, m, k, n, W, A):
    if a.dtype != torch.uint8 or w.dtype != torch.uint8:
        raise RuntimeError("packed uint8 required")
    if as_.dtype != torch.float32 or ws.dtype != torch.float32:
        raise RuntimeError("float scales/bias required")
    if not (a.is_contiguous() and as_.is_contiguous() and w.is_contiguous() and ws.is_contiguous()
            and (bias is None or bias.is_contiguous())):
        raise RuntimeError("contiguous operands required")
    if a.dim() != 2 or w.dim() != 2 or as_.dim() != 2:
        raise RuntimeError("rank mismatch")
    if not (m >= 0 and n > 0 and k > 0 and k % 64 == 0):
        raise RuntimeError("invalid dimensions")
    if a.size(0) != m or a.size(1) != k * A // 8 or w.size(1) != k * W // 8:
        raise RuntimeError("packed shape mismatch")
    if as_.size(0) != m or as_.size(1) != k // 64 or ws.numel() != n:
        raise RuntimeError("scale shape mismatch")
    if bias is not None and bias.numel() not in (0, n):
        raise RuntimeError("bias shape mismatch")


def grouped_linear(a, as_, w, ws, bias, source_or_shape, W, A, config=CONFIG_AUTO, out=None,
                   out_dtype=None):
    """The native op of grouped_native.cu:90-115 / grouped_big_m.cu:92-135:
    packed activations + scales x packed weights -> [M, N] in source.dtype.
    ``source_or_shape`` is the [M, K] source tensor (its dtype and shape
    define the output), as in the reference op signature."""
    _require_cuda(a, as_, w, ws, bias)
    if isinstance(source_or_shape, torch.Tensor):
        m, k = source_or_shape.shape
        dtype = source_or_shape.dtype
    else:
        m, k = source_or_shape
        dtype = out_dtype or torch.bfloat16
    n = w.size(0)
    if W not in (2, 4, 8) or A not in (2, 4, 8):
        raise ValueError("Unsupported integer width")
    _check_linear_operands(a, as_, w, ws, bias, m, k, n, W, A)
    if bias is not None and bias.numel() == 0:
        bias = None
    bias_dt = _bias_code(bias)
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=dtype)
    _check_buffer(out, "out", (m, n), dtype, a.device)
    _check(lib().actune_grouped_linear(
        _ptr(a), _ptr(as_), _ptr(w), _ptr(ws), _ptr(bias), bias_dt,
        _ptr(out), _dtype_code(out), m, n, k, W, A, config, _stream(a.device)))
    return out


def grouped_forward(flat, w, ws, bias, W, A, input_scale=None, config=CONFIG_AUTO, out=None,
                    packed=None, scales=None):
    """Quantize + GEMM for a contiguous [M, K] input (GroupedLinear.forward's
    device work, grouped.py:127-143); returns [M, N] in flat.dtype.
    packed [M, K*A/8] / scales [M, K/64] / out may be preallocated."""
    _require_cuda(flat, w, ws, bias, input_scale, out, packed, scales)
    _check_widths(W, A)
    _check_flat(flat)
    m, k = flat.shape
    n = _check_weights(w, ws, bias, k, W)
    _check_input_scale(input_scale, flat)
    flat, input_scale = _aligned16(flat), _aligned16(input_scale)
    packed, scales = _act_buffers(packed, scales, m, k, A, flat.device)
    if out is None:
        out = torch.empty((m, n), device=flat.device, dtype=flat.dtype)
    _check_buffer(out, "out", (m, n), flat.dtype, flat.device)
    bias_dt = _bias_code(bias)
    _check(lib().actune_grouped_forward(
        _ptr(flat), _dtype_code(flat), _ptr(input_scale), _ptr(packed), _ptr(scales), _ptr(w), _ptr(ws),
        _ptr(bias), bias_dt, _ptr(out), m, n, k, W, A, config, _stream(flat.device)))
    return out


def grouped_forward_multi(flat, targets, W, A, input_scale=None, config=CONFIG_AUTO, packed=None,
                          scales=None):
    """Quantize + GEMM of one [M, K] input against up to 4 linears in one
    launch. targets: sequence of (w, ws, bias, out) with out [M, N_t] (None
    to allocate), or (w, ws, bias, out, W_t) for a target whose weight width
    W_t differs from W (the call then runs the widths in one decode launch
    where the kernel takes them, else one launch per width on one
    quantization). Returns the list of outputs."""
    if not 1 <= len(targets) <= MAX_TARGETS:
        raise ValueError("between 1 and 4 targets required")
    _require_cuda(flat, input_scale, packed, scales, *[t for tgt in targets for t in tgt[:4]])
    _check_widths(W, A)
    _check_flat(flat)
    m, k = flat.shape
    _check_input_scale(input_scale, flat)
    flat, input_scale = _aligned16(flat), _aligned16(input_scale)
    biases = [t[2] for t in targets]
    if len({(b.dtype if b is not None else None) for b in biases}) != 1:
        raise ValueError("all targets must share one bias dtype (or none)")
    bias_dt = _bias_code(biases[0])
    arr = (_Target * len(targets))()
    outs = []
    for j, tgt in enumerate(targets):
        w, ws, bias, out = tgt[:4]
        wt = tgt[4] if len(tgt) > 4 else W
        _check_widths(wt, A)
        n = _check_weights(w, ws, bias, k, wt)
        if out is None:
            out = torch.empty((m, n), device=flat.device, dtype=flat.dtype)
        _check_buffer(out, f"out[{j}]", (m, n), flat.dtype, flat.device)
        outs.append(out)
        arr[j] = _Target(w.data_ptr(), ws.data_ptr(), None if bias is None else bias.data_ptr(), out.data_ptr(), n,
                         wt)
    packed, scales = _act_buffers(packed, scales, m, k, A, flat.device)
    _check(lib().actune_grouped_forward_multi(_ptr(flat), _dtype_code(flat), _ptr(input_scale), _ptr(packed),
                                              _ptr(scales), arr, len(targets), bias_dt, m, k, W, A, config,
                                              _stream(flat.device)))
    return outs


def grouped_dots(a, w, m, k, W, A, config=CONFIG_AUTO):
    """Exact int32 per-group dots [M, N, K/64] through kernel ``config``."""
    _require_cuda(a, w)
    n = w.size(0)
    dots = torch.empty((m, n, k // 64), device=a.device, dtype=torch.int32)
    _check(lib().actune_grouped_dots_i32(_ptr(a), _ptr(w), m, n, k, W, A, config, _ptr(dots),
                                         _stream(a.device)))
    return dots


class Extension:
    """Object form of the reference's JIT extension (grouped.py:97-105): its
    ``linear`` has the reference op signature plus an optional config."""

    @staticmethod
    def linear(a, as_, w, ws, bias, source, W, A, config=CONFIG_AUTO):
        return grouped_linear(a, as_, w, ws, bias, source, W, A, config)


def extension() -> Extension:
    lib()
    return Extension()


# ---------------------------------------------------------------- tokenwise family
TW_KMAJOR_W8, TW_KMAJOR_W4, TW_KMAJOR_W2, TW_ROWS_S4, TW_ROWS_S2, TW_KMAJOR_W4R4 = 0, 1, 2, 3, 4, 5
TW_ACT_A8, TW_ACT_A4 = 0, 1
TW_EPI_A8, TW_EPI_A4 = 0, 1


def tokenwise_quantize(x, bits, codes=None, scales=None):
    """Per-row dynamic A8 (int8 [M, K]) or A4 (packed u8 [M, K/2]) codes and
    f32 [M] scales of a contiguous [M, K] tensor."""
    _require_cuda(x, codes, scales)
    _check_flat(x)
    if bits not in (8, 4):
        raise ValueError("tokenwise activations are A8 or A4")
    x = _aligned16(x)
    m, k = x.shape
    if codes is None:
        codes = torch.empty((m, k) if bits == 8 else (m, k // 2), device=x.device,
                            dtype=torch.int8 if bits == 8 else torch.uint8)
    if scales is None:
        scales = torch.empty(m, device=x.device, dtype=torch.float32)
    _check_buffer(codes, "codes", (m, k) if bits == 8 else (m, k // 2), torch.int8 if bits == 8 else torch.uint8,
                  x.device)
    _check_buffer(scales, "scales", (m,), torch.float32, x.device)
    _check(lib().actune_tokenwise_quantize(_ptr(x), _dtype_code(x), m, k, bits, _ptr(codes), _ptr(scales),
                                           _stream(x.device)))
    return codes, scales


def tokenwise_workspace_bytes(m, n, k, w_layout, a_layout):
    need = lib().actune_tokenwise_workspace_bytes(m, n, k, w_layout, a_layout)
    if need < 0:
        raise ValueError(lib().actune_last_error().decode())
    return need


def tokenwise_fused_max_k(m):
    """Longest row actune_tokenwise_linear_x quantizes for m rows (one row:
    16384; 2, 3-4, 5-8 rows: 16384, 8192, 4096), 0 past 8 rows."""
    if m == 1:
        return 16384
    if not 1 < m <= 8:
        return 0
    return 16 * 8 * (256 // (2 if m <= 2 else 4 if m <= 4 else 8))


def tokenwise_linear_x(x, as_out, w, w_layout, ws, bias, n, k, epilogue, out, workspace=None):
    """Rows of x ([M, K], M = 1..8; bf16 / f16, or f32 for one row) quantized
    to A8 inside the GEMM launch (actune_tokenwise_linear_x): the result of
    tokenwise_quantize(x, 8) followed by tokenwise_linear on its codes, bit
    for bit. as_out: float32 [M], receives the rows' activation scales; w: a
    K-major layout; workspace as for tokenwise_linear with A8 activations."""
    _require_cuda(x, as_out, w, ws, bias, out, workspace)
    if x.dim() != 2 or not 1 <= x.shape[0] <= 8 or x.shape[1] != k:
        raise RuntimeError("fused quantization takes x of shape [M, K] with M <= 8")
    m = x.shape[0]
    if not (x.is_contiguous() and w.is_contiguous() and ws.is_contiguous()
            and (bias is None or bias.is_contiguous())):
        raise RuntimeError("contiguous operands required")
    x = _aligned16(x)
    if as_out.dtype != torch.float32 or ws.dtype != torch.float32:
        raise RuntimeError("float scales/bias required")
    if as_out.numel() != m or not as_out.is_contiguous() or ws.numel() != n or (bias is not None and bias.numel() != n):
        raise RuntimeError("scale shape mismatch")
    wbytes = {TW_KMAJOR_W8: k * n, TW_KMAJOR_W4: k // 2 * n, TW_KMAJOR_W2: k // 4 * n,
              TW_KMAJOR_W4R4: k // 2 * n}.get(w_layout)
    if wbytes is None:
        raise RuntimeError("fused quantization takes the K-major (A8) weight layouts")
    if w.numel() != wbytes or w.element_size() != 1:
        raise RuntimeError("packed weight shape mismatch")
    _check_buffer(out, "out", (m, n), out.dtype, x.device)
    need = tokenwise_workspace_bytes(m, n, k, w_layout, TW_ACT_A8)
    if need and (workspace is None or workspace.numel() < need or workspace.dtype != torch.uint8):
        raise RuntimeError(f"workspace of at least {need} bytes required")
    _check(lib().actune_tokenwise_linear_x(
        _ptr(x), _dtype_code(x), _ptr(as_out), _ptr(w), w_layout, _ptr(ws), _ptr(bias), _bias_code(bias), _ptr(out),
        _dtype_code(out), m, n, k, epilogue, _ptr(workspace) if need else None, need, _stream(x.device)))
    return out


def tokenwise_linear(a, a_layout, as_, w, w_layout, ws, bias, n, k, epilogue, out, workspace=None):
    """out[m, n] = epilogue(exact int32 sum_k a[m, k] w[n, k]) through
    actune_tokenwise_linear. a: int8 [M, K] (A8) or u8 [M, K/2] (A4); w in
    layout w_layout; out: preallocated [M, N]; workspace: u8 tensor of at
    least tokenwise_workspace_bytes() bytes (None when that is 0)."""
    _require_cuda(a, as_, w, ws, bias, out, workspace)
    m = a.shape[0]
    if not (a.is_contiguous() and as_.is_contiguous() and w.is_contiguous() and ws.is_contiguous()
            and (bias is None or bias.is_contiguous())):
        raise RuntimeError("contiguous operands required")
    if as_.dtype != torch.float32 or ws.dtype != torch.float32:
        raise RuntimeError("float scales/bias required")
    if as_.numel() != m or ws.numel() != n or (bias is not None and bias.numel() != n):
        raise RuntimeError("scale shape mismatch")
    abytes = k if a_layout == TW_ACT_A8 else k // 2
    if a.dim() != 2 or a.shape[1] != abytes or a.element_size() != 1:
        raise RuntimeError("packed activation shape mismatch")
    wbytes = {TW_KMAJOR_W8: k * n, TW_KMAJOR_W4: k // 2 * n, TW_KMAJOR_W2: k // 4 * n,
              TW_ROWS_S4: n * k // 2, TW_ROWS_S2: n * k // 4, TW_KMAJOR_W4R4: k // 2 * n}[w_layout]
    if w.numel() != wbytes or w.element_size() != 1:
        raise RuntimeError("packed weight shape mismatch")
    _check_buffer(out, "out", (m, n), out.dtype, a.device)
    need = tokenwise_workspace_bytes(m, n, k, w_layout, a_layout)
    if need and (workspace is None or workspace.numel() < need or workspace.dtype != torch.uint8):
        raise RuntimeError(f"workspace of at least {need} bytes required")
    _check(lib().actune_tokenwise_linear(
        _ptr(a), a_layout, _ptr(as_), _ptr(w), w_layout, _ptr(ws), _ptr(bias), _bias_code(bias), _ptr(out),
        _dtype_code(out), m, n, k, epilogue, _ptr(workspace) if need else None, need, _stream(a.device)))
    return out


def tokenwise_linear_multi(targets, w_layout, n, k, epilogue, scales, *, codes=None, a_layout=TW_ACT_A8, x=None,
                           workspace=None, residuals=None):
    """1 to MAX_TARGETS sibling projections on the same rows in one GEMM
    launch (and one reduce when K is split): actune_tokenwise_linear_multi.
    targets: [(w, ws, bias, out)] sharing n, k and w_layout, out [M, N]
    preallocated; each bias may be None, those present share one dtype.
    Pass either codes (in a_layout; scales [M] read) or x (rows [M, K]
    quantized to A8 in the launch; scales [M] written).
    residuals: with TW_KMAJOR_W4R4 only, one entry per target, each a u8
    [K/2, N] residual in the KMAJOR_W4 packing or None (that target reads
    r4 = 0, its result equals TW_KMAJOR_W4's).
    workspace: u8 tensor of at least len(targets) x tokenwise_workspace_bytes()
    bytes (None when that is 0). Each output equals the single-target call."""
    if (codes is None) == (x is None):
        raise ValueError("pass either codes or x")
    if not 1 <= len(targets) <= MAX_TARGETS:
        raise ValueError(f"1 to {MAX_TARGETS} targets")
    if w_layout == TW_KMAJOR_W4R4:
        residuals = [None] * len(targets) if residuals is None else list(residuals)
        if len(residuals) != len(targets):
            raise ValueError("one residual (or None) per target")
    elif residuals is not None and any(r is not None for r in residuals):
        raise ValueError("residuals go with the TW_KMAJOR_W4R4 layout only")
    else:
        residuals = [None] * len(targets)
    act = codes if codes is not None else x
    _require_cuda(act, scales, workspace, *[t for tgt in targets for t in tgt], *residuals)
    if x is not None:
        a_layout = TW_ACT_A8
        if x.dim() != 2 or not 1 <= x.shape[0] <= 8 or x.shape[1] != k or not x.is_contiguous():
            raise RuntimeError("fused quantization takes contiguous x of shape [M, K] with M <= 8")
        _dtype_code(x)
        x = act = _aligned16(x)
    else:
        abytes = k if a_layout == TW_ACT_A8 else k // 2
        if codes.dim() != 2 or codes.shape[1] != abytes or codes.element_size() != 1 or not codes.is_contiguous():
            raise RuntimeError("packed activation shape mismatch")
    m = act.shape[0]
    if scales.dtype != torch.float32 or scales.numel() != m or not scales.is_contiguous():
        raise RuntimeError("scale shape mismatch")
    wbytes = {TW_KMAJOR_W8: k * n, TW_KMAJOR_W4: k // 2 * n, TW_KMAJOR_W2: k // 4 * n,
              TW_ROWS_S4: n * k // 2, TW_ROWS_S2: n * k // 4, TW_KMAJOR_W4R4: k // 2 * n}[w_layout]
    out_dtype = targets[0][3].dtype
    present = [t[2] for t in targets if t[2] is not None]
    bias0 = present[0] if present else None
    structs = (_TwTarget * len(targets))()
    for r in residuals:
        if r is not None and (not r.is_contiguous() or r.numel() != wbytes or r.element_size() != 1):
            raise RuntimeError("packed residual shape mismatch (contiguous u8 [K/2, N] required)")
    residuals = [_aligned16(r) for r in residuals]  # held until the launch is issued
    for i, ((w, ws, bias, out), r) in enumerate(zip(targets, residuals)):
        if not (w.is_contiguous() and ws.is_contiguous() and (bias is None or bias.is_contiguous())):
            raise RuntimeError("contiguous operands required")
        if w.numel() != wbytes or w.element_size() != 1:
            raise RuntimeError("packed weight shape mismatch")
        if ws.dtype != torch.float32 or ws.numel() != n or (bias is not None and bias.numel() != n):
            raise RuntimeError("scale shape mismatch")
        if bias is not None and bias.dtype != bias0.dtype:
            raise RuntimeError("the sibling biases present must share one dtype")
        _check_buffer(out, "out", (m, n), out_dtype, act.device)
        structs[i] = _TwTarget(w.data_ptr(), None if r is None else r.data_ptr(), ws.data_ptr(),
                               None if bias is None else bias.data_ptr(), out.data_ptr())
    need = len(targets) * tokenwise_workspace_bytes(m, n, k, w_layout, a_layout)
    if need and (workspace is None or workspace.numel() < need or workspace.dtype != torch.uint8):
        raise RuntimeError(f"workspace of at least {need} bytes required")
    _check(lib().actune_tokenwise_linear_multi(
        _ptr(codes), a_layout, _ptr(x), _dtype_code(x) if x is not None else 0, _ptr(scales), w_layout, structs,
        len(targets), _bias_code(bias0), _dtype_code(targets[0][3]), m, n, k, epilogue,
        _ptr(workspace) if need else None, need, _stream(act.device)))
    return [t[3] for t in targets]

