"""GPU parity of the tokenwise family against the CPU oracle, through the
C ABI (actune_tokenwise_quantize / actune_tokenwise_linear) and the modules.

Bar: per-row activation codes and scales bit-exact; outputs bit-exact
against oracle/tokenwise_oracle.c (exact int32 accumulation, then the
family's fixed fp32 epilogue) for every layout pair, row counts from 1 to
200, ragged N tiles, K splits and biases; the oracle's torch-GPU division
semantics pinned against torch on the GPU itself.
"""
import numpy as np
import pytest
import torch

from actune_amd import _native
from actune_amd.kernels import tokenwise as T
from oracle import oracle as O
from tests.helpers import bits, dtype_name, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
# (module class, weight bits, activation bits, epilogue mode)
FAMILY = [(T.W4A8TritonLinear, 4, 8, 0), (T.W8A8TritonLinear, 8, 8, 0), (T.W2A8TritonLinear, 2, 8, 0),
          (T.W4A4NativeLinear, 4, 4, 1), (T.W2A4NativeLinear, 2, 4, 1), (T.W8A4NativeLinear, 8, 4, 0)]


# ---------------------------------------------------------------- quantizer
@pytest.mark.parametrize("A", [8, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 64), (7, 4096), (33, 11008), (3, 16384), (2, 96)])
def test_row_quantizer_bit_exact(A, dtype, shape):
    m, k = shape
    x, _, _ = seeded_inputs(m, k, 1, seed=m + k + A, dtype=dtype)
    if m > 1:
        x[1] = 0  # an all-zero row: the 1e-8 floor
    codes, scales = _native.tokenwise_quantize(x.to(DEV), A)
    want_c, want_s = O.tw_quantize_rows(bits(x), A, dtype_name(dtype))
    np.testing.assert_array_equal(scales.cpu().numpy(), want_s)
    got = codes.cpu().numpy()
    if A == 4:
        np.testing.assert_array_equal(got, O.pack_rows(want_c, 4))
    else:
        np.testing.assert_array_equal(got, want_c)


def test_row_quantizer_equals_torch_gpu_eager_formula():
    """The reference's unfused path (w4a8_triton.py:400-401) run by torch on
    the GPU: amax.clamp_min(1e-8) / 127.0 (a reciprocal multiply there) and
    (x / scale).round().clamp(). Pins the oracle's reciprocal semantics on
    the hardware the product runs on."""
    x, _, _ = seeded_inputs(64, 4096, 1, seed=11)
    xd = x.to(DEV)
    scale = xd.float().abs().amax(dim=1).clamp_min(1e-8) / 127.0
    act = (xd.float() / scale[:, None]).round().clamp(-128, 127).to(torch.int8)
    codes, scales = _native.tokenwise_quantize(xd, 8)
    assert torch.equal(scales, scale) and torch.equal(codes, act)
    want_c, want_s = O.tw_quantize_rows(bits(x), 8)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)
    scale4 = xd.float().abs().amax(dim=1).clamp_min(1e-8) / 7.0
    np.testing.assert_array_equal(scale4.cpu().numpy(), O.tw_quantize_rows(bits(x), 4)[1])


def test_weight_codes_on_gpu_follow_torch_gpu():
    """A module built from a GPU-resident layer has the scales torch computes
    there (w4a8_triton.py:370-371: amax.clamp_min(1e-8) / 7.0 on the GPU)."""
    torch.manual_seed(3)
    lin = torch.nn.Linear(512, 256, bias=False, dtype=torch.bfloat16, device=DEV)
    w = lin.weight.detach().float()
    s4 = w.abs().amax(dim=1).clamp_min(1e-8) / 7.0
    q4 = (w / s4[:, None]).round().clamp(-8, 7).to(torch.int8)
    mod = T.W4A8TritonLinear(lin)
    assert torch.equal(mod.weight_scale, s4)
    half = 256
    packed = ((q4[:, :half].to(torch.int16) & 15) | ((q4[:, half:].to(torch.int16) & 15) << 4)).to(torch.uint8)
    assert torch.equal(mod.packed_weight, packed.t().contiguous())
    s8 = w.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    assert torch.equal(T.W8A8TritonLinear(lin).weight_scale, s8)


# ---------------------------------------------------------------- modules vs oracle
def _oracle_out(x, lin, W, A, mode, dtype):
    codes, scale = O.weight_codes(lin.weight.detach().float().cpu().numpy(), W, A, gpu_division=True)
    a_codes, a_scales = O.tw_quantize_rows(bits(x), A, dtype_name(dtype))
    acc = O.tw_dots(a_codes, codes)
    bias = None if lin.bias is None else lin.bias.detach().float().cpu().numpy()
    return O.round_out(O.tw_epilogue(acc, a_scales, scale, bias, mode), dtype_name(dtype))


@pytest.mark.parametrize("cls,W,A,mode", FAMILY)
@pytest.mark.parametrize("m,k,n", [(1, 256, 48), (3, 512, 80), (16, 1024, 128), (17, 384, 16),
                                   (40, 256, 96), (130, 512, 144), (200, 128, 32), (1, 4096, 256),
                                   # out_features not a multiple of 16 (padded K-major operands)
                                   (5, 256, 100), (1, 512, 40), (9, 1024, 1000), (2, 256, 8), (64, 512, 24)])
@pytest.mark.parametrize("bias", [False, True])
def test_modules_bit_exact(cls, W, A, mode, m, k, n, bias):
    if k % (128 if cls in (T.W8A8TritonLinear, T.W2A8TritonLinear, T.W8A4NativeLinear) else 64):
        pytest.skip("in_features not allowed for this module")
    torch.manual_seed(m + k + n)
    lin = torch.nn.Linear(k, n, bias=bias, dtype=torch.bfloat16, device=DEV)
    x, _, _ = seeded_inputs(m, k, 1, seed=m * 3 + k)
    mod = cls(lin)
    with torch.inference_mode():
        out = mod(x.to(DEV))
    torch.cuda.synchronize()
    want = _oracle_out(x, lin, W, A, mode, torch.bfloat16)
    np.testing.assert_array_equal(bits(out), want)


@pytest.mark.parametrize("case", range(40))
def test_modules_random_sweep(case):
    """Seeded random cases through the six modules: the class, M (1-600),
    K (any multiple the class takes, up to 4096), N (1-1299), the dtype and a
    bias drawn per case; every output bit against the oracle. (A one-off run
    of 1500 such cases found no failure.)"""
    rng = np.random.default_rng(50000 + case)
    cls, W, A, mode = FAMILY[int(rng.integers(len(FAMILY)))]
    step = 128 if cls in (T.W8A8TritonLinear, T.W2A8TritonLinear, T.W8A4NativeLinear) else 64
    k = step * int(rng.integers(1, 4096 // step + 1)) if rng.random() < 0.7 else step * int(rng.integers(1, 9))
    n = int(rng.integers(1, 1300))
    m = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 31, 32, 33, 48, 64, 65, 100, 128, 129, 200, 256, 257,
                        320, 384, 512, 600]))
    dtype = (torch.bfloat16, torch.float16, torch.float32)[int(rng.integers(3))]
    bias = bool(rng.random() < 0.5)
    torch.manual_seed(case)
    lin = torch.nn.Linear(k, n, bias=bias, dtype=dtype, device=DEV)
    x, _, _ = seeded_inputs(m, k, 1, seed=case, dtype=dtype)
    with torch.inference_mode():
        out = cls(lin)(x.to(DEV))
    np.testing.assert_array_equal(bits(out), _oracle_out(x, lin, W, A, mode, dtype),
                                  err_msg=f"{cls.__name__} m={m} n={n} k={k} {dtype} bias={bias}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_output_dtypes(dtype):
    torch.manual_seed(1)
    lin = torch.nn.Linear(256, 64, bias=True, dtype=dtype, device=DEV)
    x, _, _ = seeded_inputs(5, 256, 1, seed=2, dtype=dtype)
    for cls, W, A, mode in FAMILY:
        if cls in (T.W8A8TritonLinear, T.W2A8TritonLinear, T.W8A4NativeLinear) and 256 % 128:
            continue
        out = cls(lin)(x.to(DEV))
        np.testing.assert_array_equal(bits(out), _oracle_out(x, lin, W, A, mode, dtype), err_msg=cls.__name__)


def test_w4a8_ragged_k_tail():
    """in_features = 96 (divisible by 32, not 64): the last K-step of the
    nibble-pair layout is half empty."""
    torch.manual_seed(4)
    lin = torch.nn.Linear(96, 32, bias=True, dtype=torch.bfloat16, device=DEV)
    for m in (1, 3, 40):
        x, _, _ = seeded_inputs(m, 96, 1, seed=m)
        out = T.W4A8TritonLinear(lin)(x.to(DEV))
        np.testing.assert_array_equal(bits(out), _oracle_out(x, lin, 4, 8, 0, torch.bfloat16))


# ---------------------------------------------------------------- split-K and decode
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (8, 4096, 4096),
                                   (2, 256, 2048), (64, 512, 4096), (512, 4096, 4096), (512, 8192, 2048),
                                   (200, 11008, 512), (256, 4096, 4096), (128, 4096, 11008)])
def test_split_k_full_size_sampled(m, n, k):
    """Llama-2-7B / Gemma shapes through the C ABI with every layout pair:
    the K split the library picks is exact, and so is each large-M ring
    configuration (M = 512 at N = 4096: fewer than 512 tiles of 64 x 128;
    N = 8192: 512 tiles; M = 200: a ragged last row tile; M = 256 and 128:
    ring grids split in two or four), checked on 64 sampled columns."""
    x, w, _ = seeded_inputs(m, k, n, seed=m + n + k)
    xd = x.to(DEV)
    cols = np.sort(np.random.default_rng(n).choice(n, size=64, replace=False))
    for W, A, wl, mode in ((4, 8, _native.TW_KMAJOR_W4, 0), (8, 8, _native.TW_KMAJOR_W8, 0),
                           (2, 8, _native.TW_KMAJOR_W2, 0), (4, 4, _native.TW_ROWS_S4, 1),
                           (2, 4, _native.TW_ROWS_S2, 1), (8, 4, _native.TW_KMAJOR_W8, 0)):
        codes, scale = O.weight_codes(w.float().numpy(), W, A, gpu_division=True)
        packed = O.pack_kmajor(codes, W) if wl <= _native.TW_KMAJOR_W2 else O.pack_rows(codes, W)
        a_layout = _native.TW_ACT_A8 if A == 8 else _native.TW_ACT_A4
        act, s = _native.tokenwise_quantize(xd, A)
        need = _native.tokenwise_workspace_bytes(m, n, k, wl, a_layout)
        ws = torch.full((max(need, 1),), 0x5A, dtype=torch.uint8, device=DEV)
        out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
        for _ in range(2):  # the workspace holds no state between calls
            _native.tokenwise_linear(act, a_layout, s, torch.from_numpy(packed).to(DEV), wl,
                                     torch.from_numpy(scale).to(DEV), None, n, k, mode, out,
                                     workspace=ws if need else None)
        a_codes, a_scales = O.tw_quantize_rows(bits(x), A)
        acc = O.tw_dots(a_codes, codes[cols])
        want = O.round_out(O.tw_epilogue(acc, a_scales, scale[cols], None, mode), "bf16")
        np.testing.assert_array_equal(bits(out)[:, cols], want, err_msg=f"W{W}A{A}")


@pytest.mark.parametrize("m,n,k", [(1, 50, 2048), (3, 1001, 4096), (40, 30, 4096), (8, 4095, 1024), (1, 128, 20480),
                                   (2, 75, 20480), (40, 7001, 1024)])
def test_split_reduce_columns(m, n, k):
    """The row-major S4 / S2 layouts take any out_features. The reduce adds
    the K splits one column per thread, or four where M * N >= 262144 (M =
    40, N = 7001: four 4-byte loads per split, zeros past N; N a multiple of
    4 takes one 16-byte load, as in the full-size cases above); more than 32
    splits (K = 20480: 40) take two rounds. Every column against the
    oracle."""
    x, w, _ = seeded_inputs(m, k, n, seed=m * 7 + n)
    xd = x.to(DEV)
    for W, wl in ((4, _native.TW_ROWS_S4), (2, _native.TW_ROWS_S2)):
        codes, scale = O.weight_codes(w.float().numpy(), W, 4, gpu_division=True)
        act, s = _native.tokenwise_quantize(xd, 4)
        need = _native.tokenwise_workspace_bytes(m, n, k, wl, _native.TW_ACT_A4)
        assert need >= 2 * m * n * 4, "the case must split K"
        ws = torch.full((need,), 0x5A, dtype=torch.uint8, device=DEV)
        out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
        _native.tokenwise_linear(act, _native.TW_ACT_A4, s, torch.from_numpy(O.pack_rows(codes, W)).to(DEV), wl,
                                 torch.from_numpy(scale).to(DEV), None, n, k, _native.TW_EPI_A4, out, workspace=ws)
        a_codes, a_scales = O.tw_quantize_rows(bits(x), 4)
        want = O.round_out(O.tw_epilogue(O.tw_dots(a_codes, codes), a_scales, scale, None, 1), "bf16")
        np.testing.assert_array_equal(bits(out), want, err_msg=f"W{W}A4")


def test_w4a8_decode_graph_plan_and_counters():
    """M = 1 bf16: the module replays its DecodeGraphPlan (quantizer + split-K
    GEMM in one hipGraph); outputs equal the direct path and the oracle, and
    the decode counters advance as the reference's do."""
    torch.manual_seed(6)
    lin = torch.nn.Linear(4096, 4096, bias=False, dtype=torch.bfloat16, device=DEV)
    mod = T.W4A8TritonLinear(lin)
    x, _, _ = seeded_inputs(1, 4096, 1, seed=6)
    xd = x.to(DEV)
    with T.decode_optimization_scope() as stats:
        a = mod(xd)
        b = mod(xd[None])  # [1, 1, K] takes the same plan
    assert stats.graph_replays == 2 and stats.split_k_calls == 2
    assert T.decode_workspace_summary(mod)["decode_graph_plan_count"] == 1
    with T.decode_optimization_scope(enabled=False):
        direct = mod(xd)
    assert torch.equal(a, direct) and torch.equal(b.reshape(1, -1), direct)
    np.testing.assert_array_equal(bits(a), _oracle_out(x, lin, 4, 8, 0, torch.bfloat16))


def test_shared_a8_cache_reuses_one_quantization():
    """q/k/v siblings on the same input quantize once inside a scope
    (w4a8_triton.py:270-325), and the outputs are unchanged."""
    torch.manual_seed(7)
    mods = [T.W4A8TritonLinear(torch.nn.Linear(512, n, bias=False, dtype=torch.bfloat16, device=DEV))
            for n in (512, 128, 128)] + [T.W8A8TritonLinear(torch.nn.Linear(512, 64, bias=False,
                                                                              dtype=torch.bfloat16, device=DEV))]
    x = torch.randn(9, 512, device=DEV).to(torch.bfloat16)
    alone = [m(x) for m in mods]
    with T.shared_a8_cache_scope() as state:
        shared = [m(x) for m in mods]
    assert state.misses == 1 and state.hits == 3
    assert all(torch.equal(a, b) for a, b in zip(alone, shared))


def test_launch_decode_into_caller_buffers():
    """launch_decode into caller-owned buffers holding arbitrary values, as
    benchmarks use it (decode_w4a8_triton.py:113-149)."""
    torch.manual_seed(8)
    n, k = 4096, 4096
    mod = T.W4A8TritonLinear(torch.nn.Linear(k, n, bias=True, dtype=torch.bfloat16, device=DEV))
    x = torch.randn(1, k, device=DEV).to(torch.bfloat16)
    act, s = _native.tokenwise_quantize(x, 8)
    out = torch.empty(1, n, device=DEV, dtype=torch.bfloat16)
    partial = torch.full((32, n), 7, dtype=torch.int32, device=DEV)
    T.launch_decode(act, mod.packed_weight, None, s, mod.weight_scale, mod.bias, out, partial)
    with T.decode_optimization_scope(enabled=False):
        want = mod(x)
    assert torch.equal(out, want)


# ---------------------------------------------------------------- fused one-row quantization
def _kmajor_weights(n, k, W, seed):
    w = torch.from_numpy(np.random.default_rng(seed).standard_normal((n, k)).astype(np.float32))
    codes, scale = O.weight_codes(w.numpy(), W, 8, gpu_division=True)
    return torch.from_numpy(O.pack_kmajor(codes, W)).to(DEV), torch.from_numpy(scale).to(DEV)


@pytest.mark.parametrize("W,wl", [(4, _native.TW_KMAJOR_W4), (8, _native.TW_KMAJOR_W8), (2, _native.TW_KMAJOR_W2)])
@pytest.mark.parametrize("n,k", [(4096, 4096), (11008, 4096), (4096, 11008), (256, 2048), (48, 256), (32, 96),
                                 (128, 16384), (64, 64), (48, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_row_quantization_equals_two_step(W, wl, n, k, dtype):
    """actune_tokenwise_linear_x (the row quantized inside the split GEMM)
    gives the quantizer + linear result bit for bit, scale included; K = 64
    is one K-step, so the launch is unsplit and its epilogue reads the row
    scale the launch computed."""
    if k % {4: 32, 8: 64, 2: 128}[W]:
        pytest.skip("in_features not allowed for this layout")
    w, ws = _kmajor_weights(n, k, W, seed=n + k + W)
    bias = torch.randn(n, device=DEV).to(dtype) if n % 3 == 0 else None
    x = (torch.randn(1, k, device=DEV) * 3).to(dtype)
    act, s = _native.tokenwise_quantize(x, 8)
    need = _native.tokenwise_workspace_bytes(1, n, k, wl, _native.TW_ACT_A8)
    if k == 64:
        assert need == 0  # one K-step: no split
    ws_buf = torch.full((max(need, 1),), 0x5A, dtype=torch.uint8, device=DEV)
    want = torch.empty(1, n, device=DEV, dtype=dtype)
    _native.tokenwise_linear(act, _native.TW_ACT_A8, s, w, wl, ws, bias, n, k, _native.TW_EPI_A8, want,
                             workspace=ws_buf if need else None)
    got = torch.full((1, n), 3.0, device=DEV, dtype=dtype)
    s_out = torch.full((1,), -1.0, device=DEV)
    for _ in range(2):  # repeated calls on the same buffers
        _native.tokenwise_linear_x(x, s_out, w, wl, ws, bias, n, k, _native.TW_EPI_A8, got,
                                   workspace=ws_buf if need else None)
    torch.cuda.synchronize()
    assert torch.equal(s_out, s)
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("scale", [0.0, 1e-30, 1e-4, 1e3])
def test_fused_row_quantization_magnitudes_against_oracle(scale):
    """Zero, subnormal-scale, small and large rows through the fused launch,
    against the CPU oracle (per-row codes, exact dots, epilogue)."""
    n, k = 256, 4096
    rng = np.random.default_rng(11)
    w = rng.standard_normal((n, k)).astype(np.float32)
    codes, wscale = O.weight_codes(w, 4, 8, gpu_division=True)
    x = torch.from_numpy((rng.standard_normal((1, k)) * scale).astype(np.float32)).to(torch.bfloat16)
    out = torch.empty(1, n, device=DEV, dtype=torch.bfloat16)
    s_out = torch.empty(1, device=DEV)
    need = _native.tokenwise_workspace_bytes(1, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    ws_buf = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
    _native.tokenwise_linear_x(x.to(DEV), s_out, torch.from_numpy(O.pack_kmajor(codes, 4)).to(DEV),
                               _native.TW_KMAJOR_W4, torch.from_numpy(wscale).to(DEV), None, n, k,
                               _native.TW_EPI_A8, out, workspace=ws_buf if need else None)
    a_codes, a_scales = O.tw_quantize_rows(bits(x), 8)
    want = O.round_out(O.tw_epilogue(O.tw_dots(a_codes, codes), a_scales, wscale, None, 0), "bf16")
    np.testing.assert_array_equal(bits(out), want)
    np.testing.assert_array_equal(s_out.cpu().numpy(), a_scales)


@pytest.mark.parametrize("W,wl", [(4, _native.TW_KMAJOR_W4), (8, _native.TW_KMAJOR_W8), (2, _native.TW_KMAJOR_W2)])
@pytest.mark.parametrize("m,n,k", [(2, 4096, 4096), (2, 256, 16384), (3, 11008, 4096), (4, 128, 8192),
                                   (5, 4096, 4096), (8, 4096, 4096), (8, 11008, 4096), (8, 48, 256), (7, 64, 64),
                                   (6, 256, 2048), (2, 32, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_rows_quantization_equals_two_step(W, wl, m, n, k, dtype):
    """Two to eight rows quantized inside the split GEMM (each row padded
    count P = 2, 4, 8 reads K <= 32768 / P): the quantizer + linear result
    bit for bit, row scales included; K = 64 is unsplit, so the epilogue
    reads the scales the launch computed."""
    if k % {4: 32, 8: 64, 2: 128}[W]:
        pytest.skip("in_features not allowed for this layout")
    assert k <= _native.tokenwise_fused_max_k(m)
    w, ws = _kmajor_weights(n, k, W, seed=n + k + W + m)
    bias = torch.randn(n, device=DEV).to(dtype) if n % 3 == 0 else None
    x = torch.randn(m, k, device=DEV) * 3
    x[m // 2] *= 1e-3  # rows of different magnitude
    x = x.to(dtype)
    act, s = _native.tokenwise_quantize(x, 8)
    need = _native.tokenwise_workspace_bytes(m, n, k, wl, _native.TW_ACT_A8)
    ws_buf = torch.full((max(need, 1),), 0x5A, dtype=torch.uint8, device=DEV)
    want = torch.empty(m, n, device=DEV, dtype=dtype)
    _native.tokenwise_linear(act, _native.TW_ACT_A8, s, w, wl, ws, bias, n, k, _native.TW_EPI_A8, want,
                             workspace=ws_buf if need else None)
    got = torch.full((m, n), 3.0, device=DEV, dtype=dtype)
    s_out = torch.full((m,), -1.0, device=DEV)
    for _ in range(2):
        _native.tokenwise_linear_x(x, s_out, w, wl, ws, bias, n, k, _native.TW_EPI_A8, got,
                                   workspace=ws_buf if need else None)
    torch.cuda.synchronize()
    assert torch.equal(s_out, s)
    np.testing.assert_array_equal(bits(got), bits(want))


def test_fused_rows_quantization_against_oracle():
    """Eight rows (zero, tiny, ordinary and large) through the fused launch
    against the CPU oracle (per-row codes, exact dots, epilogue)."""
    n, k, m = 256, 4096, 8
    rng = np.random.default_rng(12)
    w = rng.standard_normal((n, k)).astype(np.float32)
    codes, wscale = O.weight_codes(w, 4, 8, gpu_division=True)
    mags = np.array([0.0, 1e-30, 1e-4, 1.0, 3.0, 1e3, 0.5, 7.0], dtype=np.float32)[:, None]
    x = torch.from_numpy((rng.standard_normal((m, k)) * mags).astype(np.float32)).to(torch.bfloat16)
    out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    s_out = torch.empty(m, device=DEV)
    need = _native.tokenwise_workspace_bytes(m, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    ws_buf = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
    _native.tokenwise_linear_x(x.to(DEV), s_out, torch.from_numpy(O.pack_kmajor(codes, 4)).to(DEV),
                               _native.TW_KMAJOR_W4, torch.from_numpy(wscale).to(DEV), None, n, k,
                               _native.TW_EPI_A8, out, workspace=ws_buf if need else None)
    a_codes, a_scales = O.tw_quantize_rows(bits(x), 8)
    want = O.round_out(O.tw_epilogue(O.tw_dots(a_codes, codes), a_scales, wscale, None, 0), "bf16")
    np.testing.assert_array_equal(bits(out), want)
    np.testing.assert_array_equal(s_out.cpu().numpy(), a_scales)


def test_fused_row_quantization_rejects_what_it_does_not_take():
    x = torch.randn(9, 256, device=DEV).to(torch.bfloat16)
    w = torch.zeros(256 // 2 * 64, dtype=torch.uint8, device=DEV)
    ws = torch.ones(64, device=DEV)
    out = torch.empty(9, 64, device=DEV, dtype=torch.bfloat16)
    s_out = torch.empty(9, device=DEV)
    with pytest.raises(RuntimeError, match=r"M <= 8"):
        _native.tokenwise_linear_x(x, s_out, w, _native.TW_KMAJOR_W4, ws, None, 64, 256, _native.TW_EPI_A8, out)
    lib = _native.lib()
    # the C ABI checks the row count, K, the dtype and the layout itself
    rc = lib.actune_tokenwise_linear_x(x.data_ptr(), 0, s_out.data_ptr(), w.data_ptr(), _native.TW_KMAJOR_W4,
                                       ws.data_ptr(), None, 0, out.data_ptr(), 0, 9, 64, 256, 0, None, 0, None)
    assert rc != 0 and b"1 to 8 rows" in lib.actune_last_error()
    rc = lib.actune_tokenwise_linear_x(x.data_ptr(), 0, s_out.data_ptr(), w.data_ptr(), _native.TW_KMAJOR_W4,
                                       ws.data_ptr(), None, 0, out.data_ptr(), 0, 1, 64, 32768, 0, None, 0, None)
    assert rc != 0 and b"16384" in lib.actune_last_error()
    rc = lib.actune_tokenwise_linear_x(x.data_ptr(), 0, s_out.data_ptr(), w.data_ptr(), _native.TW_KMAJOR_W4,
                                       ws.data_ptr(), None, 0, out.data_ptr(), 0, 5, 64, 8192, 0, None, 0, None)
    assert rc != 0 and b"4096" in lib.actune_last_error()
    rc = lib.actune_tokenwise_linear_x(x.data_ptr(), 2, s_out.data_ptr(), w.data_ptr(), _native.TW_KMAJOR_W4,
                                       ws.data_ptr(), None, 0, out.data_ptr(), 0, 2, 64, 256, 0, None, 0, None)
    assert rc != 0 and b"bf16 or f16" in lib.actune_last_error()
    rc = lib.actune_tokenwise_linear_x(x.data_ptr(), 0, s_out.data_ptr(), w.data_ptr(), _native.TW_ROWS_S4,
                                       ws.data_ptr(), None, 0, out.data_ptr(), 0, 1, 64, 256, 0, None, 0, None)
    assert rc != 0 and b"K-major" in lib.actune_last_error()


# ---------------------------------------------------------------- sibling projections in one launch
MULTI_LAYOUTS = [(4, 8, _native.TW_KMAJOR_W4, 0), (8, 8, _native.TW_KMAJOR_W8, 0), (2, 8, _native.TW_KMAJOR_W2, 0),
                 (4, 4, _native.TW_ROWS_S4, 1), (2, 4, _native.TW_ROWS_S2, 1), (8, 4, _native.TW_KMAJOR_W8, 0)]


def _packed_targets(n, k, W, A, wl, count, seed, bias_every=None, dtype=torch.bfloat16, m=1):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        w = rng.standard_normal((n, k)).astype(np.float32)
        codes, scale = O.weight_codes(w, W, A, gpu_division=True)
        packed = O.pack_kmajor(codes, W) if wl <= _native.TW_KMAJOR_W2 else O.pack_rows(codes, W)
        bias = None
        if bias_every:
            bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(DEV).to(dtype)
        out.append(dict(codes=codes, scale=scale, w=torch.from_numpy(packed).to(DEV),
                        ws=torch.from_numpy(scale).to(DEV), bias=bias,
                        out=torch.full((m, n), 5.0, device=DEV, dtype=dtype)))
    return out


@pytest.mark.parametrize("W,A,wl,mode", MULTI_LAYOUTS)
@pytest.mark.parametrize("m,n,k", [(1, 256, 2048), (8, 512, 4096), (17, 96, 1024), (300, 256, 512)])
@pytest.mark.parametrize("count", [1, 3, 4])
def test_multi_target_equals_single_calls(W, A, wl, mode, m, n, k, count):
    """actune_tokenwise_linear_multi on codes: every target equals its own
    actune_tokenwise_linear call bit for bit (split and unsplit shapes,
    small-M and ring geometries, with biases); the first target also
    against the oracle."""
    x, _, _ = seeded_inputs(m, k, 1, seed=m + n + k + count)
    a_layout = _native.TW_ACT_A8 if A == 8 else _native.TW_ACT_A4
    act, s = _native.tokenwise_quantize(x.to(DEV), A)
    tg = _packed_targets(n, k, W, A, wl, count, seed=W * 10 + A + count, bias_every=count > 1, m=m)
    need = _native.tokenwise_workspace_bytes(m, n, k, wl, a_layout)
    work = torch.full((max(count * need, 1),), 0x5A, dtype=torch.uint8, device=DEV)
    _native.tokenwise_linear_multi([(t["w"], t["ws"], t["bias"], t["out"]) for t in tg], wl, n, k, mode, s,
                                   codes=act, a_layout=a_layout, workspace=work if need else None)
    for i, t in enumerate(tg):
        want = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
        single = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        _native.tokenwise_linear(act, a_layout, s, t["w"], wl, t["ws"], t["bias"], n, k, mode, want,
                                 workspace=single if need else None)
        assert torch.equal(t["out"], want), (i, W, A)
    a_codes, a_scales = O.tw_quantize_rows(bits(x), A)
    b0 = None if tg[0]["bias"] is None else tg[0]["bias"].float().cpu().numpy()
    want0 = O.round_out(O.tw_epilogue(O.tw_dots(a_codes, tg[0]["codes"]), a_scales, tg[0]["scale"], b0, mode), "bf16")
    np.testing.assert_array_equal(bits(tg[0]["out"]), want0)


@pytest.mark.parametrize("m,n,k,count", [(1, 4096, 4096, 3), (1, 11008, 4096, 2), (8, 4096, 4096, 3),
                                         (8, 11008, 4096, 2), (1, 4096, 11008, 1), (3, 256, 2048, 2)])
def test_multi_target_quantizes_rows_in_launch_full_size(m, n, k, count):
    """Llama-2-7B q/k/v and gate/up at M = 1 and 8 with the rows quantized
    inside the launch: the written row scales equal the quantizer's, and
    each target equals the oracle on 64 sampled columns."""
    x, _, _ = seeded_inputs(m, k, 1, seed=n + k + m)
    xd = x.to(DEV)
    tg = _packed_targets(n, k, 4, 8, _native.TW_KMAJOR_W4, count, seed=n + count + m, m=m)
    need = count * _native.tokenwise_workspace_bytes(m, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    work = torch.full((max(need, 1),), 0x5A, dtype=torch.uint8, device=DEV)
    s_out = torch.full((m,), -1.0, device=DEV)
    _native.tokenwise_linear_multi([(t["w"], t["ws"], None, t["out"]) for t in tg], _native.TW_KMAJOR_W4, n, k,
                                   _native.TW_EPI_A8, s_out, x=xd, workspace=work if need else None)
    torch.cuda.synchronize()
    a_codes, a_scales = O.tw_quantize_rows(bits(x), 8)
    np.testing.assert_array_equal(s_out.cpu().numpy(), a_scales)
    cols = np.sort(np.random.default_rng(k).choice(n, size=64, replace=False))
    for i, t in enumerate(tg):
        want = O.round_out(O.tw_epilogue(O.tw_dots(a_codes, t["codes"][cols]), a_scales, t["scale"][cols], None, 0),
                           "bf16")
        np.testing.assert_array_equal(bits(t["out"])[:, cols], want, err_msg=str(i))


def test_multi_target_rejects_bad_calls():
    x = torch.randn(1, 256, device=DEV).to(torch.bfloat16)
    tg = _packed_targets(64, 256, 4, 8, _native.TW_KMAJOR_W4, 2, seed=1)
    s = torch.empty(1, device=DEV)
    targets = [(t["w"], t["ws"], t["bias"], t["out"]) for t in tg]
    with pytest.raises(ValueError, match="either codes or x"):
        _native.tokenwise_linear_multi(targets, _native.TW_KMAJOR_W4, 64, 256, 0, s)
    with pytest.raises(ValueError, match="1 to 4 targets"):
        _native.tokenwise_linear_multi(targets * 3, _native.TW_KMAJOR_W4, 64, 256, 0, s, x=x)
    lib = _native.lib()
    structs = (_native._TwTarget * 5)()
    rc = lib.actune_tokenwise_linear_multi(None, 0, x.data_ptr(), 0, s.data_ptr(), _native.TW_KMAJOR_W4, structs, 5,
                                           2, 0, 1, 64, 256, 0, None, 0, None)
    assert rc != 0 and b"ACTUNE_MAX_TARGETS" in lib.actune_last_error()
    rc = lib.actune_tokenwise_linear_multi(x.data_ptr(), 0, x.data_ptr(), 0, s.data_ptr(), _native.TW_KMAJOR_W4,
                                           structs, 2, 2, 0, 1, 64, 256, 0, None, 0, None)
    assert rc != 0 and b"either" in lib.actune_last_error()


def test_decode_group_plan_and_launch_group():
    """q/k/v of one row as ONE decode plan (one GEMM launch over the three
    projections + one reduce, the row quantized in the launch) and through
    launch_decode_group on caller buffers: both equal the modules' own
    direct calls bit for bit, and the counters record one projection group."""
    torch.manual_seed(9)
    mods = [T.W4A8TritonLinear(torch.nn.Linear(4096, 4096, bias=b, dtype=torch.bfloat16, device=DEV))
            for b in (False, True, False)]
    x, _, _ = seeded_inputs(1, 4096, 1, seed=9)
    xd = x.to(DEV)
    with T.decode_optimization_scope(enabled=False):
        want = [m(xd) for m in mods]
    plan = T.DecodeGraphPlan(xd, [m.packed_weight for m in mods], [None] * 3, [m.weight_scale for m in mods],
                             [m.bias for m in mods])
    with T.decode_optimization_scope() as stats:
        for _ in range(3):
            got = plan.run(xd)
            torch.cuda.synchronize()
            assert all(torch.equal(got[i:i + 1], want[i]) for i in range(3))
    assert stats.graph_replays == 3 and stats.projection_groups == 3 and stats.projection_calls_fused == 9
    assert stats.graph_quantization_kernels == 0  # the row is quantized inside the GEMM launch
    act, s = _native.tokenwise_quantize(xd, 8)
    outs = [torch.empty(1, 4096, device=DEV, dtype=torch.bfloat16) for _ in mods]
    partial = torch.full((3 * 32, 4096), 7, dtype=torch.int32, device=DEV)
    T.launch_decode_group(act, [m.packed_weight for m in mods], [None] * 3, s, [m.weight_scale for m in mods],
                          [m.bias for m in mods], outs, partial)
    assert all(torch.equal(o, w) for o, w in zip(outs, want))


def test_captured_split_workspace_survives_later_calls():
    """A W4A8 module captured at M = 1 (its split-K workspace comes from the
    graph's pool), then called eagerly at M = 8 (a larger workspace), then
    filler tensors allocated and written: replays leave the fillers
    untouched and still equal the eager result."""
    torch.manual_seed(10)
    mod = T.W4A8TritonLinear(torch.nn.Linear(4096, 4096, bias=False, dtype=torch.bfloat16, device=DEV))
    x1 = torch.randn(1, 4096, device=DEV).to(torch.bfloat16)
    x8 = torch.randn(8, 4096, device=DEV).to(torch.bfloat16)
    with T.decode_optimization_scope(enabled=False):
        want1 = mod(x1)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            mod(x1)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = mod(x1)
        want8 = mod(x8)
        fillers = [torch.full((1 << 18,), 1234 + i, dtype=torch.int32, device=DEV) for i in range(16)]
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want1)
        assert all(bool((f == 1234 + i).all()) for i, f in enumerate(fillers))
        assert torch.equal(mod(x8), want8)


# ---------------------------------------------------------------- signed-R4 residual decode
def _r4_targets(n, k, count, seed, m=1, with_residual=(True,), bias_dtype=torch.bfloat16):
    """count W4R4 projections: random q4 / r4 codes (about 1 in 32 pairs
    wraps), residual present per with_residual (cycled), a bias on every
    other projection; the oracle's expected codes and epilogue scale."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        q = rng.integers(-8, 8, (n, k)).astype(np.int8)
        has = with_residual[i % len(with_residual)]
        r = rng.integers(-8, 8, (n, k)).astype(np.int8) if has else np.zeros((n, k), np.int8)
        ws = rng.uniform(1e-3, 3e-2, n).astype(np.float32)
        bias = None
        if i % 2:
            bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(DEV).to(bias_dtype)
        out.append(dict(q=q, nested=O.nested_r4_codes(q, r), scale=ws, w=torch.from_numpy(O.pack_kmajor(q, 4)).to(DEV),
                        r=torch.from_numpy(O.pack_kmajor(r, 4)).to(DEV) if has else None,
                        ws=torch.from_numpy(ws).to(DEV), bias=bias,
                        out=torch.full((m, n), 5.0, device=DEV, dtype=torch.bfloat16)))
    return out


def _r4_oracle(a_codes, a_scales, t, cols=None):
    sel = slice(None) if cols is None else cols
    b = None if t["bias"] is None else t["bias"].float().cpu().numpy()[sel]
    acc = O.tw_dots(a_codes, t["nested"][sel])
    return O.round_out(O.tw_epilogue(acc, a_scales, t["scale"][sel] / np.float32(16), b, 0), "bf16")


@pytest.mark.parametrize("m,n,k,count", [(1, 4096, 4096, 3), (1, 11008, 4096, 2), (1, 4096, 11008, 1),
                                         (8, 512, 2048, 2), (32, 256, 1024, 4), (3, 96, 160, 1), (17, 48, 64, 2)])
@pytest.mark.parametrize("source", ["codes", "x"])
def test_w4r4_multi_against_oracle(m, n, k, count, source):
    """actune_tokenwise_linear_multi in the W4R4 layout, residuals present on
    some projections and absent on others: every output equals the oracle
    (int8 codes 16 q4 + r4 with the reference's wrap, epilogue scale ws / 16)
    on sampled columns, from activation codes or from rows quantized in the
    launch (M <= 8); K = 160 ends in a half K-step."""
    if source == "x" and m > 8:
        pytest.skip("rows are quantized in the launch up to M = 8")
    x, _, _ = seeded_inputs(m, k, 1, seed=m * 7 + n + k)
    xd = x.to(DEV)
    tg = _r4_targets(n, k, count, seed=n + k + count, m=m, with_residual=(True, False))
    wl = _native.TW_KMAJOR_W4R4
    need = count * _native.tokenwise_workspace_bytes(m, n, k, wl, _native.TW_ACT_A8)
    work = torch.full((max(need, 1),), 0x5A, dtype=torch.uint8, device=DEV) if need else None
    targets = [(t["w"], t["ws"], t["bias"], t["out"]) for t in tg]
    residuals = [t["r"] for t in tg]
    if source == "codes":
        act, s = _native.tokenwise_quantize(xd, 8)
        _native.tokenwise_linear_multi(targets, wl, n, k, _native.TW_EPI_A8, s, codes=act, workspace=work,
                                       residuals=residuals)
    else:
        s = torch.full((m,), -1.0, device=DEV)
        _native.tokenwise_linear_multi(targets, wl, n, k, _native.TW_EPI_A8, s, x=xd, workspace=work,
                                       residuals=residuals)
    torch.cuda.synchronize()
    a_codes, a_scales = O.tw_quantize_rows(bits(x), 8)
    np.testing.assert_array_equal(s.cpu().numpy(), a_scales)
    cols = None if n <= 512 else np.sort(np.random.default_rng(k + 1).choice(n, size=96, replace=False))
    for i, t in enumerate(tg):
        got = bits(t["out"]) if cols is None else bits(t["out"])[:, cols]
        np.testing.assert_array_equal(got, _r4_oracle(a_codes, a_scales, t, cols), err_msg=f"projection {i}")


def test_w4r4_without_residual_equals_w4():
    """A W4R4 launch whose projection has no residual gives the plain
    KMAJOR_W4 call's result bit for bit (codes 16 q4, scale ws / 16)."""
    m, n, k = 4, 1024, 4096
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    act, s = _native.tokenwise_quantize(x, 8)
    (t,) = _r4_targets(n, k, 1, seed=4, m=m, with_residual=(False,))
    need = _native.tokenwise_workspace_bytes(m, n, k, _native.TW_KMAJOR_W4, _native.TW_ACT_A8)
    want = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    _native.tokenwise_linear(act, _native.TW_ACT_A8, s, t["w"], _native.TW_KMAJOR_W4, t["ws"], None, n, k,
                             _native.TW_EPI_A8, want,
                             workspace=torch.empty(need, dtype=torch.uint8, device=DEV) if need else None)
    need4 = _native.tokenwise_workspace_bytes(m, n, k, _native.TW_KMAJOR_W4R4, _native.TW_ACT_A8)
    _native.tokenwise_linear_multi([(t["w"], t["ws"], None, t["out"])], _native.TW_KMAJOR_W4R4, n, k,
                                   _native.TW_EPI_A8, s, codes=act, residuals=[None],
                                   workspace=torch.empty(need4, dtype=torch.uint8, device=DEV) if need4 else None)
    assert torch.equal(t["out"], want)


def test_w4r4_decode_surface_mixed_group():
    """The decode API with residuals (decode_w4a8_triton.py:113-239, 312-425):
    a mixed W4/R4 q/k/v group through launch_decode_group on caller buffers
    and through a DecodeGraphPlan (three replays), decode_linear and
    launch_decode on one residual projection: all equal the oracle."""
    n, k = 4096, 4096
    tg = _r4_targets(n, k, 3, seed=12, with_residual=(True, False, True), bias_dtype=torch.bfloat16)
    x, _, _ = seeded_inputs(1, k, 1, seed=12)
    xd = x.to(DEV)
    a_codes, a_scales = O.tw_quantize_rows(bits(x), 8)
    want = [_r4_oracle(a_codes, a_scales, t) for t in tg]
    act, s = _native.tokenwise_quantize(xd, 8)
    weights, residuals = [t["w"] for t in tg], [t["r"] for t in tg]
    scales, biases = [t["ws"] for t in tg], [t["bias"] for t in tg]
    outs = [torch.empty(1, n, device=DEV, dtype=torch.bfloat16) for _ in tg]
    partial = torch.full((3 * 32, n), 7, dtype=torch.int32, device=DEV)
    T.launch_decode_group(act, weights, residuals, s, scales, biases, outs, partial)
    for i, o in enumerate(outs):
        np.testing.assert_array_equal(bits(o), want[i], err_msg=f"group projection {i}")
    plan = T.DecodeGraphPlan(xd, weights, residuals, scales, biases)
    with T.decode_optimization_scope() as stats:
        for _ in range(3):
            got = plan.run(xd)
            torch.cuda.synchronize()
            for i in range(3):
                np.testing.assert_array_equal(bits(got[i:i + 1]), want[i], err_msg=f"plan projection {i}")
    assert stats.graph_replays == 3 and stats.projection_calls_fused == 9
    one = torch.empty(1, n, device=DEV, dtype=torch.bfloat16)
    with T.decode_optimization_scope() as stats:
        T.decode_linear(act, tg[0]["w"], tg[0]["r"], s, tg[0]["ws"], tg[0]["bias"], one)
    assert stats.split_k_calls == 1
    np.testing.assert_array_equal(bits(one), want[0])
    one.fill_(0)
    T.launch_decode(act, tg[2]["w"], tg[2]["r"], s, tg[2]["ws"], tg[2]["bias"], one, partial)
    np.testing.assert_array_equal(bits(one), want[2])


def test_w4r4_rejects_bad_calls():
    m, n, k = 1, 64, 256
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    act, s = _native.tokenwise_quantize(x, 8)
    (t,) = _r4_targets(n, k, 1, seed=2, m=m)
    tgt = [(t["w"], t["ws"], None, t["out"])]
    with pytest.raises(ValueError, match="actune_tokenwise_linear_multi"):
        _native.tokenwise_linear(act, _native.TW_ACT_A8, s, t["w"], _native.TW_KMAJOR_W4R4, t["ws"], None, n, k,
                                 _native.TW_EPI_A8, t["out"])
    with pytest.raises(ValueError, match="W4R4 layout only"):
        _native.tokenwise_linear_multi(tgt, _native.TW_KMAJOR_W4, n, k, 0, s, codes=act, residuals=[t["r"]])
    with pytest.raises(ValueError, match="one residual"):
        _native.tokenwise_linear_multi(tgt, _native.TW_KMAJOR_W4R4, n, k, 0, s, codes=act, residuals=[t["r"]] * 2)
    with pytest.raises(RuntimeError, match="residual shape"):
        _native.tokenwise_linear_multi(tgt, _native.TW_KMAJOR_W4R4, n, k, 0, s, codes=act, residuals=[t["r"][:-1]])
    big = torch.zeros(33, k, dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError, match="up to 32 rows"):
        _native.tokenwise_linear_multi([(t["w"], t["ws"], None, torch.empty(33, n, device=DEV))],
                                       _native.TW_KMAJOR_W4R4, n, k, 0, torch.ones(33, device=DEV), codes=big,
                                       residuals=[t["r"]])


def test_ragged_width_operands_follow_buffer_updates():
    """A K-major module of out_features 100 runs on padded copies of its
    buffers; an in-place update of the buffers (load_state_dict) is seen by
    the next call, and the state dict keeps the reference's shapes."""
    torch.manual_seed(21)
    lin_a = torch.nn.Linear(256, 100, bias=True, dtype=torch.bfloat16, device=DEV)
    lin_b = torch.nn.Linear(256, 100, bias=True, dtype=torch.bfloat16, device=DEV)
    mod, other = T.W4A8TritonLinear(lin_a), T.W4A8TritonLinear(lin_b)
    assert mod.packed_weight.shape == (128, 100) and mod.weight_scale.shape == (100,)
    x = torch.randn(3, 256, device=DEV).to(torch.bfloat16)
    with torch.inference_mode():
        first = mod(x)
        mod.load_state_dict(other.state_dict())
        second = mod(x)
        want = other(x)
    assert torch.equal(second, want) and not torch.equal(first, second)
