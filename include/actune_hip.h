/*
 * actune_hip.h - C ABI of the MI355X (gfx950) group-64 packed-integer linear
 * backend, libactune_hip.so.
 *
 * Plain pointers, sizes and a hipStream_t passed as void*. No allocation, no
 * host synchronisation, no exceptions: every entry point is legal inside
 * hipStreamBeginCapture and returns a status; on failure
 * actune_last_error() holds a message for the calling thread.
 *
 * Data formats are the reference's (zanehpn/Actune):
 *   packed activations  u8  [M, K*A/8]  code k at byte k*A/8, bit (k%(8/A))*A
 *   activation scales   f32 [M, K/64]
 *   packed weights      u8  [N, K*W/8]  same little-endian field order
 *   weight scale        f32 [N]
 *   output              [M, N] in bf16 / f16 / f32 (row-major)
 * Pointers to packed data and to x must be 16-byte aligned.
 */
#ifndef ACTUNE_HIP_H
#define ACTUNE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ACTUNE_OK = 0, ACTUNE_ERR_INVALID = 1, ACTUNE_ERR_DEVICE = 2 };
#define ACTUNE_MAX_TARGETS 4

/* One linear of a multi-target call (all targets share x, K and A). */
typedef struct actune_linear_target {
  const uint8_t* w;      /* packed weights [N, K*W/8] */
  const float* w_scale;  /* [N] */
  const void* bias;      /* [N] in the call's bias dtype, or NULL */
  void* out;             /* [M, N] in x's dtype */
  int64_t N;
  int32_t W;             /* this target's weight width (2, 4, 8), or 0 for the call's W */
} actune_linear_target;
enum { ACTUNE_DTYPE_BF16 = 0, ACTUNE_DTYPE_F16 = 1, ACTUNE_DTYPE_F32 = 2 };
#define ACTUNE_CONFIG_AUTO (-1)

/* Library version string. */
const char* actune_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* actune_last_error(void);

/*
 * Group-64 activation quantizer. Replaces the _quantize_groups Triton launch,
 * actune/kernels/grouped.py:55-71 (launched at :132-133), with the
 * channel-scale division of actune/layers.py:41-42 fused in when input_scale
 * is non-NULL (input_scale has x's dtype and K entries; the quotient is
 * rounded to that dtype before quantization).
 * x: [M, K] in x_dtype; packed: [M, K*A/8]; scales: [M, K/64].
 */
int actune_quantize_groups(const void* x, int x_dtype, const void* input_scale, int64_t M, int64_t K,
                           int A, uint8_t* packed, float* scales, void* stream);

/*
 * Group-64 quantizer of a gated MLP's down-projection input p = act(gate) *
 * up: the product is formed in x_dtype as torch forms it (the activation in
 * fp32, rounded to x_dtype, times up, rounded to x_dtype), optionally divided
 * by input_scale as actune_quantize_groups divides, and quantized exactly as
 * actune_quantize_groups would quantize a tensor holding p. gate and up:
 * [M, K], 16-byte aligned. act: ACTUNE_ACT_SILU (torch.nn.functional.silu)
 * or ACTUNE_ACT_GELU_TANH (gelu(approximate="tanh"), Gemma's
 * gelu_pytorch_tanh). No reference counterpart: it folds the activation and
 * the product of the reference's patched MLP forward
 * (actune/kernels/grouped.py:18-25) into the down projection's quantizer
 * launch (grouped.py:132-133), three launches into one.
 */
enum { ACTUNE_ACT_SILU = 0, ACTUNE_ACT_GELU_TANH = 1 };
int actune_quantize_gated(const void* gate, const void* up, int x_dtype, int act, const void* input_scale,
                          int64_t M, int64_t K, int A, uint8_t* packed, float* scales, void* stream);

/*
 * Packed grouped linear. Replaces the native op `linear(a, as, w, ws, bias,
 * source, W, A[, config])` of actune/kernels/grouped_native.cu:90-115 and
 * grouped_big_m.cu:92-135, and the _group_gemm Triton launch of
 * actune/kernels/grouped.py:74-94, 138-142, for all nine W{2,4,8} x A{2,4,8}
 * pairs. bias may be NULL; bias_dtype gives its element type (the reference
 * keeps it in the weight dtype, or f32 when A == 4, grouped.py:123-125).
 * config: ACTUNE_CONFIG_AUTO or an id below actune_num_configs(); every
 * config gives bit-identical results (fixed chunked fp32 reduction order).
 */
int actune_grouped_linear(const uint8_t* a, const float* a_scales, const uint8_t* w,
                          const float* w_scale, const void* bias, int bias_dtype, void* out,
                          int out_dtype, int64_t M, int64_t N, int64_t K, int W, int A, int config,
                          void* stream);

/*
 * Quantize + linear in one call (two launches): the whole per-call device
 * work of GroupedLinear.forward, actune/kernels/grouped.py:127-143.
 * a_buf [M, K*A/8] and scale_buf [M, K/64] are caller-owned scratch (not
 * written when the quantizer is fused into the GEMM, see below).
 */
int actune_grouped_forward(const void* x, int x_dtype, const void* input_scale, uint8_t* a_buf,
                           float* scale_buf, const uint8_t* w, const float* w_scale, const void* bias,
                           int bias_dtype, void* out, int64_t M, int64_t N, int64_t K, int W, int A,
                           int config, void* stream);

/*
 * Quantize + linear for up to ACTUNE_MAX_TARGETS linears that read the same
 * input x (sibling projections such as q/k/v or gate/up): one quantization
 * and one GEMM launch for all of them. Each target is the computation of
 * GroupedLinear.forward (grouped.py:127-143); results equal separate
 * actune_grouped_forward calls bit for bit. No reference counterpart for the
 * group-64 path; it mirrors the sibling-projection grouping of the
 * reference's tokenwise decode path (actune/kernels/decode_w4a8_triton.py:152-239).
 * The quantizer runs inside the GEMM (a_buf / scale_buf are then not
 * written) for M <= 4 on the small-M and streaming configs and, on the
 * decode configs, for bf16 x wherever the decode kernel's activation passes
 * cover a wave's K-range; otherwise a_buf / scale_buf receive the packed
 * activations and scales.
 * Targets may differ in weight width (actune_linear_target.W; W sizes the
 * call, the widest width when they differ): one decode launch over every
 * width where the decode config takes each of them (in-launch quantization
 * as above), else one quantization and one launch per width on its codes.
 */
int actune_grouped_forward_multi(const void* x, int x_dtype, const void* input_scale, uint8_t* a_buf,
                                 float* scale_buf, const actune_linear_target* targets, int ntargets,
                                 int bias_dtype, int64_t M, int64_t K, int W, int A, int config,
                                 void* stream);

/*
 * 1 when actune_grouped_forward(_multi) with these arguments quantizes x
 * inside the GEMM launch (nothing is written to a_buf / scale_buf), 0 when
 * it launches the quantizer and runs the GEMM on its codes, -1 for invalid
 * arguments. N is the total output width of the call. Lets callers reuse
 * one quantization of x for several linears (no reference counterpart; the
 * reference shares per-row A8 codes the same way, w4a8_triton.py:270-325).
 */
int actune_forward_fuses_quantizer(int64_t M, int64_t N, int64_t K, int W, int A, int x_dtype, int config);

/*
 * actune_grouped_forward without caller-owned scratch: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under
 * stream capture, tight serving loops, harnesses that forbid hipMalloc).
 * The packed activation codes and group scales live in a static device array
 * of 8 MiB per GPU that the library holds until the process ends; calls with
 * M*K*A/8 (rounded up to 256) + M*K/16 bytes above 8388608 are rejected
 * (ACTUNE_ERR_INVALID). All calls on one GPU share that array: calls that
 * overlap on one GPU (two streams or two threads) race. Results equal
 * actune_grouped_forward's bit for bit; nothing is allocated.
 */
int actune_grouped_forward_noalloc(const void* x, int x_dtype, const void* input_scale, const uint8_t* w,
                                   const float* w_scale, const void* bias, int bias_dtype, void* out,
                                   int64_t M, int64_t N, int64_t K, int W, int A, int config, void* stream);

/*
 * Exact per-group int32 dots dots[m][n][g] = sum_{k in g} a[m,k] * w[n,k]
 * computed by the integer path of kernel config `config` (test/debug; the
 * reference has no counterpart, it checks dots only through its float
 * output, tests/test_kernels.py:28-49). dots: [M, N, K/64].
 */
int actune_grouped_dots_i32(const uint8_t* a, const uint8_t* w, int64_t M, int64_t N, int64_t K,
                            int W, int A, int config, int32_t* dots, void* stream);

/*
 * Kernel configurations, the counterpart of the 13 tile geometries of
 * actune/kernels/grouped_big_m.cu:115-130 selected by tuning.py:16-45.
 *   0, 1, 2  small-M split-K kernel with 4, 8, 16 waves (M <= 64)
 *   3 .. 6   MFMA-tiled kernel shapes (any M)
 *   7, 8, 9  persistent streaming kernel with 4, 8, 16 waves (M <= 16)
 *   10 .. 13 prefill kernel (weights streamed per wave, activations staged
 *            per workgroup) with tiles 128x64, 128x32, 64x64, 64x32 (any M)
 *   14 .. 16 decode kernel with 4, 8, 16 waves (M <= 1024 in blocks of 16
 *            tokens; bf16 x quantized in the launch where the in-launch
 *            work is light and a wave's K-range fits its passes, other
 *            dtypes, more tokens and longer
 *            K-ranges through the quantizer launch; a K too long for a
 *            wave's load ring and the dots mode run the small-M kernel with
 *            the same waves)
 * actune_config_valid: 1 if `config` can run a call with M rows.
 * actune_default_config: the config ACTUNE_CONFIG_AUTO resolves to in
 *   actune_grouped_forward(_multi). actune_grouped_linear and
 *   actune_grouped_dots_i32 (packed activations) resolve AUTO to the same
 *   kernels without the in-launch quantization (a decode config where the
 *   decode kernel fits the codes). For a width or dimension that no call
 *   takes it returns ACTUNE_CONFIG_AUTO (-1); a call with such arguments
 *   returns ACTUNE_ERR_INVALID naming them, whatever its config.
 */
int actune_num_configs(void);
int actune_config_valid(int config, int64_t M);
int actune_default_config(int64_t M, int64_t N, int64_t K, int W, int A);

/* ------------------------------------------------------------------------
 * Tokenwise family: per-row dynamic activation scales, full-K int32
 * accumulation. Replaces the reference's tokenwise Triton and CUDA kernels
 * (actune/kernels/w4a8_triton.py, w8a8_triton.py, w2a8_triton.py,
 * decode_w4a8_triton.py, resident_a8_triton.py, wxa4_native.py and
 * native_s4_extension_kernel.cu) with one quantizer and one GEMM over the
 * reference's own weight layouts:
 *   ACTUNE_TW_KMAJOR_W8  int8 [K, N]                  (w8a8_triton.py:106; W8A4 nested codes, wxa4_native.py:334)
 *   ACTUNE_TW_KMAJOR_W4  u8 [K/2, N], byte j = codes j | (j + K/2) << 4   (w4a8_triton.py:380-383)
 *   ACTUNE_TW_KMAJOR_W2  u8 [K/4, N], byte j = codes j + f K/4 at bits 2f (w2a8_triton.py:149-159)
 *   ACTUNE_TW_ROWS_S4    u8 [N, K/2], consecutive nibbles               (wxa4_native.py:206-211)
 *   ACTUNE_TW_ROWS_S2    u8 [N, K/4], consecutive 2-bit fields          (wxa4_native.py:212-219)
 *   ACTUNE_TW_KMAJOR_W4R4  two KMAJOR_W4 buffers, q4 codes and the signed
 *                        R4 residual r4; the weight code is the int8
 *                        16 q4 + r4, wrapped to 8 bits as the reference
 *                        forms it (decode_w4a8_triton.py:61-66), and the
 *                        A8 epilogue uses ws[n] / 16 (:103-104). Through
 *                        actune_tokenwise_linear_multi only, M <= 32; a
 *                        target with no residual reads r4 = 0 (its result
 *                        equals KMAJOR_W4's).
 * Activations: ACTUNE_TW_ACT_A8 int8 codes [M, K]; ACTUNE_TW_ACT_A4 packed
 * [M, K/2] (low nibble = even k). Supported pairs: the K-major layouts with
 * A8, and KMAJOR_W8 / ROWS_S4 / ROWS_S2 with A4.
 * Epilogues (fp32, then rounded to out_dtype):
 *   ACTUNE_TW_EPI_A8  t = f32(acc) * as[m]; y = bias ? fmaf(t, ws[n], bias[n]) : t * ws[n]
 *                     (w4a8_triton.py:105-113, decode_w4a8_triton.py:102-110)
 *   ACTUNE_TW_EPI_A4  q = as[m] * ws[n]; y = bias ? fmaf(f32(acc), q, bias[n]) : f32(acc) * q
 *                     (native_s4_extension_kernel.cu:224-229)
 */
enum {
  ACTUNE_TW_KMAJOR_W8 = 0, ACTUNE_TW_KMAJOR_W4 = 1, ACTUNE_TW_KMAJOR_W2 = 2,
  ACTUNE_TW_ROWS_S4 = 3, ACTUNE_TW_ROWS_S2 = 4, ACTUNE_TW_KMAJOR_W4R4 = 5
};
enum { ACTUNE_TW_ACT_A8 = 0, ACTUNE_TW_ACT_A4 = 1 };
enum { ACTUNE_TW_EPI_A8 = 0, ACTUNE_TW_EPI_A4 = 1 };

/*
 * Per-row dynamic quantizer. Replaces _quantize_rows_kernel
 * (actune/kernels/w4a8_triton.py:161-201; the same arithmetic as
 * _quantize_decode_kernel, decode_w4a8_triton.py:21-28, and
 * _resident_a8_kernel, resident_a8_triton.py:13-21) for A = 8 and
 * _quantize_rows_a4_kernel (wxa4_native.py:28-65) for A = 4:
 *   s = fl(max(max|x|, f32(1e-8)) * fl(1/p)), p = 127 or 7,
 *   c = clamp(rint(x / s), -p-1, p).
 * x: [M, K] (K % 8 == 0, 16-byte aligned); codes: int8 [M, K] (A = 8) or
 * u8 [M, K/2] (A = 4); scales: f32 [M].
 */
int actune_tokenwise_quantize(const void* x, int x_dtype, int64_t M, int64_t K, int A, void* codes,
                              float* scales, void* stream);

/*
 * Bytes of workspace actune_tokenwise_linear needs for this shape (0 when
 * it runs without a K split), or -1 for an invalid shape. The workspace
 * holds the int32 partial sums of the K splits (no state between calls);
 * a split call is two launches, the split GEMM and an integer reduce that
 * finishes the outputs.
 */
int64_t actune_tokenwise_workspace_bytes(int64_t M, int64_t N, int64_t K, int w_layout, int a_layout);

/*
 * Tokenwise packed linear: out[m, n] = epilogue(sum_k a[m, k] w[n, k]) with
 * the exact int32 sum. Replaces _w4a8_gemm_kernel (w4a8_triton.py:57-114),
 * _w8a8_gemm_kernel (w8a8_triton.py:21-77), _w2a8_gemm_kernel
 * (w2a8_triton.py:24-112), the split-K decode pair _decode_partial_kernel +
 * _decode_reduce_kernel (decode_w4a8_triton.py:31-149) and the native
 * linear op (native_s4_extension_kernel.cu:483-573). a_scales: [M];
 * w_scale: [N]; bias: [N] or NULL; out: [M, N]. workspace: at least
 * actune_tokenwise_workspace_bytes() bytes; calls sharing one workspace
 * must not overlap in time. Results do not depend on the split.
 * workspace alignment: 16 bytes.
 */
int actune_tokenwise_linear(const void* a, int a_layout, const float* a_scales, const void* w, int w_layout,
                            const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                            int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * Tokenwise A8 linear of 1-8 rows with the per-row quantizer inside the GEMM
 * launch: the result of actune_tokenwise_quantize (A = 8) on x followed by
 * actune_tokenwise_linear on its codes, bit for bit, in one launch fewer
 * (a split call is the split GEMM and the integer reduce). Writes the rows'
 * activation scales to a_scales[0 .. M-1]; no codes are written. M = 1 takes
 * K <= 16384 and x in bf16, f16 or f32; M = 2, 3-4, 5-8 take K <= 16384,
 * 8192, 4096 and bf16 or f16 x. The weight layout is K-major (the A8 pairs);
 * x: [M, K], 16-byte aligned. Workspace as for actune_tokenwise_linear with
 * a_layout = ACTUNE_TW_ACT_A8. No counterpart in the reference, whose decode
 * launches the quantizer on its own (_quantize_decode_kernel,
 * decode_w4a8_triton.py:21-28); for decode callers.
 */
int actune_tokenwise_linear_x(const void* x, int x_dtype, float* a_scales, const void* w, int w_layout,
                              const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                              int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* One projection of a multi-target tokenwise call. */
typedef struct actune_tw_target {
  const void* w;          /* weights [.., N] in the call's layout */
  const void* r;          /* ACTUNE_TW_KMAJOR_W4R4: residual codes [K/2, N], or NULL; else unused */
  const float* w_scale;   /* [N] */
  const void* bias;       /* [N] in the call's bias dtype, or NULL */
  void* out;              /* [M, N] in out_dtype */
} actune_tw_target;

/*
 * Tokenwise linear for 1 to ACTUNE_MAX_TARGETS sibling projections that read
 * the same activation rows (q/k/v, gate/up) and share N, K and the layouts:
 * one GEMM launch over every target's tiles and K splits, and, when K is
 * split, one integer reduce for all of them. Replaces the grouped decode pair
 * _decode_group_partial_kernel + _decode_group_reduce_kernel
 * (actune/kernels/decode_w4a8_triton.py:150-239, launched by
 * launch_decode_group at :205-239). Each target's output equals
 * actune_tokenwise_linear (codes) or actune_tokenwise_linear_x (rows) on the
 * same operands bit for bit.
 * Exactly one of a / x is non-NULL:
 *   a: activation codes in a_layout, a_scales [M] read;
 *   x: rows [M, K] of x_dtype quantized inside the launch (A8, the rows and
 *      K actune_tokenwise_linear_x takes), a_scales [M] written.
 * workspace: ntargets x actune_tokenwise_workspace_bytes(M, N, K, w_layout,
 * a_layout) bytes (none when that is 0), 16-byte aligned.
 */
int actune_tokenwise_linear_multi(const void* a, int a_layout, const void* x, int x_dtype, float* a_scales,
                                  int w_layout, const actune_tw_target* targets, int ntargets, int bias_dtype,
                                  int out_dtype, int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * Host-only check of the operand element orders the kernels rely on
 * (sub-byte unpack and cross-width reorder for every (W, A) pair). Returns 0
 * when all orders agree; touches no GPU. No reference counterpart.
 */
int actune_layout_selftest(void);

#ifdef __cplusplus
}
#endif

#endif /* ACTUNE_HIP_H */
