/*
 * CPU oracle for the tokenwise (per-row) packed-integer linears.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library (actune_amd/) may
 * link, load or call this file; only tests/ use it, as the checker.
 *
 * Plain C restatement of the reference arithmetic (zanehpn/Actune):
 *   per-row A8 quantizer   actune/kernels/w4a8_triton.py:161-201 (fused),
 *                          :400-401 (eager), decode_w4a8_triton.py:21-28,
 *                          resident_a8_triton.py:13-21
 *   per-row A4 quantizer   actune/kernels/wxa4_native.py:28-65
 *   epilogue, A8 family    w4a8_triton.py:105-113, w8a8_triton.py:64-76,
 *                          w2a8_triton.py:99-111, decode_w4a8_triton.py:102-110
 *   epilogue, native A4    native_s4_extension_kernel.cu:224-229 (and :332-338,
 *                          :472-478)
 *
 * Build with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() and every other operation rounds on its own, exactly as written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_bf16_to_f32(uint16_t b);
float oracle_f16_to_f32(uint16_t h);

enum { TW_DT_BF16 = 0, TW_DT_F16 = 1, TW_DT_F32 = 2 };

static float tw_load(const void* p, int dtype, int64_t i) {
  if (dtype == TW_DT_BF16) return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == TW_DT_F16) return oracle_f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

/* fp32 reciprocal of the code bound p (127 or 7), as both reference forms
 * produce it: torch's GPU tensor/scalar division computes 1.0f / p in fp32
 * on the host, Triton rounds the Python double 1.0 / p to fp32; both equal
 * the correctly rounded fp32 reciprocal for p in {7, 127} (pinned by
 * tests/test_oracle_tokenwise.py with exact rational arithmetic). */
float oracle_tw_recip(int p) {
  volatile float one = 1.0f, fp = (float)p;
  return one / fp;
}

/*
 * Per-row dynamic quantizer: p = 127 (bits 8) or 7 (bits 4),
 *   s = fl32(max(max|v|, f32(1e-8)) * fl32(1/p))        (reciprocal multiply)
 *   c = clamp(rint_half_even(fl32(v / s)), -p-1, p)      (IEEE division)
 * over all K elements of each row. codes: [M, K] int8, scales: [M].
 */
int oracle_tw_quantize_rows(const void* x, int dtype, int64_t M, int64_t K, int bits, int8_t* codes,
                            float* scales) {
  if ((bits != 8 && bits != 4) || K <= 0 || M < 0 || dtype < 0 || dtype > 2) return -1;
  const int p = bits == 8 ? 127 : 7;
  const float r = oracle_tw_recip(p);
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(tw_load(x, dtype, m * K + k));
      if (a > amax) amax = a;
    }
    if (amax < 1e-8f) amax = 1e-8f;
    const float s = amax * r;
    scales[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float c = rintf(tw_load(x, dtype, m * K + k) / s);
      if (c < (float)(-p - 1)) c = (float)(-p - 1);
      if (c > (float)p) c = (float)p;
      codes[m * K + k] = (int8_t)c;
    }
  }
  return 0;
}

/*
 * Output epilogue on exact int32 accumulators acc [M, N]:
 *   mode 0 (A8 family and the decode reduce):
 *       t = fl(f32(acc) * as[m]);  y = bias ? fmaf(t, ws[n], bias[n]) : fl(t * ws[n])
 *   mode 1 (native A4 kernels):
 *       q = fl(as[m] * ws[n]);     y = bias ? fmaf(f32(acc), q, bias[n]) : fl(f32(acc) * q)
 * f32(acc) is the round-to-nearest-even int32 -> fp32 conversion. The bias
 * add is taken fused with the preceding product (the reference compilers
 * contract a product followed by an add; without a bias nothing is fused).
 * bias (nullable) is the fp32 value of each bias element.
 */
int oracle_tw_epilogue(const int32_t* acc, int64_t M, int64_t N, const float* as, const float* ws,
                       const float* bias, int mode, float* out) {
  if (mode != 0 && mode != 1) return -1;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const float a = (float)acc[m * N + n];
      float y;
      if (mode == 0) {
        const float t = a * as[m];
        y = bias ? fmaf(t, ws[n], bias[n]) : t * ws[n];
      } else {
        const float q = as[m] * ws[n];
        y = bias ? fmaf(a, q, bias[n]) : a * q;
      }
      out[m * N + n] = y;
    }
  return 0;
}
