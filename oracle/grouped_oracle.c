/*
 * CPU oracle for the group-64 packed-integer linear path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library (actune_amd/) may
 * link, load or call this file; only tests/, the smoke check and the CPU
 * baseline leg of bench.py use it, and only as the checker.
 *
 * Plain C restatement of the reference arithmetic (zanehpn/Actune):
 *   activation quantizer  actune/calibration.py:7-16, actune/kernels/grouped.py:55-71
 *   input channel scale   actune/layers.py:40-42
 *   weight codebooks      actune/kernels/quantizers.py:4-94
 *   packing               actune/kernels/grouped.py:67-71, 108-111
 *   int32 group dots      actune/kernels/grouped.py:83-89, grouped_native.cu:59-74
 *   fp32 group epilogue   actune/kernels/grouped.py:90-94, grouped_native.cu:75,85
 *
 * Build with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() and every other operation rounds on its own, exactly as written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* dtype codes shared with the product ABI: 0 = bf16, 1 = f16, 2 = f32 */
enum { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);  /* round to nearest, ties to even */
  return (uint16_t)(u >> 16);
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;  /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x = f32_bits(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);       /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                           /* f16 subnormal range */
    float r = rintf(bits_f32(ax) * 16777216.0f);                    /* |f| * 2^24, exact scaling */
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t mant = ax & 0x7fffffu, h = ((((ax >> 23) - 112u)) << 10) | (mant >> 13), rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

static float load_elem(const void* p, int dtype, int64_t i) {
  if (dtype == DT_BF16) return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == DT_F16) return oracle_f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

/* Round an fp32 value to the storage dtype and back (x / input_scale produces
 * a tensor of the activation dtype before quantization, layers.py:41-42). */
static float round_to_dtype(float v, int dtype) {
  if (dtype == DT_BF16) return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
  if (dtype == DT_F16) return oracle_f16_to_f32(oracle_f32_to_f16(v));
  return v;
}

/*
 * Group-64 activation quantizer (calibration.py:12-14; grouped.py:62-71):
 *   p = 2^(A-1)-1, s = fl32(max(amax, f32(1e-8)) / p),
 *   c = clamp(rint_half_even(fl32(v / s)), -p-1, p),
 *   code k of row m lands in byte m*(K*A/8) + k*A/8 at bit (k % (8/A))*A.
 * input_scale (nullable, same dtype as x, length K) divides x first and
 * rounds the quotient to x's dtype (layers.py:41-42).
 * codes (nullable) receives the unpacked int8 codes [M,K].
 */
int oracle_quantize_groups(const void* x, int dtype, const void* input_scale, int64_t M, int64_t K,
                           int A, uint8_t* packed, float* scales, int8_t* codes) {
  if ((A != 2 && A != 4 && A != 8) || K % 64 || M < 0 || dtype < 0 || dtype > 2) return -1;
  const int p = (1 << (A - 1)) - 1, per = 8 / A;
  const int64_t G = K / 64, row_bytes = K * A / 8;
  float v[64];
  for (int64_t m = 0; m < M; ++m) {
    memset(packed + m * row_bytes, 0, (size_t)row_bytes);
    for (int64_t g = 0; g < G; ++g) {
      float amax = 0.0f;
      for (int j = 0; j < 64; ++j) {
        int64_t k = g * 64 + j;
        float t = load_elem(x, dtype, m * K + k);
        if (input_scale) t = round_to_dtype(t / load_elem(input_scale, dtype, k), dtype);
        v[j] = t;
        float a = fabsf(t);
        if (a > amax) amax = a;
      }
      if (amax < 1e-8f) amax = 1e-8f;
      const float s = amax / (float)p;
      scales[m * G + g] = s;
      for (int j = 0; j < 64; ++j) {
        float c = rintf(v[j] / s);
        if (c < (float)(-p - 1)) c = (float)(-p - 1);
        if (c > (float)p) c = (float)p;
        int ci = (int)c;
        int64_t k = g * 64 + j;
        if (codes) codes[m * K + k] = (int8_t)ci;
        packed[m * row_bytes + k / per] |= (uint8_t)((ci & ((1 << A) - 1)) << ((k % per) * A));
      }
    }
  }
  return 0;
}

/*
 * Per-output-row weight codebooks (quantizers.py):
 *   W2      s = amax*r,          c = clamp(rint(v/s), -2, 1)        (:59-81)
 *   W4      s = (amax*r)/7,      c = clamp(rint(v/s), -8, 7)        (:23-40)
 *   W8,A=4  nested 16*q4 + r4 with residual bounds, s = s4/16       (:42-57, :88-91)
 *   W8,A!=4 s = amax/127 (ratios ignored), c = clamp(rint(v/s), -128, 127) (:92-94)
 * amax = max|v| clamped to >= f32(1e-8). ratios (nullable) is per row, already
 * validated to lie in (0,1]. w is the fp32 image of the weight, [N,K].
 */
/* amax / p: the IEEE quotient (recip == 0: torch-CPU, and torch-GPU
 * tensor/tensor division), or amax times the fp32 reciprocal of p (recip ==
 * 1: torch-GPU division of a tensor by a Python scalar, which multiplies by
 * 1.0f / p computed in fp32; the reference's note, w4a8_triton.py:33-36). */
static float div_const(float amax, float p, int recip) {
  if (!recip) return amax / p;
  volatile float one = 1.0f;
  const float r = one / p;
  return amax * r;
}

static int weight_codes_impl(const float* w, int64_t N, int64_t K, int W, int A, const float* ratios,
                             int recip, int8_t* codes, float* scale) {
  if ((W != 2 && W != 4 && W != 8) || (A != 2 && A != 4 && A != 8)) return -1;
  for (int64_t n = 0; n < N; ++n) {
    const float* v = w + n * K;
    int8_t* c = codes + n * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) { float a = fabsf(v[k]); if (a > amax) amax = a; }
    if (amax < 1e-8f) amax = 1e-8f;
    if (W == 8 && A != 4) {
      const float s = div_const(amax, 127.0f, recip);
      scale[n] = s;
      for (int64_t k = 0; k < K; ++k) {
        float q = rintf(v[k] / s);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        c[k] = (int8_t)q;
      }
      continue;
    }
    if (ratios) amax = amax * ratios[n];
    if (W == 2) {
      const float s = amax;
      scale[n] = s;
      for (int64_t k = 0; k < K; ++k) {
        float q = rintf(v[k] / s);
        q = q < -2.0f ? -2.0f : (q > 1.0f ? 1.0f : q);
        c[k] = (int8_t)q;
      }
      continue;
    }
    const float s4 = div_const(amax, 7.0f, recip);
    for (int64_t k = 0; k < K; ++k) {
      const float t = v[k] / s4;
      float q = rintf(t);
      q = q < -8.0f ? -8.0f : (q > 7.0f ? 7.0f : q);
      const int q4 = (int)q;
      if (W == 4) { c[k] = (int8_t)q4; continue; }
      /* signed_r4_refine (quantizers.py:42-57) */
      const float rf = 16.0f * (t - (float)q4);
      float r = rintf(rf);
      r = r < -8.0f ? -8.0f : (r > 7.0f ? 7.0f : r);
      int ri = (int)r;
      const int lower = -128 - 16 * q4 > -8 ? -128 - 16 * q4 : -8;
      const int upper = 127 - 16 * q4 < 7 ? 127 - 16 * q4 : 7;
      if (ri < lower) ri = lower;
      if (ri > upper) ri = upper;
      c[k] = (int8_t)(16 * q4 + ri);
    }
    scale[n] = W == 4 ? s4 : s4 / 16.0f;
  }
  return 0;
}

int oracle_weight_codes(const float* w, int64_t N, int64_t K, int W, int A, const float* ratios,
                        int8_t* codes, float* scale) {
  return weight_codes_impl(w, N, K, W, A, ratios, 0, codes, scale);
}

/* The same codebooks as computed by torch on a GPU-resident weight: the two
 * divisions by the constants 7 and 127 multiply by their fp32 reciprocals
 * (every other division is tensor / tensor, IEEE on both devices). */
int oracle_weight_codes_recip(const float* w, int64_t N, int64_t K, int W, int A, const float* ratios,
                              int8_t* codes, float* scale) {
  return weight_codes_impl(w, N, K, W, A, ratios, 1, codes, scale);
}

/* Row-major, K-contiguous little-endian packing (grouped.py:108-111). */
int oracle_pack_rows(const int8_t* codes, int64_t R, int64_t K, int bits, uint8_t* out) {
  if ((bits != 2 && bits != 4 && bits != 8) || (K * bits) % 8) return -1;
  const int per = 8 / bits;
  const int64_t rb = K * bits / 8;
  memset(out, 0, (size_t)(R * rb));
  for (int64_t r = 0; r < R; ++r)
    for (int64_t k = 0; k < K; ++k)
      out[r * rb + k / per] |= (uint8_t)((codes[r * K + k] & ((1 << bits) - 1)) << ((k % per) * bits));
  return 0;
}

/* Sign-extending unpack ((u ^ 2^(b-1)) - 2^(b-1)), grouped.py:83-88. */
int oracle_unpack_rows(const uint8_t* packed, int64_t R, int64_t K, int bits, int8_t* codes) {
  if (bits != 2 && bits != 4 && bits != 8) return -1;
  const int per = 8 / bits, half = 1 << (bits - 1);
  const int64_t rb = K * bits / 8;
  for (int64_t r = 0; r < R; ++r)
    for (int64_t k = 0; k < K; ++k) {
      int u = (packed[r * rb + k / per] >> ((k % per) * bits)) & ((1 << bits) - 1);
      codes[r * K + k] = (int8_t)((u ^ half) - half);
    }
  return 0;
}

/*
 * Exact per-group integer dots: dots[m][n][g] = sum_{k in g} a[m,k]*w[n,k]
 * (grouped.py:89, grouped_native.cu:70-74). rows/cols (nullable) select a
 * subset of output rows m and columns n; dots is [nr][nc][G].
 */
int oracle_group_dots(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K,
                      const int64_t* rows, int64_t nr, const int64_t* cols, int64_t nc, int32_t* dots) {
  if (K % 64) return -1;
  const int64_t G = K / 64;
  if (!rows) nr = M;
  if (!cols) nc = N;
  for (int64_t i = 0; i < nr; ++i) {
    const int64_t m = rows ? rows[i] : i;
    for (int64_t j = 0; j < nc; ++j) {
      const int64_t n = cols ? cols[j] : j;
      const int8_t* ar = a + m * K;
      const int8_t* wr = w + n * K;
      for (int64_t g = 0; g < G; ++g) {
        int32_t d = 0;
        for (int t = 0; t < 64; ++t) d += (int32_t)ar[g * 64 + t] * (int32_t)wr[g * 64 + t];
        dots[(i * nc + j) * G + g] = d;
      }
    }
  }
  return 0;
}

/*
 * fp32 epilogue over precomputed dots, with an explicit reduction order.
 * bounds[0..nsplit] partitions the G groups into contiguous chunks; each chunk
 * is summed sequentially from +0 as acc = fmaf(f32(d_g), as[m,g], acc)
 * (grouped_native.cu:75 / grouped.py:91), chunk partials are added in chunk
 * order, then y = fmaf(acc, ws[n], bias[n]) with a bias, else acc*ws[n]
 * (grouped_native.cu:85 / grouped.py:92-93). bounds == NULL means one chunk
 * [0, G): the sequential order of the reference kernels.
 * dots is [nr][nc][G]; as is the full [M][G] scale array; out is [nr][nc].
 */
int oracle_group_epilogue(const int32_t* dots, const float* as, const float* ws, const float* bias,
                          int64_t G, const int64_t* rows, int64_t nr, const int64_t* cols, int64_t nc,
                          const int64_t* bounds, int64_t nsplit, float* out) {
  int64_t seq[2] = {0, G};
  if (!bounds) { bounds = seq; nsplit = 1; }
  if (nsplit < 1 || bounds[0] != 0 || bounds[nsplit] != G) return -1;
  for (int64_t i = 0; i < nr; ++i) {
    const int64_t m = rows ? rows[i] : i;
    for (int64_t j = 0; j < nc; ++j) {
      const int64_t n = cols ? cols[j] : j;
      const int32_t* d = dots + (i * nc + j) * G;
      float acc = 0.0f;
      for (int64_t s = 0; s < nsplit; ++s) {
        float part = 0.0f;
        for (int64_t g = bounds[s]; g < bounds[s + 1]; ++g) part = fmaf((float)d[g], as[m * G + g], part);
        acc = s == 0 ? part : acc + part;
      }
      out[i * nc + j] = bias ? fmaf(acc, ws[n], bias[n]) : acc * ws[n];
    }
  }
  return 0;
}

/* Rounds an fp32 buffer to bf16 / f16 bit patterns (RNE), for output dtypes. */
void oracle_round_out(const float* in, int64_t n, int dtype, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = dtype == DT_BF16 ? oracle_f32_to_bf16(in[i]) : oracle_f32_to_f16(in[i]);
}
