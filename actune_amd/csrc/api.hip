// C ABI of libactune_hip.so: argument validation, config selection and
// launches. Declarations and contracts: include/actune_hip.h.
#include <stdio.h>
#include <string.h>

#include <climits>

#include "../../include/actune_hip.h"
#include "common.hpp"
#include "launch.hpp"

using namespace actune;

namespace {

constexpr int kNumConfigs = 7;
constexpr int kSmallMConfigs = 3;  // ids 0..2 need M <= 16
thread_local char g_err[512];

int fail(int code, const char* fmt, const char* detail = "") {
  snprintf(g_err, sizeof g_err, fmt, detail);
  return code;
}

bool width_ok(int b) { return b == 2 || b == 4 || b == 8; }
bool dtype_ok(int d) { return d == kBF16 || d == kF16 || d == kF32; }
bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ACTUNE_ERR_DEVICE, "HIP launch failed: %s", hipGetErrorString(e));
  return ACTUNE_OK;
}

int check_quantize(const void* x, int dt, const void* sc, int64_t M, int64_t K, int A,
                   const uint8_t* packed, const float* scales) {
  if (!width_ok(A)) return fail(ACTUNE_ERR_INVALID, "Unsupported integer width");
  if (!dtype_ok(dt)) return fail(ACTUNE_ERR_INVALID, "unsupported activation dtype");
  if (M < 0 || K <= 0 || K % 64) return fail(ACTUNE_ERR_INVALID, "Grouped backend requires K divisible by 64");
  if (M * (K / 64) / 32 >= INT_MAX) return fail(ACTUNE_ERR_INVALID, "activation too large");
  if (M == 0) return ACTUNE_OK;
  if (!x || !packed || !scales) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(x, 16) || (sc && !aligned(sc, 16)) || !aligned(packed, 8) || !aligned(scales, 4))
    return fail(ACTUNE_ERR_INVALID, "misaligned operand (x/input_scale need 16 B, packed 8 B)");
  return ACTUNE_OK;
}

int check_linear(const uint8_t* a, const float* as, const uint8_t* w, const float* ws, int bias_dt,
                 const void* out, int out_dt, int64_t M, int64_t N, int64_t K, int W, int A, int config) {
  if (!width_ok(W) || !width_ok(A)) return fail(ACTUNE_ERR_INVALID, "Unsupported integer width");
  if (M < 0 || N <= 0 || K <= 0 || K % 64) return fail(ACTUNE_ERR_INVALID, "invalid dimensions");
  if (M > INT_MAX || N > INT_MAX - 64 || K > INT_MAX / 8) return fail(ACTUNE_ERR_INVALID, "dimensions too large");
  if (!dtype_ok(out_dt) || !dtype_ok(bias_dt)) return fail(ACTUNE_ERR_INVALID, "unsupported output/bias dtype");
  if (config < 0 || config >= kNumConfigs) return fail(ACTUNE_ERR_INVALID, "invalid configuration");
  if (config < kSmallMConfigs && M > 16) return fail(ACTUNE_ERR_INVALID, "configuration needs M <= 16");
  if (M == 0) return ACTUNE_OK;
  if (!a || !as || !w || !ws || !out) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(as, 4) || !aligned(ws, 4))
    return fail(ACTUNE_ERR_INVALID, "misaligned operand (packed data needs 16 B)");
  return ACTUNE_OK;
}

int resolve(int config, int64_t M, int64_t N, int64_t K, int W, int A) {
  return config == ACTUNE_CONFIG_AUTO ? actune_default_config(M, N, K, W, A) : config;
}

}  // namespace

extern "C" {

const char* actune_version(void) { return "actune_hip 0.1.0 gfx950"; }

const char* actune_last_error(void) { return g_err; }

int actune_num_configs(void) { return kNumConfigs; }

int actune_config_valid(int config, int64_t M) {
  if (config < 0 || config >= kNumConfigs) return 0;
  return config >= kSmallMConfigs || M <= 16;
}

int actune_default_config(int64_t M, int64_t N, int64_t K, int W, int A) {
  (void)K; (void)W; (void)A;
  if (M <= 16) return 2;
  return M <= 64 ? 3 : 6;
}

int actune_quantize_groups(const void* x, int x_dtype, const void* input_scale, int64_t M, int64_t K,
                           int A, uint8_t* packed, float* scales, void* stream) {
  g_err[0] = 0;
  int rc = check_quantize(x, x_dtype, input_scale, M, K, A, packed, scales);
  if (rc || M == 0) return rc;
  launch_quantize(x, x_dtype, input_scale, M, K, A, packed, scales, (hipStream_t)stream);
  return check_launch();
}

int actune_grouped_linear(const uint8_t* a, const float* a_scales, const uint8_t* w,
                          const float* w_scale, const void* bias, int bias_dtype, void* out,
                          int out_dtype, int64_t M, int64_t N, int64_t K, int W, int A, int config,
                          void* stream) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A);
  int rc = check_linear(a, a_scales, w, w_scale, bias_dtype, out, out_dtype, M, N, K, W, A, config);
  if (rc || M == 0) return rc;
  GemmArgs g{a, a_scales, w, w_scale, bias, bias_dtype, out, out_dtype, nullptr, (int)M, (int)N, (int)K};
  launch_gemm(W, A, config, g, (hipStream_t)stream);
  return check_launch();
}

int actune_grouped_forward(const void* x, int x_dtype, const void* input_scale, uint8_t* a_buf,
                           float* scale_buf, const uint8_t* w, const float* w_scale, const void* bias,
                           int bias_dtype, void* out, int64_t M, int64_t N, int64_t K, int W, int A,
                           int config, void* stream) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A);
  int rc = check_quantize(x, x_dtype, input_scale, M, K, A, a_buf, scale_buf);
  if (!rc) rc = check_linear(a_buf, scale_buf, w, w_scale, bias_dtype, out, x_dtype, M, N, K, W, A, config);
  if (rc || M == 0) return rc;
  launch_quantize(x, x_dtype, input_scale, M, K, A, a_buf, scale_buf, (hipStream_t)stream);
  GemmArgs g{a_buf, scale_buf, w, w_scale, bias, bias_dtype, out, x_dtype, nullptr, (int)M, (int)N, (int)K};
  launch_gemm(W, A, config, g, (hipStream_t)stream);
  return check_launch();
}

int actune_grouped_dots_i32(const uint8_t* a, const uint8_t* w, int64_t M, int64_t N, int64_t K,
                            int W, int A, int config, int32_t* dots, void* stream) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A);
  // scales/out are unused in the dots mode; pass a and w to satisfy the null checks
  int rc = check_linear(a, (const float*)w, w, (const float*)w, kF32, dots, kF32, M, N, K, W, A, config);
  if (rc || M == 0) return rc;
  if (!aligned(dots, 4)) return fail(ACTUNE_ERR_INVALID, "misaligned dots buffer");
  GemmArgs g{a, nullptr, w, nullptr, nullptr, kF32, nullptr, kF32, dots, (int)M, (int)N, (int)K};
  launch_dots(W, A, config, g, (hipStream_t)stream);
  return check_launch();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Host-only self-test of the operand element orders.
namespace {

template <int B>
int check_unpack(unsigned seed) {
  int codes[16];
  uint8_t bytes[16] = {0};
  for (int e = 0; e < 16; ++e) {
    seed = seed * 1103515245u + 12345u;
    const int lo = -(1 << (B - 1)), span = 1 << B;
    codes[e] = lo + (int)((seed >> 16) % (unsigned)span);
    const int per = 8 / B;
    bytes[e / per] |= (uint8_t)((codes[e] & ((1 << B) - 1)) << ((e % per) * B));
  }
  uint32_t p[4];
  memcpy(p, bytes, sizeof p);
  uint32_t d[4];
  unpack_slot<B>(p, d);
  for (int r = 0; r < 4; ++r)
    for (int t = 0; t < 4; ++t) {
      const int8_t got = (int8_t)((d[r] >> (8 * t)) & 0xffu);
      if (got != (int8_t)(codes[slot_elem(B, r, t)] * (1 << (8 - B)))) return 1;
    }
  return 0;
}

template <int FROM, int TO>
int check_reorder(unsigned seed) {
  uint32_t d[4];
  int vals[16];
  for (int e = 0; e < 16; ++e) { seed = seed * 1664525u + 1013904223u; vals[e] = (int)(seed >> 24); }
  for (int r = 0; r < 4; ++r) {
    d[r] = 0;
    for (int t = 0; t < 4; ++t) d[r] |= (uint32_t)(vals[slot_elem(FROM, r, t)] & 0xff) << (8 * t);
  }
  reorder_slot<FROM, TO>(d);
  for (int r = 0; r < 4; ++r)
    for (int t = 0; t < 4; ++t)
      if ((int)((d[r] >> (8 * t)) & 0xffu) != (vals[slot_elem(TO, r, t)] & 0xff)) return 1;
  return 0;
}

}  // namespace

extern "C" int actune_layout_selftest(void) {
  int bad = 0;
  for (unsigned s = 1; s < 64; ++s) {
    bad |= check_unpack<8>(s) << 0;
    bad |= check_unpack<4>(s) << 1;
    bad |= check_unpack<2>(s) << 2;
    bad |= check_reorder<8, 4>(s) << 3;
    bad |= check_reorder<4, 8>(s) << 4;
    bad |= check_reorder<8, 2>(s) << 5;
    bad |= check_reorder<2, 8>(s) << 6;
    bad |= check_reorder<4, 2>(s) << 7;
    bad |= check_reorder<2, 4>(s) << 8;
  }
  // chunk bounds cover [0, G) in order for every G up to 4096 groups
  for (int G = 1; G <= 4096 && !bad; ++G) {
    if (chunk_begin(0, G) != 0 || chunk_begin(kChunks, G) != G) bad |= 1 << 9;
    for (int c = 0; c < kChunks; ++c)
      if (chunk_begin(c + 1, G) < chunk_begin(c, G) || (chunk_begin(c, G) % 4 && chunk_begin(c, G) != G))
        bad |= 1 << 9;
  }
  if (bad) snprintf(g_err, sizeof g_err, "layout self-test failed, mask 0x%x", bad);
  return bad;
}
