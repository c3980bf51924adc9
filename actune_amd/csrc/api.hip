// C ABI of libactune_hip.so: argument validation, config selection and
// launches. Declarations and contracts: include/actune_hip.h.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <climits>

#include "../../include/actune_hip.h"
#include "common.hpp"
#include "launch.hpp"

using namespace actune;

namespace {

constexpr int kNumConfigs = 17;
constexpr int kSmallMConfigs = 3;  // ids 0..2: small-M kernel, M <= kSmallMMax
constexpr int kSmallMMax = 64;
constexpr int kTiledConfigs = 4;   // ids 3..6: MFMA-tiled kernel, any M
constexpr int kStreamFirst = kSmallMConfigs + kTiledConfigs;  // ids 7..9: streaming kernel, M <= 16
constexpr int kStreamMax = 16;
constexpr int kStreamConfigs = 3;
constexpr int kPrefillFirst = kStreamFirst + kStreamConfigs;  // ids 10..13: prefill kernel, any M
constexpr int kPrefillConfigs = 4;
constexpr int kDecodeFirst = kPrefillFirst + kPrefillConfigs;  // ids 14..16: decode kernel, M <= 1024
constexpr int kDecodeMax = 1024;      // decode configs: 16-token blocks on grid z
constexpr int kDecodeAutoMax = 64;   // decode_packed_config and the small-M defaults up to this M
constexpr int kFusedMaxM = 4;      // small-M and streaming calls up to this M quantize inside the GEMM
constexpr int kSmallMWaves[kSmallMConfigs] = {4, 8, 16};
thread_local char g_err[512];
// Kernels address every operand through 32-bit buffer offsets and use
// 2^31 as the "no load" offset, so each operand buffer must stay below 2 GiB.
constexpr int64_t kMaxBufferBytes = (int64_t)1 << 31;

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
  // (bounds on M and K first, so that the group count cannot overflow)
  if (M > INT_MAX || K > INT_MAX / 8 || M * (K / 64) / 32 >= INT_MAX)
    return fail(ACTUNE_ERR_INVALID, "activation too large");
  if (M == 0) return ACTUNE_OK;
  if (!x || !packed || !scales) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(x, 16) || (sc && !aligned(sc, 16)) || !aligned(packed, 8) || !aligned(scales, 4))
    return fail(ACTUNE_ERR_INVALID, "misaligned operand (x/input_scale need 16 B, packed 8 B)");
  return ACTUNE_OK;
}

int check_shape(int64_t M, int64_t K, int W, int A, int out_dt, int bias_dt, int config) {
  if (!width_ok(W) || !width_ok(A)) return fail(ACTUNE_ERR_INVALID, "Unsupported integer width");
  if (M < 0 || K <= 0 || K % 64) return fail(ACTUNE_ERR_INVALID, "invalid dimensions");
  if (M > INT_MAX || K > INT_MAX / 8) return fail(ACTUNE_ERR_INVALID, "dimensions too large");
  if (M * K * 4 >= kMaxBufferBytes) return fail(ACTUNE_ERR_INVALID, "operand too large (each buffer must stay below 2 GiB)");
  if (!dtype_ok(out_dt) || !dtype_ok(bias_dt)) return fail(ACTUNE_ERR_INVALID, "unsupported output/bias dtype");
  if (config < 0 || config >= kNumConfigs) return fail(ACTUNE_ERR_INVALID, "invalid configuration");
  if (config < kSmallMConfigs && M > kSmallMMax) return fail(ACTUNE_ERR_INVALID, "configuration needs M <= 64");
  if (config >= kStreamFirst && config < kPrefillFirst && M > kStreamMax)
    return fail(ACTUNE_ERR_INVALID, "configuration needs M <= 16");
  if (config >= kDecodeFirst && M > kDecodeMax) return fail(ACTUNE_ERR_INVALID, "configuration needs M <= 1024");
  return ACTUNE_OK;
}

int check_target(const uint8_t* w, const float* ws, const void* out, int64_t N, int64_t M, int64_t K, int W) {
  if (N <= 0 || N > INT_MAX / 2) return fail(ACTUNE_ERR_INVALID, "invalid dimensions");
  if (N * K * W / 8 >= kMaxBufferBytes || M * N * 4 >= kMaxBufferBytes)
    return fail(ACTUNE_ERR_INVALID, "operand too large (each buffer must stay below 2 GiB)");
  if (M == 0) return ACTUNE_OK;
  if (!w || !ws || !out) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(w, 16) || !aligned(ws, 4)) return fail(ACTUNE_ERR_INVALID, "misaligned operand (packed data needs 16 B)");
  return ACTUNE_OK;
}

int packed_default(int64_t M, int64_t N, int64_t K, int W, int A);

// Whether a decode-config call quantizes x inside the GEMM. Every workgroup
// quantizes the whole activation, so the in-launch work grows as workgroups
// (row tiles / tiles per workgroup) x groups x tokens; measured on MI355X
// (W4A8, M = 1..8, N = 2048..22016), past about 180 (4-token tiles) or 160
// (one 16-token block, M = 9..16) group-rows per SIMD (1024 SIMDs) the
// quantizer launch followed by the GEMM on its codes is faster. With
// 8-token tiles (M = 5..8) the limit is 300: every launch measured up to 301
// was faster fused (W4A8 and W2A8 2 x 11008x4096, W4A8 22016x4096, M = 5-7:
// +0.3 to +9%, e.g. W4A8 2 x 11008x4096 at M = 5 16.3 -> 14.9 us), at 344
// one was slower (W2A8 2 x 11008x4096 at M = 8: 13.4 against 14.1 us).
// With 16-token blocks (M > 16) the limit is 200: at M = 50 every launch
// measured at 200 was faster fused (W4A4 4096x1024 8.9 -> 8.5 us, 8192x1024
// and 2 x 4096x1024 12.3 -> 11.5 and 12.6 -> 12.0 us, 2048x2048 8.2 -> 7.7
// us), at 256 some were slower (8192x1024 at M = 64: 13.0 against 13.4 us).
// Where the codes path cannot run the decode kernel (M <= 4), the fused
// small-M kernel runs instead.
// compact: as for decode_row_tiles (false for the mixed-width kernel).
bool decode_light(int64_t M, int64_t n_total, int64_t K, int W, int nw, bool compact = true) {
  const int64_t tiles = (n_total + 15) / 16;
  const int tr = decode_row_tiles((int)K, (int)M, W, nw, (int)std::min<int64_t>(tiles, INT_MAX), 1, compact);
  const int64_t limit = (M <= kFusedMaxM ? 180 : M <= 8 ? 300 : M <= 16 ? 160 : 200) * 1024;
  return (tiles + tr - 1) / tr * (K / kGroup) * M <= limit;
}

bool decode_fused(int64_t M, int64_t n_total, int64_t K, int W, int nw, int x_dt) {
  if (decode_fits((int)K, (int)M, W, nw, false, x_dt) && decode_light(M, n_total, K, W, nw)) return true;
  return M <= kFusedMaxM && !decode_fits((int)K, (int)M, W, nw, true, x_dt);
}

// Whether a forward call on x with the (resolved) config quantizes x inside
// the GEMM launch. The quantizer is fused into the GEMM for M <= 4 on the
// small-M and streaming kernels (for larger M its per-workgroup cost is no
// longer hidden under the weight loads; measured on MI355X). On the decode
// configs decode_fused decides.
bool forward_fuses(int config, int64_t M, int64_t n_total, int64_t K, int W, int x_dt) {
  if (config >= kDecodeFirst) return decode_fused(M, n_total, K, W, kSmallMWaves[config - kDecodeFirst], x_dt);
  return M <= kFusedMaxM && (config < kSmallMConfigs || (config >= kStreamFirst && config < kPrefillFirst));
}

// Arguments some call can take: the config selection reasons only about
// these (its arithmetic divides by the widths and casts the dimensions).
bool selectable(int64_t M, int64_t N, int64_t K, int W, int A) {
  return width_ok(W) && width_ok(A) && M >= 0 && M <= INT_MAX && N > 0 && N <= INT_MAX / 2 && K > 0 &&
         K % kGroup == 0 && K <= INT_MAX / 8;
}

// ACTUNE_CONFIG_AUTO: calls that hand over x (and may fuse the quantizer) use
// actune_default_config; calls on packed activations use packed_default (the
// same choice without the in-launch quantization). Arguments no call takes
// resolve to the first prefill config, valid at every M, so that the call's
// own checks name what is wrong.
int resolve(int config, int64_t M, int64_t N, int64_t K, int W, int A, bool has_x) {
  if (config != ACTUNE_CONFIG_AUTO) return config;
  if (!selectable(M, N, K, W, A)) return kPrefillFirst;
  return has_x ? actune_default_config(M, N, K, W, A) : packed_default(M, N, K, W, A);
}

// Fill the problem table of a launch; returns the number of 16-row tiles.
int add_problem(LinearArgs& g, const uint8_t* w, const float* ws, const void* bias, void* out, int64_t N, int W) {
  Problem& p = g.prob[g.nprob++];
  p = Problem{w, ws, bias, out, (int)N, g.tiles, W};
  g.tiles += (int)((N + 15) / 16);
  return g.tiles;
}

// Launch the GEMM of `g` (all problems) with kernel config `config`. A
// streaming config whose LDS staging would not fit (or the dots mode) runs
// the small-M kernel with the same wave count; results are identical.
void run_gemm(int W, int A, int config, int mode, const LinearArgs& g, hipStream_t st) {
  if (config >= kDecodeFirst) {
    // the decode kernel serves the fused (bf16 x) and packed modes where a
    // wave's K-range fits its loads; other calls and the dots mode run the
    // small-M kernel with the same wave count
    const int nw = kSmallMWaves[config - kDecodeFirst];
    if (mode != kModeDots && decode_fits(g.K, g.M, W, nw, mode == kModePacked, g.x_dt)) {
      launch_decode(W, A, nw, mode == kModePacked, g, st);
      return;
    }
    launch_smallm(W, A, nw, mode, g, st);
    return;
  }
  if (config >= kPrefillFirst) {
    for (int p = 0; p < g.nprob; ++p) {
      LinearArgs one = g;
      one.prob[0] = g.prob[p];
      one.prob[0].tile0 = 0;
      one.nprob = 1;
      launch_prefill(W, A, config - kPrefillFirst, mode == kModeDots, one, st);
    }
    return;
  }
  if (config >= kStreamFirst) {
    const int nw = kSmallMWaves[config - kStreamFirst];
    if (mode != kModeDots && stream_lds_bytes(g.K, g.M, nw) <= kStreamLdsMax) {
      launch_stream(W, A, nw, mode, g, st);
      return;
    }
    config -= kStreamFirst;
  }
  if (config < kSmallMConfigs) {
    launch_smallm(W, A, kSmallMWaves[config], mode, g, st);
    return;
  }
  for (int p = 0; p < g.nprob; ++p) {
    LinearArgs one = g;
    one.prob[0] = g.prob[p];
    one.prob[0].tile0 = 0;
    one.nprob = 1;
    launch_tiled(W, A, config - kSmallMConfigs, mode == kModeDots, one, st);
  }
}

LinearArgs base_args(int64_t M, int64_t K, int bias_dt, int out_dt) {
  LinearArgs g{};
  g.M = (int)M;
  g.K = (int)K;
  g.bias_dt = bias_dt;
  g.out_dt = out_dt;
  g.m_div = M > 0 ? (uint32_t)((65536 + M - 1) / M) : 0u;
  const int64_t tail = M > 0 ? M - 16 * ((M - 1) / 16) : 0;
  g.m_div_tail = tail > 0 ? (uint32_t)((65536 + tail - 1) / tail) : 0u;
  return g;
}

}  // namespace

void actune::set_last_error(const char* msg) { snprintf(g_err, sizeof g_err, "%s", msg); }

extern "C" {

const char* actune_version(void) { return "actune_hip 0.2.0 gfx950"; }

const char* actune_last_error(void) { return g_err; }

int actune_num_configs(void) { return kNumConfigs; }

int actune_config_valid(int config, int64_t M) {
  if (config < 0 || config >= kNumConfigs) return 0;
  if (config < kSmallMConfigs) return M <= kSmallMMax;
  if (config >= kStreamFirst && config < kPrefillFirst) return M <= kStreamMax;
  if (config >= kDecodeFirst) return M <= kDecodeMax;
  return 1;
}

namespace {
// Waves of a decode workgroup that get work: the canonical chunks split K
// into min(16, ceil(G/4)) nonempty quads, so a wave count above that leaves
// waves with an empty K-range that still load and quantize nothing but cost
// their launch and barrier time (measured on MI355X at K = 1024 / 2048:
// 16 waves 0.9-1.7 us slower than 4 or 8).
bool decode_waves_useful(int64_t K, int nw) {
  const int64_t q = (K / kGroup + 3) / 4;
  return nw <= 4 || nw <= q;
}
}  // namespace

int actune_default_config(int64_t M, int64_t N, int64_t K, int W, int A) {
  if (!selectable(M, N, K, W, A)) return ACTUNE_CONFIG_AUTO;
  // Decode (M <= 64, measured on MI355X at Llama/Gemma shapes): the decode
  // kernel beats the small-M and streaming kernels wherever a wave's K-range
  // fits its load ring. Calls that hand over bf16 x first try to quantize it
  // inside the launch (where light), then use the quantizer's codes
  // (packed_default, which also sends narrow problems above 64 tokens to the
  // decode kernel).
  const int64_t tiles = (N + 15) / 16;
  auto fused_at = [&](int c) {
    const int nw = kSmallMWaves[c];
    return decode_fits((int)K, (int)M, W, nw, false, kBF16) && decode_light(M, N, K, W, nw);
  };
  if (M >= 2 && M <= kDecodeAutoMax && tiles > 256) {
    // Wide N: several row tiles share a workgroup and its quantized x
    // (decode_row_tiles); 16 waves, whose short K-ranges allow four tiles,
    // below 1024 row tiles, 8 waves from there on. Two tokens below 1024 row
    // tiles: one tile per 4-wave workgroup, as for M = 1 (measured W4A8
    // 11008x4096 8.9 -> 7.8 us, 12288x4096 9.1 -> 8.2 us). Where K gives
    // that many waves no work (decode_waves_useful), the most waves that all
    // get work: at K = 1024, 4 waves against 16 for 8192 rows (W4A4 and
    // W2A4, also as 2 x 4096) are 12-35% faster at M = 4..32 (M = 17: 7.5
    // against 11.5 us).
    if (M == 2 && tiles < 1024 && fused_at(0)) return kDecodeFirst;
    int pref = tiles >= 1024 ? 1 : 2;
    while (pref > 0 && !decode_waves_useful(K, kSmallMWaves[pref])) --pref;
    if (fused_at(pref)) return kDecodeFirst + pref;
  } else if (M > kFusedMaxM && M <= kDecodeAutoMax) {
    // narrow N, 8- and 16-token tiles: the most waves that get work quantize
    // x in the launch where light. Above 12 tokens 16 waves do not: at 1024
    // rows and K = 4096 the 8-wave launch on the quantizer's codes is faster
    // (measured W4A4/W8A4/W2A8, M = 14-24: 7.9-8.4 against 8.2-9.0 us;
    // M = 9-12: 16 waves in-launch 6.3-7.9 against 7.2-8.1 us). W8 with
    // 8-token tiles: 8 waves where they quantize x in the launch (a full
    // ring at K = 4096; W8A8/A4/A2, N = 1024-4096, K = 4096: 13-16% faster
    // than 16 waves at M = 5, 3-5% at M = 8, e.g. W8A8 4096x4096 at M = 5
    // 6.7 against 7.6 us; W4 keeps 16 waves, faster at M = 8)
    if (W == 8 && M <= 8 && decode_waves_useful(K, 8) && fused_at(1)) return kDecodeFirst + 1;
    for (int c = 2; c >= 0; --c) {
      if (kSmallMWaves[c] == 16 && M > 12) continue;
      if (decode_waves_useful(K, kSmallMWaves[c]) && fused_at(c)) return kDecodeFirst + c;
    }
  } else if (M == 1) {
    // narrow N, one token: the launch is latency-bound, and the fewest waves
    // whose ring holds the K-range finish first (measured on MI355X at the
    // Gemma-2B and Llama-2-7B shapes, W2/W4/W8: 4096x4096 4.4 us, 2048x2048
    // 3.4 us, 256x2048 3.2 us)
    for (int c = 0; c < 3; ++c)
      if (fused_at(c)) return kDecodeFirst + c;
  } else if (M >= 2 && M <= kFusedMaxM) {
    // narrow N, M <= 4: fewer waves per tile cost less per-workgroup work, so
    // take the smallest wave count that still gives every SIMD a wave (tiles
    // x waves >= 1024, or the most waves that get work) and fits K, with x
    // quantized in the launch where that pays (decode_light). W8 takes at
    // most 8 waves: over W8A8/A4/A2 at N = 1024-4096, K = 1024-4096, M = 2-4
    // 16 waves were never the fastest (W8A4 1024x4096 at M = 2: 8 waves 4.75
    // against 5.69 us for 16). W2 at K >= 4096 takes 16 waves where they
    // quantize x in the launch (one load slot per wave): 4-11% faster at
    // 2048x4096 and 4096x4096, M = 2-4, every A (W2A4 4096x4096 at M = 4:
    // 5.15 against 5.64 us for 8 waves)
    if (W == 2 && K >= 4096 && decode_waves_useful(K, 16) && fused_at(2)) return kDecodeFirst + 2;
    for (int c = 0; c < 3; ++c) {
      const bool last = c == 2 || !decode_waves_useful(K, kSmallMWaves[c + 1]) || (W == 8 && c == 1);
      if (!(tiles * kSmallMWaves[c] >= 1024 || last)) continue;
      if (decode_waves_useful(K, kSmallMWaves[c]) && fused_at(c)) return kDecodeFirst + c;
    }
  }
  return packed_default(M, N, K, W, A);
}

namespace {
// The decode config for a call on packed codes, or -1 where no wave count
// fits (measured on MI355X, W2/W4/W8 x A4/A8, M = 1..64): M <= 4 and narrow
// N, the fewest waves that still give every SIMD a wave; wide N (more than
// 256 row tiles), 4 waves (16 above 8 tokens, whose tiles then share
// workgroups four at a time, but 8 for two 16-token blocks: W4A8 11008x4096
// at M = 24 / 32, 21.3 / 22.5 against 22.7 / 23.6 us) below 1024 row tiles
// and 8 waves from there on;
// narrow N above 4 tokens, the fewest waves that fit, except 16 waves for
// 256 row tiles with K >= 4096 at W8 or above 32 tokens. From 1024 row tiles
// above 16 tokens: 16 waves first for K >= 4096 (W4A8 22016x4096 and 2 x
// 11008x4096, W8A8 2 x 11008x4096, M = 17..64: 7-15% faster than 8 waves,
// e.g. W4A8 2 x 11008x4096 at M = 32 33.2 against 38.4 us), 4 waves first
// below (W4A4 16384x2048 alone, 2 x 8192x2048 and 2 x 16384x2048: 3-9%).
int decode_packed_config(int64_t M, int64_t N, int64_t K, int W) {
  if (M < 1 || M > kDecodeAutoMax) return -1;
  const int64_t tiles = (N + 15) / 16;
  auto packed_at = [&](int c) { return decode_fits((int)K, (int)M, W, kSmallMWaves[c], true, kBF16); };
  int order[3] = {0, 1, 2};
  if (tiles > 256 && M >= 2) {
    if (tiles >= 1024 && M > 16) {
      if (K >= 4096) { order[0] = 2; order[1] = 1; order[2] = 0; }
    } else if (tiles >= 1024) { order[0] = 1; order[1] = M > 8 ? 2 : 0; order[2] = M > 8 ? 0 : 2; }
    else if (M > 16 && M <= 32) { order[0] = 1; order[1] = 2; order[2] = 0; }  // two 16-token blocks
    else if (M > 8) { order[0] = 2; order[1] = 1; order[2] = 0; }
  } else if (M > 8 && tiles >= 256 && K >= 4096 && ((W == 8 && !(M > 12 && M <= 16)) || M > 32)) {
    // (W8 at 13-16 tokens keeps 8 waves first: 4096x4096 W8A8/A4/A2 on
    // codes 4-12% faster than 16, e.g. W8A4 at M = 13 9.5 against 10.6 us)
    order[0] = 2; order[1] = 1; order[2] = 0;
  }
  for (int c : order) {
    const bool last = c == 2 || !decode_waves_useful(K, kSmallMWaves[c + 1]);
    if (M <= kFusedMaxM && tiles <= 256 && !(tiles * kSmallMWaves[c] >= 1024 || last)) continue;
    if (decode_waves_useful(K, kSmallMWaves[c]) && packed_at(c)) return kDecodeFirst + c;
  }
  for (int c : order)  // every useful count failed to fit: any that fits
    if (packed_at(c)) return kDecodeFirst + c;
  return -1;
}

int packed_default(int64_t M, int64_t N, int64_t K, int W, int A) {
  (void)A;
  const int dec = decode_packed_config(M, N, K, W);
  if (dec >= 0) return dec;
  // Measured on MI355X (W4A8, Llama/Gemma shapes), where the decode kernel
  // does not fit: the one-tile-per-CU small-M kernel with 16 waves up to
  // ~512 row tiles; beyond that, and for M > 4, the persistent streaming
  // kernel with 8 waves (it keeps the next tile's weights in flight).
  const int64_t tiles = (N + 15) / 16;
  if (M <= kFusedMaxM) return tiles >= 512 ? kStreamFirst + 1 : 2;
  if (M <= kStreamMax) return tiles >= 512 ? kStreamFirst + 1 : kStreamFirst + 2;
  if (M <= kSmallMMax) return 1;
  // Narrow problems above 64 tokens (at most 128 tiles of 64 rows x 32
  // tokens, K <= 4096): the decode kernel in 16-token blocks, which gives
  // every CU work where the prefill kernel has a few dozen tiles. Measured on
  // MI355X (us, prefill 64x32 -> decode): W4A4 256x2048 at M = 96 / 256 / 512
  // 10.3 / 10.4 / 10.9 -> 6.0 / 6.2 / 8.1, W4A4 2048x2048 at M = 128 10.8 ->
  // 9.3, W4A4 1024x1024 at M = 128 / 256 9.0 / 9.2 -> 6.3 / 8.6, W8A8
  // 512x4096 at M = 128 / 256 16.9 / 17.6 -> 8.5 / 11.9. Four waves take K <=
  // 1024, 16 waves K = 4096 from 256 tokens, 8 waves the rest.
  if (M <= kDecodeMax && K <= 4096 && ((N + 63) / 64) * ((M + 31) / 32) <= 128) {
    const int c = K <= 1024 ? 0 : (K >= 4096 && M >= 256 ? 2 : 1);
    if (decode_fits((int)K, (int)M, W, kSmallMWaves[c], true, kBF16)) return kDecodeFirst + c;
  }
  // Prefill (measured on C3/C4 shapes): the prefill kernel with 64x64 tiles
  // when there are at least two tiles per CU, 64x32 tiles below that (more
  // workgroups for small problems), 128x64 tiles for W <= 4 from four tiles
  // per CU (each unpacked weight slot feeds twice the tokens; 2-7% faster at
  // N=16384 M=256 and N=4096 M=1024; W8's 128x64 tiles hold too many
  // registers for two waves per SIMD), and the LDS-staged tiled kernel for
  // the largest problems, whose 4-wave 64x64 tiles share weight fragments in
  // LDS.
  const int64_t t64 = ((N + 63) / 64) * ((M + 63) / 64);
  if (t64 < 512) return kPrefillFirst + 3;
  if (t64 < 1024) return kPrefillFirst + 2;
  if (t64 < 2048) return W <= 4 ? kPrefillFirst + 0 : kPrefillFirst + 2;
  return kSmallMConfigs;
}
}  // namespace

int actune_forward_fuses_quantizer(int64_t M, int64_t N, int64_t K, int W, int A, int x_dtype, int config) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A, true);
  if (check_shape(M, K, W, A, x_dtype, kF32, config) || N <= 0) return -1;
  return forward_fuses(config, M, N, K, W, x_dtype) ? 1 : 0;
}

int actune_quantize_groups(const void* x, int x_dtype, const void* input_scale, int64_t M, int64_t K,
                           int A, uint8_t* packed, float* scales, void* stream) {
  g_err[0] = 0;
  int rc = check_quantize(x, x_dtype, input_scale, M, K, A, packed, scales);
  if (rc || M == 0) return rc;
  launch_quantize(x, x_dtype, input_scale, M, K, A, packed, scales, (hipStream_t)stream);
  return check_launch();
}

int actune_quantize_gated(const void* gate, const void* up, int x_dtype, int act, const void* input_scale,
                          int64_t M, int64_t K, int A, uint8_t* packed, float* scales, void* stream) {
  g_err[0] = 0;
  if (act != ACTUNE_ACT_SILU && act != ACTUNE_ACT_GELU_TANH) return fail(ACTUNE_ERR_INVALID, "unknown gate activation");
  int rc = check_quantize(gate, x_dtype, input_scale, M, K, A, packed, scales);
  if (!rc && M > 0 && (!up || !aligned(up, 16))) rc = fail(ACTUNE_ERR_INVALID, "null or misaligned up operand");
  if (rc || M == 0) return rc;
  launch_quantize_gated(gate, up, x_dtype, act, input_scale, M, K, A, packed, scales, (hipStream_t)stream);
  return check_launch();
}

int actune_grouped_linear(const uint8_t* a, const float* a_scales, const uint8_t* w,
                          const float* w_scale, const void* bias, int bias_dtype, void* out,
                          int out_dtype, int64_t M, int64_t N, int64_t K, int W, int A, int config,
                          void* stream) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A, false);
  int rc = check_shape(M, K, W, A, out_dtype, bias_dtype, config);
  if (!rc) rc = check_target(w, w_scale, out, N, M, K, W);
  if (rc || M == 0) return rc;
  if (!a || !a_scales) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(a, 16) || !aligned(a_scales, 4)) return fail(ACTUNE_ERR_INVALID, "misaligned operand (packed data needs 16 B)");
  LinearArgs g = base_args(M, K, bias_dtype, out_dtype);
  g.a = a;
  g.as = a_scales;
  add_problem(g, w, w_scale, bias, out, N, W);
  run_gemm(W, A, config, kModePacked, g, (hipStream_t)stream);
  return check_launch();
}

namespace {
// Targets of different weight widths (one A). The decode kernel runs them in
// one launch where its config takes every width: x quantized in the launch
// where the widest width's launch would quantize it, else on the quantizer's
// codes. Otherwise x is quantized once and each width runs its own launch on
// the codes (its own default config under ACTUNE_CONFIG_AUTO). Either way
// every output equals the single-width call.
int forward_mixed(LinearArgs& g, int config, bool auto_config, int64_t n_total, const void* x, int x_dtype,
                  const void* input_scale, uint8_t* a_buf, float* scale_buf, int A, hipStream_t st) {
  int wmax = 2;
  for (int q = 0; q < g.nprob; ++q) wmax = std::max(wmax, g.prob[q].W);
  if (config >= kDecodeFirst) {
    const int nw = kSmallMWaves[config - kDecodeFirst];
    const bool fused =
        decode_fits(g.K, g.M, wmax, nw, false, x_dtype) && decode_light(g.M, n_total, g.K, wmax, nw, false);
    bool fits = true;
    for (int q = 0; q < g.nprob; ++q) fits = fits && decode_fits(g.K, g.M, g.prob[q].W, nw, !fused, x_dtype);
    if (fits) {
      if (fused) {
        g.x = x;
        g.xscale = input_scale;
        g.x_dt = x_dtype;
      } else {
        launch_quantize(x, x_dtype, input_scale, g.M, g.K, A, a_buf, scale_buf, st);
        g.a = a_buf;
        g.as = scale_buf;
      }
      launch_decode_mixed(A, nw, !fused, g, st);
      return check_launch();
    }
  }
  launch_quantize(x, x_dtype, input_scale, g.M, g.K, A, a_buf, scale_buf, st);
  bool done[kMaxProblems] = {};
  for (int q = 0; q < g.nprob; ++q) {
    if (done[q]) continue;
    const int w = g.prob[q].W;
    LinearArgs one = base_args(g.M, g.K, g.bias_dt, g.out_dt);
    one.a = a_buf;
    one.as = scale_buf;
    int64_t n_w = 0;
    for (int r = q; r < g.nprob; ++r)
      if (!done[r] && g.prob[r].W == w) {
        add_problem(one, g.prob[r].w, g.prob[r].ws, g.prob[r].bias, g.prob[r].out, g.prob[r].N, w);
        n_w += g.prob[r].N;
        done[r] = true;
      }
    run_gemm(w, A, auto_config ? packed_default(g.M, n_w, g.K, w, A) : config, kModePacked, one, st);
  }
  return check_launch();
}
}  // namespace

int actune_grouped_forward_multi(const void* x, int x_dtype, const void* input_scale, uint8_t* a_buf,
                                 float* scale_buf, const actune_linear_target* targets, int ntargets,
                                 int bias_dtype, int64_t M, int64_t K, int W, int A, int config,
                                 void* stream) {
  g_err[0] = 0;
  if (ntargets < 1 || ntargets > ACTUNE_MAX_TARGETS || !targets)
    return fail(ACTUNE_ERR_INVALID, "between 1 and 4 targets required");
  // each target's width: its own W field, or the call's W where that is 0
  int widths[ACTUNE_MAX_TARGETS];
  bool mixed = false;
  for (int t = 0; t < ntargets; ++t) {
    widths[t] = targets[t].W ? targets[t].W : W;
    if (!width_ok(widths[t])) return fail(ACTUNE_ERR_INVALID, "Unsupported integer width");
    mixed = mixed || widths[t] != widths[0];
  }
  // the widest width sizes the launch (its weight ring is the tightest)
  W = *std::max_element(widths, widths + ntargets);
  int64_t n_total = 0;
  for (int t = 0; t < ntargets; ++t) {
    if (targets[t].N <= 0 || targets[t].N > INT_MAX / 2) return fail(ACTUNE_ERR_INVALID, "invalid dimensions");
    n_total += targets[t].N;
  }
  const bool auto_config = config == ACTUNE_CONFIG_AUTO;
  config = resolve(config, M, n_total, K, W, A, true);
  int rc = check_shape(M, K, W, A, x_dtype, bias_dtype, config);
  if (!rc) rc = check_quantize(x, x_dtype, input_scale, M, K, A, a_buf, scale_buf);
  for (int t = 0; t < ntargets && !rc; ++t)
    rc = check_target(targets[t].w, targets[t].w_scale, targets[t].out, targets[t].N, M, K, widths[t]);
  if (!rc && n_total / 16 >= INT_MAX / 2) rc = fail(ACTUNE_ERR_INVALID, "dimensions too large");
  if (rc || M == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  LinearArgs g = base_args(M, K, bias_dtype, x_dtype);
  for (int t = 0; t < ntargets; ++t)
    add_problem(g, targets[t].w, targets[t].w_scale, targets[t].bias, targets[t].out, targets[t].N, widths[t]);
  if (mixed)
    return forward_mixed(g, config, auto_config, n_total, x, x_dtype, input_scale, a_buf, scale_buf, A, st);
  const bool fused = forward_fuses(config, M, n_total, K, W, x_dtype);
  if (fused) {
    g.x = x;
    g.xscale = input_scale;
    g.x_dt = x_dtype;
    run_gemm(W, A, config, kModeFused, g, st);
  } else {
    launch_quantize(x, x_dtype, input_scale, M, K, A, a_buf, scale_buf, st);
    g.a = a_buf;
    g.as = scale_buf;
    run_gemm(W, A, config, kModePacked, g, st);
  }
  return check_launch();
}

int actune_grouped_forward(const void* x, int x_dtype, const void* input_scale, uint8_t* a_buf,
                           float* scale_buf, const uint8_t* w, const float* w_scale, const void* bias,
                           int bias_dtype, void* out, int64_t M, int64_t N, int64_t K, int W, int A,
                           int config, void* stream) {
  const actune_linear_target t{w, w_scale, bias, out, N};
  return actune_grouped_forward_multi(x, x_dtype, input_scale, a_buf, scale_buf, &t, 1, bias_dtype, M, K,
                                      W, A, config, stream);
}

int actune_grouped_dots_i32(const uint8_t* a, const uint8_t* w, int64_t M, int64_t N, int64_t K,
                            int W, int A, int config, int32_t* dots, void* stream) {
  g_err[0] = 0;
  config = resolve(config, M, N, K, W, A, false);
  int rc = check_shape(M, K, W, A, kF32, kF32, config);
  if (!rc && (N <= 0 || N > INT_MAX / 2)) rc = fail(ACTUNE_ERR_INVALID, "invalid dimensions");
  if (!rc && N * K * W / 8 >= kMaxBufferBytes) rc = fail(ACTUNE_ERR_INVALID, "operand too large (each buffer must stay below 2 GiB)");
  if (rc || M == 0) return rc;
  if (!a || !w || !dots) return fail(ACTUNE_ERR_INVALID, "null pointer");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(dots, 4)) return fail(ACTUNE_ERR_INVALID, "misaligned operand");
  LinearArgs g = base_args(M, K, kF32, kF32);
  g.a = a;
  g.dots = dots;
  add_problem(g, w, nullptr, nullptr, nullptr, N, W);
  run_gemm(W, A, config, kModeDots, g, (hipStream_t)stream);
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
