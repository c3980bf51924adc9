// Register-resident compute ceilings of the prefill inner loop (a diagnostic
// library, libactune_ceiling.so, timed by bench.py; not part of the
// library's C ABI).
//
// Each kernel repeats, on operands held in registers, the per-group
// instruction mix of one prefill design: no global or LDS traffic, no
// barriers. Its throughput is therefore the most that design can reach on
// MI355X, whatever the memory side does. Every wave runs the same number of
// iterations and writes one value at the end.
//
//  kind 0: the library's prefill kernel (gemm_prefill): per 64-K group, one
//          16-row weight tile unpacked from W4 (shifted int8 codes), four
//          v_mfma_i32_16x16x64_i8 against four 16-token tiles, then the
//          per-group rescale of the previous group: v_cvt_f32_i32 + fma per
//          output; chunk partials added every 4 groups.
//  kind 1: an exact fp8 alternative for W <= 4, A <= 4: per group, W4 codes
//          moved to offset-binary e4m3 bytes (c + 8, exact; 3 VALU per packed
//          dword), a v_mfma_scale_f32_32x32x64_f8f6f4 of the constant -8
//          against the activations (the offset correction -8 sum a) feeding
//          the C operand of the main MFMA, then one fma per output (the MFMA
//          result is already fp32).
//  kind 2: as kind 1 for A8: the activation codes split into two planes
//          (a = 16 hi + lo, both exact in e4m3): two correction and two
//          main MFMAs, chained.
//  kind 3: kind 1 without the correction MFMA (its C operand taken from
//          registers): the bound of an fp8 design whose correction costs
//          nothing.
//  kind 4: kind 0 on v_mfma_i32_32x32x32_i8 (the 16x16x64 form issues at
//          half the int8 rate on gfx950): per 64-K group one 32-row weight
//          tile unpacked from W4, two chained 32x32x32 MFMAs against each of
//          two 32-token tiles, then the rescale of the previous group
//          (16 outputs per lane and tile).
//  kind 5: MFMAs alone, 16x16x64 (the instruction's own issue rate).
//  kind 6: MFMAs alone, 32x32x32.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

// keeps a value opaque to the compiler, so that loop-invariant operands are
// not hoisted out of the loop
#define ACT_OPAQUE(x) asm volatile("" : "+v"(x))

constexpr int kWords = 48;  // input dwords per thread

__global__ __launch_bounds__(256) void ceiling_int8(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  uint32_t wp0 = s[0], wp1 = s[1];
  v4i b[4];
  float sc[4];
  for (int y = 0; y < 4; ++y) {
    b[y] = v4i{(int)s[2 + 4 * y], (int)s[3 + 4 * y], (int)s[4 + 4 * y], (int)s[5 + 4 * y]};
    sc[y] = __uint_as_float(s[20 + y] & 0x3fffffffu);
  }
  v4i D[2][4];
  float p[4][4], acc[4][4];
  for (int y = 0; y < 4; ++y)
    for (int r = 0; r < 4; ++r) { p[y][r] = acc[y][r] = 0.f; D[0][y][r] = D[1][y][r] = 0; }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ACT_OPAQUE(wp0);
      ACT_OPAQUE(wp1);
      const v4i wd = v4i{(int)((wp0 << 4) & 0xF0F0F0F0u), (int)(wp0 & 0xF0F0F0F0u),
                         (int)((wp1 << 4) & 0xF0F0F0F0u), (int)(wp1 & 0xF0F0F0F0u)};
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        ACT_OPAQUE(b[y]);
        D[g & 1][y] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wd, b[y], v4i{0, 0, 0, 0}, 0, 0, 0);
      }
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[y][r] = __builtin_fmaf((float)D[(g + 1) & 1][y][r], sc[y], p[y][r]);
    }
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) { acc[y][r] += p[y][r]; p[y][r] = 0.f; }
  }
  float t = 0.f;
  for (int y = 0; y < 4; ++y)
    for (int r = 0; r < 4; ++r) t += acc[y][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

template <bool HILO, bool CORR>
__global__ __launch_bounds__(256) void ceiling_fp8(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  uint32_t wp[4];
  for (int j = 0; j < 4; ++j) wp[j] = s[j] & 0x77777777u;
  v8i alo, ahi;
  for (int j = 0; j < 8; ++j) { alo[j] = (int)(s[8 + j] & 0x07070707u); ahi[j] = (int)(s[16 + j] & 0x07070707u); }
  float sc[16];
  v16f corr;
  for (int r = 0; r < 16; ++r) { sc[r] = __uint_as_float(s[24 + r] & 0x3fffffffu); corr[r] = (float)(int)(s[24 + r] & 0xffu); }
  v16f D[2];
  float p[16], acc[16];
  for (int r = 0; r < 16; ++r) { p[r] = acc[r] = 0.f; D[0][r] = D[1][r] = 0.f; }
  v8i neg8;  // -8 (byte 0x88) everywhere
  for (int j = 0; j < 8; ++j) neg8[j] = (int)0x88888888u;
  const v16f zero16 = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ACT_OPAQUE(alo);
      ACT_OPAQUE(ahi);
      ACT_OPAQUE(corr);
      v8i w;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ACT_OPAQUE(wp[j]);
        w[2 * j] = (int)((wp[j] ^ 0x88888888u) & 0x0F0F0F0Fu);
        w[2 * j + 1] = (int)(((wp[j] >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu);
      }
      // scale operands: E8M0 exponents (127 = 2^0, 131 = 2^4 for the hi plane)
      v16f c = corr;
      if constexpr (CORR) {
        c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(alo, neg8, zero16, 0, 0, 0, 127, 0, 127);
        if constexpr (HILO) c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ahi, neg8, c, 0, 0, 0, 131, 0, 127);
      }
      v16f d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(alo, w, c, 0, 0, 0, 127, 0, 127);
      if constexpr (HILO) d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ahi, w, d, 0, 0, 0, 131, 0, 127);
      D[g & 1] = d;
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = __builtin_fmaf(D[(g + 1) & 1][r], sc[r], p[r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[r] += p[r]; p[r] = 0.f; }
  }
  float t = 0.f;
  for (int r = 0; r < 16; ++r) t += acc[r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

__global__ __launch_bounds__(256) void ceiling_int8_32(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  uint32_t wp[4];
  for (int j = 0; j < 4; ++j) wp[j] = s[j];
  v4i b[2][2];
  float sc[2];
  for (int y = 0; y < 2; ++y) {
    for (int h = 0; h < 2; ++h) b[y][h] = v4i{(int)s[4 + 8 * y + 4 * h], (int)s[5 + 8 * y + 4 * h], (int)s[6 + 8 * y + 4 * h], (int)s[7 + 8 * y + 4 * h]};
    sc[y] = __uint_as_float(s[20 + y] & 0x3fffffffu);
  }
  v16i D[2][2];
  float p[2][16], acc[2][16];
  for (int y = 0; y < 2; ++y)
    for (int r = 0; r < 16; ++r) { p[y][r] = acc[y][r] = 0.f; D[0][y][r] = D[1][y][r] = 0; }
  const v16i zero = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ACT_OPAQUE(wp[j]);
      const v4i w0 = v4i{(int)((wp[0] << 4) & 0xF0F0F0F0u), (int)(wp[0] & 0xF0F0F0F0u),
                         (int)((wp[1] << 4) & 0xF0F0F0F0u), (int)(wp[1] & 0xF0F0F0F0u)};
      const v4i w1 = v4i{(int)((wp[2] << 4) & 0xF0F0F0F0u), (int)(wp[2] & 0xF0F0F0F0u),
                         (int)((wp[3] << 4) & 0xF0F0F0F0u), (int)(wp[3] & 0xF0F0F0F0u)};
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        ACT_OPAQUE(b[y][0]);
        ACT_OPAQUE(b[y][1]);
        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(w0, b[y][0], zero, 0, 0, 0);
        D[g & 1][y] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w1, b[y][1], d, 0, 0, 0);
      }
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int r = 0; r < 16; ++r) p[y][r] = __builtin_fmaf((float)D[(g + 1) & 1][y][r], sc[y], p[y][r]);
    }
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) { acc[y][r] += p[y][r]; p[y][r] = 0.f; }
  }
  float t = 0.f;
  for (int y = 0; y < 2; ++y)
    for (int r = 0; r < 16; ++r) t += acc[y][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

// MFMAs alone: 4 groups x 4 (16x16x64) or 4 groups x 2 (32x32x32) per
// iteration, independent accumulators, the same int8 MACs either way
template <bool M32>
__global__ __launch_bounds__(256) void ceiling_mfma(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  v4i a = v4i{(int)s[0], (int)s[1], (int)s[2], (int)s[3]}, b = v4i{(int)s[4], (int)s[5], (int)s[6], (int)s[7]};
  int t = 0;
  if constexpr (M32) {
    // four accumulators of 16 registers (eight would hold 128 VGPRs and cap
    // the occupancy), two MFMAs each per iteration
    v16i c[4];
    for (int j = 0; j < 4; ++j)
      for (int r = 0; r < 16; ++r) c[j][r] = 0;
    for (int it = 0; it < iters; ++it) {
      ACT_OPAQUE(a);
      ACT_OPAQUE(b);
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j & 3], 0, 0, 0);
    }
    for (int j = 0; j < 4; ++j)
      for (int r = 0; r < 16; ++r) t += c[j][r];
  } else {
    v4i c[16];
    for (int j = 0; j < 16; ++j) c[j] = v4i{0, 0, 0, 0};
    for (int it = 0; it < iters; ++it) {
      ACT_OPAQUE(a);
      ACT_OPAQUE(b);
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
    }
    for (int j = 0; j < 16; ++j) t += c[j][0] + c[j][1] + c[j][2] + c[j][3];
  }
  out[blockIdx.x * 256 + threadIdx.x] = (float)t;
}

}  // namespace

extern "C" {

// Input dwords per thread the kernels read (the caller passes blocks * 256 *
// this many) and int8-equivalent multiply-accumulates per wave iteration of
// a kind: 4 groups of 64 K against a 16 x 64 tile (kind 0) or a 32 x 32 tile
// (kinds 1-3), 4 * 65536, and the MFMA-only kinds 5 and 6 the same; kind 4
// against a 32 x 64 tile, 8 * 65536. -1 for an unknown kind.
int actune_ceiling_words(void) { return kWords; }
long actune_ceiling_macs_per_iter(int kind) {
  if (kind < 0 || kind > 6) return -1;
  return kind == 4 ? 8L * 65536L : 4L * 65536L;
}

// Runs kind 0 .. 6 on `blocks` workgroups of 4 waves; 0 on success.
int actune_ceiling_run(int kind, const uint32_t* in, float* out, int blocks, int iters, void* stream) {
  if (!in || !out || blocks <= 0 || iters <= 0) return -1;
  const hipStream_t st = (hipStream_t)stream;
  if (kind == 0) ceiling_int8<<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 1) ceiling_fp8<false, true><<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 2) ceiling_fp8<true, true><<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 3) ceiling_fp8<false, false><<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 4) ceiling_int8_32<<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 5) ceiling_mfma<false><<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 6) ceiling_mfma<true><<<blocks, 256, 0, st>>>(in, out, iters);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
