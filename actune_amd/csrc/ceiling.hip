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
//  kind 4: kind 0 on v_mfma_i32_32x32x32_i8 (a 32x32 tile holds four
//          times the outputs per operand load): per 64-K group one 32-row weight
//          tile unpacked from W4, two chained 32x32x32 MFMAs against each of
//          two 32-token tiles, then the rescale of the previous group
//          (16 outputs per lane and tile).
//  kind 5: MFMAs alone, 16x16x64 (the instruction's own issue rate).
//  kind 6: MFMAs alone, 32x32x32.
//  kind 7: bf6 (e3m2) for W4A4: per group the W4 operand (32 two's-complement
//          codes per lane) converted in registers to sign-magnitude e3m2
//          fields (|c| <= 8 is the 4-bit exponent-mantissa field itself) and
//          packed densely into six dwords, then v_mfma_scale_f32_32x32x64_f8f6f4
//          on bf6 x bf6 against two 32-token tiles of pre-packed bf6
//          activations, and one fma per output for the rescale.
//  kind 8: bf6 x bf6 32x32x64 MFMAs alone (the format's own rate).
//
// It also holds the load floor of the decode launches
// (actune_ceiling_decode_floor): the memory side of gemm_decode with nothing
// else, timed by bench.py over the M=1 step's schedule.
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

// Six dwords of densely packed 6-bit fields from 32 two's-complement W4
// codes (four dwords of nibbles): field = sign << 5 | |c|, which is the e3m2
// encoding of c in units of 1/16 (the block scale restores the unit).
__device__ __forceinline__ void w4_to_bf6(const uint32_t wp[4], v8i& out) {
  uint32_t c24[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = (j & 1 ? wp[j >> 1] >> 4 : wp[j >> 1]) & 0x0F0F0F0Fu;  // four codes, one per byte
    const uint32_t sg = (b >> 3) & 0x01010101u;
    const uint32_t f = ((b ^ (sg * 0x0Fu)) + sg) | (sg << 5);                // sign-magnitude per byte
    c24[j] = (f & 0x3Fu) | ((f >> 2) & 0xFC0u) | ((f >> 4) & 0x3F000u) | ((f >> 6) & 0xFC0000u);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t* c = c24 + 4 * h;
    out[3 * h + 0] = (int)(c[0] | (c[1] << 24));
    out[3 * h + 1] = (int)((c[1] >> 8) | (c[2] << 16));
    out[3 * h + 2] = (int)((c[2] >> 16) | (c[3] << 8));
  }
  out[6] = out[7] = 0;
}

__global__ __launch_bounds__(256) void ceiling_bf6(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  uint32_t wp[4];
  for (int j = 0; j < 4; ++j) wp[j] = s[j];
  v8i a[2];
  for (int t = 0; t < 2; ++t)
    for (int j = 0; j < 8; ++j) a[t][j] = j < 6 ? (int)(s[4 + 6 * t + j] & 0x37DF7DF7u) : 0;
  float sc[2][16];
  for (int t = 0; t < 2; ++t)
    for (int r = 0; r < 16; ++r) sc[t][r] = __uint_as_float(s[16 + 16 * t + r] & 0x3fffffffu);
  v16f D[2][2];
  float p[2][16], acc[2][16];
  for (int t = 0; t < 2; ++t)
    for (int r = 0; r < 16; ++r) { p[t][r] = acc[t][r] = 0.f; D[0][t][r] = D[1][t][r] = 0.f; }
  const v16f zero16 = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ACT_OPAQUE(wp[0]);
      ACT_OPAQUE(wp[1]);
      ACT_OPAQUE(wp[2]);
      ACT_OPAQUE(wp[3]);
      v8i w;
      w4_to_bf6(wp, w);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        ACT_OPAQUE(a[t]);
        // format 3 = bf6 (e3m2) for both operands; E8M0 scales 2^4 each undo
        // the two 1/16 units
        D[g & 1][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a[t], zero16, 3, 3, 0, 131, 0, 131);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) p[t][r] = __builtin_fmaf(D[(g + 1) & 1][t][r], sc[t][r], p[t][r]);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) { acc[t][r] += p[t][r]; p[t][r] = 0.f; }
  }
  float t = 0.f;
  for (int u = 0; u < 2; ++u)
    for (int r = 0; r < 16; ++r) t += acc[u][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

__global__ __launch_bounds__(256) void ceiling_bf6_mfma(const uint32_t* in, float* out, int iters) {
  const uint32_t* s = in + (size_t)(blockIdx.x * 256 + threadIdx.x) * kWords;
  v8i a, b;
  for (int j = 0; j < 8; ++j) {
    a[j] = j < 6 ? (int)(s[j] & 0x37DF7DF7u) : 0;
    b[j] = j < 6 ? (int)(s[8 + j] & 0x37DF7DF7u) : 0;
  }
  v16f c[4];
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 16; ++r) c[j][r] = 0.f;
  for (int it = 0; it < iters; ++it) {
    ACT_OPAQUE(a);
    ACT_OPAQUE(b);
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c[j & 3], 3, 3, 0, 127, 0, 127);
  }
  float t = 0.f;
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 16; ++r) t += c[j][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

// ---------------------------------------------------------------- decode load floor
// gemm_decode's weight traffic alone: a workgroup per 16-row tile of up to
// four problems (grid y), nw waves splitting each row's bytes into ranges of
// `slots` 64-byte slots; lane l loads 16 bytes of row n0 + l % 16 at byte
// 16 (l / 16) of every slot of its wave's range, all loads issued at entry
// (slots past the range or the row are switched off and read nothing). The
// only arithmetic is an XOR of the loaded words, stored once per thread so
// the loads stay. MODE 1: the same bytes per wave read as whole runs of 1
// KiB of one row per instruction (lane l: bytes 16 l of the run): the
// wave's rows are 16 / nw consecutive ones of the tile. MODE 2: the wave's
// K-range as in MODE 0, read 8 rows x 128 bytes per instruction (lane l: row
// l % 8 of the instruction's half of the tile, bytes 16 (l / 8)).
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr uint32_t kOff = 0x80000000u;
constexpr int kFloorMaxSlots = 8;

struct FloorArgs {
  const uint8_t* w[4];
  int n[4];
  int row_bytes, slots;
  uint32_t* sink;
};

__device__ __forceinline__ Rsrc floor_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int MODE>
__global__ __launch_bounds__(1024) void decode_load_floor(const FloorArgs a) {
  const int p = (int)blockIdx.y, N = a.n[p], n0 = (int)blockIdx.x * 16;
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6, nw = (int)blockDim.x >> 6;
  uint32_t x = 0;
  if (n0 < N) {
    const uint32_t rb = (uint32_t)a.row_bytes;
    const Rsrc r = floor_rsrc(a.w[p], (uint32_t)N * rb);
    v4u q[kFloorMaxSlots];
    if constexpr (MODE == 2) {
      const uint32_t start = (uint32_t)wave * (uint32_t)a.slots * 64u;
#pragma unroll
      for (int s = 0; s < kFloorMaxSlots; ++s) {
        const uint32_t at = start + (uint32_t)(s >> 1) * 128u + (uint32_t)(lane >> 3) * 16u;
        const int row = n0 + (lane & 7) + 8 * (s & 1);
        const bool live = s < a.slots && start + (uint32_t)(s >> 1) * 128u < rb && at < rb;
        q[s] = __builtin_amdgcn_raw_buffer_load_b128(r, live ? (uint32_t)row * rb + at : kOff, 0, 0);
      }
    } else if constexpr (MODE == 0) {
      const uint32_t start = (uint32_t)wave * (uint32_t)a.slots * 64u;
      const uint32_t base = (uint32_t)(n0 + (lane & 15)) * rb + (uint32_t)(lane >> 4) * 16u + start;
#pragma unroll
      for (int s = 0; s < kFloorMaxSlots; ++s) {
        const bool live = s < a.slots && start + (uint32_t)s * 64u < rb;
        q[s] = __builtin_amdgcn_raw_buffer_load_b128(r, base + (uint32_t)s * 64u, live ? 0u : kOff, 0);
      }
    } else {
      const int rpw = 16 / nw, runs = (int)((rb + 1023u) / 1024u);
#pragma unroll
      for (int s = 0; s < kFloorMaxSlots; ++s) {
        const int row = n0 + wave * rpw + s / runs;
        const uint32_t at = (uint32_t)(s % runs) * 1024u + (uint32_t)lane * 16u;
        const bool live = s < rpw * runs && at < rb;
        q[s] = __builtin_amdgcn_raw_buffer_load_b128(r, live ? (uint32_t)row * rb + at : kOff, 0, 0);
      }
    }
#pragma unroll
    for (int s = 0; s < kFloorMaxSlots; ++s) x ^= q[s][0] ^ q[s][1] ^ q[s][2] ^ q[s][3];
  }
  a.sink[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x] = x;
}

}  // namespace

extern "C" {

// Load floor of one decode launch: nprob (1-4) problems of n[p] rows of
// row_bytes packed bytes at w[p], nw (4, 8, 16) waves per 16-row tile, the
// decode kernel's 16-row x 64-byte loads (contig = 0), whole 1 KiB row runs
// per instruction (contig = 1) or 8-row x 128-byte loads (contig = 2). sink: at least ceil(max n / 16) * nprob * nw
// * 64 dwords. 0 on success, -1 for arguments outside that (or a row split
// needing more than 8 loads per wave), -2 on a launch error.
int actune_ceiling_decode_floor(const void* const* w, const int64_t* n, int nprob, int64_t row_bytes, int nw,
                                int contig, uint32_t* sink, int64_t sink_words, void* stream) {
  if (!w || !n || !sink || nprob < 1 || nprob > 4 || (nw != 4 && nw != 8 && nw != 16) || row_bytes <= 0)
    return -1;
  FloorArgs a{};
  int64_t nmax = 0;
  for (int p = 0; p < nprob; ++p) {
    if (!w[p] || n[p] <= 0 || n[p] * row_bytes >= ((int64_t)1 << 31)) return -1;
    a.w[p] = static_cast<const uint8_t*>(w[p]);
    a.n[p] = (int)n[p];
    nmax = n[p] > nmax ? n[p] : nmax;
  }
  a.row_bytes = (int)row_bytes;
  a.slots = (int)((row_bytes + 64 * nw - 1) / (64 * nw));
  a.sink = sink;
  const int64_t runs = (row_bytes + 1023) / 1024;
  if (a.slots > kFloorMaxSlots || (contig == 1 && (16 / nw) * runs > kFloorMaxSlots)) return -1;
  const int64_t tiles = (nmax + 15) / 16;
  if (sink_words < tiles * nprob * nw * 64) return -1;
  const dim3 grid((unsigned)tiles, (unsigned)nprob);
  const hipStream_t st = (hipStream_t)stream;
  if (contig == 1) decode_load_floor<1><<<grid, nw * 64, 0, st>>>(a);
  else if (contig == 2) decode_load_floor<2><<<grid, nw * 64, 0, st>>>(a);
  else if (contig == 0) decode_load_floor<0><<<grid, nw * 64, 0, st>>>(a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Input dwords per thread the kernels read (the caller passes blocks * 256 *
// this many) and int8-equivalent multiply-accumulates per wave iteration of
// a kind: 4 groups of 64 K against a 16 x 64 tile (kind 0) or a 32 x 32 tile
// (kinds 1-3), 4 * 65536, and the MFMA-only kinds 5 and 6 the same; kind 4
// against a 32 x 64 tile, 8 * 65536; kind 7 two 32-token tiles and kind 8
// eight 32x32x64 MFMAs, 8 * 65536 each. -1 for an unknown kind.
int actune_ceiling_words(void) { return kWords; }
long actune_ceiling_macs_per_iter(int kind) {
  if (kind < 0 || kind > 8) return -1;
  return kind == 4 || kind == 7 || kind == 8 ? 8L * 65536L : 4L * 65536L;
}

// Runs kind 0 .. 8 on `blocks` workgroups of 4 waves; 0 on success.
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
  else if (kind == 7) ceiling_bf6<<<blocks, 256, 0, st>>>(in, out, iters);
  else if (kind == 8) ceiling_bf6_mfma<<<blocks, 256, 0, st>>>(in, out, iters);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
