// Shared device helpers for the gfx950 group-64 linear kernels.
//
// Operand representation used by every kernel: a code c of width B bits is
// held as the int8 value c * 2^(8-B) (the field shifted to the top of its
// byte). An int8 MFMA over such values yields 2^(sW+sA) * d for the true
// group dot d, |2^(sW+sA) d| <= 2^20 for every (W,A) pair, so the int32
// result and its fp32 conversion are exact, and the factor folds exactly into
// the fp32 activation scale (scale * 2^-(sW+sA) is a power-of-two rescale of
// a normal float). fmaf(2^T d, s 2^-T, acc) == fmaf(d, s, acc) bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace actune {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

enum Dtype { kBF16 = 0, kF16 = 1, kF32 = 2 };

constexpr int kGroup = 64;
// Canonical fp32 reduction order: K is cut into kChunks contiguous chunks of
// whole quads (4 groups); chunk c = quads [c*Q/kChunks, (c+1)*Q/kChunks),
// Q = ceil(G/4), clipped to G. Each chunk accumulates its groups in order
// from +0 with fmaf; chunk partials are added in chunk order.
constexpr int kChunks = 16;

__host__ __device__ constexpr int shift_of(int bits) { return 8 - bits; }

__host__ __device__ inline int chunk_begin(int c, int G) {
  const int Q = (G + 3) / 4;
  const int b = (c * Q / kChunks) * 4;
  return b < G ? b : G;
}

// Chunks that hold groups: all kChunks from Q = kChunks quads on; below,
// each nonempty chunk holds exactly one quad (its bounds differ by at most
// Q / kChunks < 1 quads), so there are Q of them, in quad order. An empty
// chunk's partial is +0, and a running sum of partials is never -0 (each
// partial starts from +0 and an exact cancellation rounds to +0), so adding
// it changes no bit: a reduction may keep one slot per nonempty chunk (its
// quad) and skip the rest.
__host__ __device__ inline int chunk_slots(int G) {
  const int Q = (G + 3) / 4;
  return Q < kChunks ? Q : kChunks;
}

// v_perm_b32: byte i of the result is byte sel.i of the 8-byte pool
// {lo (bytes 0-3), hi (bytes 4-7)}. The host form emulates it so the layout
// self-test can run without a GPU.
__host__ __device__ inline uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_perm(hi, lo, sel);
#else
  uint64_t pool = ((uint64_t)hi << 32) | lo;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) {
    uint32_t s = (sel >> (8 * i)) & 0xffu;
    uint32_t byte = s < 8 ? (uint32_t)(pool >> (8 * s)) & 0xffu : (s == 12 ? 0u : 0xffu);
    r |= byte << (8 * i);
  }
  return r;
#endif
}

// ---------------------------------------------------------------------------
// Unpack one 16-element slot into 4 dwords of shifted int8, in the width's
// native order. Element index held by byte t of output dword r:
//   8 bits: 4r + t          4 bits: 8(r/2) + 2t + (r%2)        2 bits: 4t + r
// Input: 16*B/8 bytes = B/2 dwords (8 -> 4, 4 -> 2, 2 -> 1).
template <int B>
__host__ __device__ inline void unpack_slot(const uint32_t* p, uint32_t d[4]);

template <>
__host__ __device__ inline void unpack_slot<8>(const uint32_t* p, uint32_t d[4]) {
  d[0] = p[0]; d[1] = p[1]; d[2] = p[2]; d[3] = p[3];
}
template <>
__host__ __device__ inline void unpack_slot<4>(const uint32_t* p, uint32_t d[4]) {
  d[0] = (p[0] << 4) & 0xF0F0F0F0u; d[1] = p[0] & 0xF0F0F0F0u;
  d[2] = (p[1] << 4) & 0xF0F0F0F0u; d[3] = p[1] & 0xF0F0F0F0u;
}
template <>
__host__ __device__ inline void unpack_slot<2>(const uint32_t* p, uint32_t d[4]) {
  d[0] = (p[0] << 6) & 0xC0C0C0C0u; d[1] = (p[0] << 4) & 0xC0C0C0C0u;
  d[2] = (p[0] << 2) & 0xC0C0C0C0u; d[3] = p[0] & 0xC0C0C0C0u;
}

// Element order of a width, for the host self-test: element held by (r, t).
__host__ __device__ inline int slot_elem(int B, int r, int t) {
  if (B == 8) return 4 * r + t;
  if (B == 4) return 8 * (r / 2) + 2 * t + (r % 2);
  return 4 * t + r;
}

// Reorder a slot from the native order of width FROM to that of width TO,
// so that byte (r,t) of both operands refers to the same k.
template <int FROM, int TO>
__host__ __device__ inline void reorder_slot(uint32_t d[4]) {
  if constexpr (FROM == TO) {
    return;
  } else if constexpr (FROM == 8 && TO == 4) {
    // natural -> [0,2,4,6][1,3,5,7][8,10,12,14][9,11,13,15]
    uint32_t o0 = perm_b32(d[1], d[0], 0x06040200u), o1 = perm_b32(d[1], d[0], 0x07050301u);
    uint32_t o2 = perm_b32(d[3], d[2], 0x06040200u), o3 = perm_b32(d[3], d[2], 0x07050301u);
    d[0] = o0; d[1] = o1; d[2] = o2; d[3] = o3;
  } else if constexpr (FROM == 4 && TO == 8) {
    uint32_t o0 = perm_b32(d[1], d[0], 0x05010400u), o1 = perm_b32(d[1], d[0], 0x07030602u);
    uint32_t o2 = perm_b32(d[3], d[2], 0x05010400u), o3 = perm_b32(d[3], d[2], 0x07030602u);
    d[0] = o0; d[1] = o1; d[2] = o2; d[3] = o3;
  } else if constexpr (FROM == 8 && TO == 2) {
    // 4x4 byte transpose: out r = byte r of every input dword
    uint32_t t0 = perm_b32(d[1], d[0], 0x05010400u);  // [x0,x4,x1,x5]
    uint32_t t1 = perm_b32(d[3], d[2], 0x05010400u);  // [x8,x12,x9,x13]
    uint32_t t2 = perm_b32(d[1], d[0], 0x07030602u);  // [x2,x6,x3,x7]
    uint32_t t3 = perm_b32(d[3], d[2], 0x07030602u);  // [x10,x14,x11,x15]
    d[0] = perm_b32(t1, t0, 0x05040100u);
    d[1] = perm_b32(t1, t0, 0x07060302u);
    d[2] = perm_b32(t3, t2, 0x05040100u);
    d[3] = perm_b32(t3, t2, 0x07060302u);
  } else if constexpr (FROM == 2 && TO == 8) {
    // the 4x4 byte transpose is its own inverse
    reorder_slot<8, 2>(d);
  } else if constexpr (FROM == 4 && TO == 2) {
    // [0,2,4,6][1,3,5,7][8,10,12,14][9,11,13,15] -> [0,4,8,12][1,5,9,13][2,6,10,14][3,7,11,15]
    uint32_t o0 = perm_b32(d[2], d[0], 0x06040200u), o1 = perm_b32(d[3], d[1], 0x06040200u);
    uint32_t o2 = perm_b32(d[2], d[0], 0x07050301u), o3 = perm_b32(d[3], d[1], 0x07050301u);
    d[0] = o0; d[1] = o1; d[2] = o2; d[3] = o3;
  } else if constexpr (FROM == 2 && TO == 4) {
    uint32_t o0 = perm_b32(d[2], d[0], 0x05010400u), o1 = perm_b32(d[3], d[1], 0x05010400u);
    uint32_t o2 = perm_b32(d[2], d[0], 0x07030602u), o3 = perm_b32(d[3], d[1], 0x07030602u);
    d[0] = o0; d[1] = o1; d[2] = o2; d[3] = o3;
  }
}

// ---------------------------------------------------------------------------
// float <-> storage dtype
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// round to nearest even (v_cvt_f16_f32 under the default rounding mode)
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, long i) {
  if constexpr (DT == kBF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == kF16) return f16_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}

template <int DT>
__device__ __forceinline__ float round_to_dtype(float v) {
  if constexpr (DT == kBF16) return bf16_to_f32(f32_to_bf16(v));
  else if constexpr (DT == kF16) return f16_to_f32(f32_to_f16(v));
  else return v;
}

__device__ __forceinline__ float load_bias(const void* bias, int dt, int n) {
  if (dt == kBF16) return bf16_to_f32(((const uint16_t*)bias)[n]);
  if (dt == kF16) return f16_to_f32(((const uint16_t*)bias)[n]);
  return ((const float*)bias)[n];
}

template <int DT>
__device__ __forceinline__ void store_out(void* out, long i, float v) {
  if constexpr (DT == kBF16) ((uint16_t*)out)[i] = f32_to_bf16(v);
  else if constexpr (DT == kF16) ((uint16_t*)out)[i] = f32_to_f16(v);
  else ((float*)out)[i] = v;
}

// y = fmaf(acc, ws, bias) with a bias, acc * ws without one.
__device__ __forceinline__ float finish(float acc, float ws, const void* bias, int bias_dt, int n) {
  return bias ? __builtin_fmaf(acc, ws, load_bias(bias, bias_dt, n)) : acc * ws;
}

__device__ __forceinline__ v4i mfma16x16x64(const uint32_t a[4], const uint32_t b[4], v4i c) {
  v4i av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
  v4i bv = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, c, 0, 0, 0);
}

}  // namespace actune
