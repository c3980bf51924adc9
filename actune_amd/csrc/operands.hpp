// Operand fetch / exchange helpers and the exact group-64 code computation
// shared by the quantizer and the GEMM kernels.
#pragma once
#include "common.hpp"

namespace actune {

// ---------------------------------------------------------------------------
// Raw buffer loads. A buffer resource covers `bytes` bytes from `base`; a
// lane whose 32-bit offset is at or beyond that range reads zeros, so
// predicated operand loads need no branch and a wave can keep all of its
// loads in flight (a predicated global load would be wrapped in an exec
// branch with its own wait). kOff marks a lane's load as switched off; the
// C ABI keeps every operand buffer below 2 GiB so kOff is always outside.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOff = 0x80000000u;

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the gfx9-family raw buffer setting
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 2B bytes (one 16-element slot of width B) at byte offset off; zeros if off
// is out of range.
template <int B>
__device__ __forceinline__ void buffer_slot(Rsrc r, uint32_t off, uint32_t out[4]) {
  if constexpr (B == 8) {
    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    out[0] = q[0]; out[1] = q[1]; out[2] = q[2]; out[3] = q[3];
  } else if constexpr (B == 4) {
    const v2u q = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    out[0] = q[0]; out[1] = q[1]; out[2] = 0u; out[3] = 0u;
  } else {
    out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    out[1] = out[2] = out[3] = 0u;
  }
}

__device__ __forceinline__ float buffer_f32(Rsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Epilogue constants of one output channel, fetched early so that their
// latency hides under the weight stream: the weight scale and the raw bits
// of the bias element (fp32 bits, or the 16-bit payload for bf16/f16). The
// conversion waits until the value is used, so nothing stalls on the load.
struct ChannelConst {
  float ws;
  uint32_t bias_bits;
};

__device__ __forceinline__ ChannelConst fetch_channel(const float* ws, const void* bias, int bias_dt, int N,
                                                      int n, bool live) {
  const Rsrc wr = make_rsrc(ws, (uint32_t)N * 4u);
  const Rsrc br = make_rsrc(bias, bias ? (uint32_t)N * (bias_dt == kF32 ? 4u : 2u) : 0u);
  live = live && n < N;
  ChannelConst c;
  c.ws = buffer_f32(wr, live ? (uint32_t)n * 4u : kOff);
  if (bias_dt == kF32) c.bias_bits = __builtin_amdgcn_raw_buffer_load_b32(br, live ? (uint32_t)n * 4u : kOff, 0, 0);
  else c.bias_bits = __builtin_amdgcn_raw_buffer_load_b16(br, live ? (uint32_t)n * 2u : kOff, 0, 0);
  return c;
}

// The bias value held by raw bias bits of dtype bias_dt.
__device__ __forceinline__ float bias_from_bits(uint32_t bits, int bias_dt) {
  return bias_dt == kF32 ? __uint_as_float(bits)
       : bias_dt == kBF16 ? bf16_to_f32((uint16_t)bits)
                          : f16_to_f32((uint16_t)bits);
}

// y = fmaf(acc, ws, bias) with a bias, acc * ws without one (same as finish()).
__device__ __forceinline__ float finish_const(float acc, ChannelConst c, bool has_bias, int bias_dt) {
  if (!has_bias) return acc * c.ws;
  return __builtin_fmaf(acc, c.ws, bias_from_bits(c.bias_bits, bias_dt));
}

// Eight consecutive elements of dtype DT at byte offset off as fp32 (zeros
// when off is out of range).
template <int DT>
__device__ __forceinline__ void buffer_load8(Rsrc r, uint32_t off, float v[8]) {
  if constexpr (DT == kF32) {
    const v4u a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const v4u b = __builtin_amdgcn_raw_buffer_load_b128(r, off == kOff ? kOff : off + 16, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = __uint_as_float(a[e]); v[e + 4] = __uint_as_float(b[e]); }
  } else {
    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = (uint16_t)(q[e] & 0xffffu), hi = (uint16_t)(q[e] >> 16);
      if constexpr (DT == kBF16) { v[2 * e] = bf16_to_f32(lo); v[2 * e + 1] = bf16_to_f32(hi); }
      else { v[2 * e] = f16_to_f32(lo); v[2 * e + 1] = f16_to_f32(hi); }
    }
  }
}

// Eight consecutive elements of dtype DT held in q0 (and q1 for fp32) as fp32.
template <int DT>
__device__ __forceinline__ void unpack8(const v4u& q0, const v4u& q1, float v[8]) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = __uint_as_float(q0[e]); v[e + 4] = __uint_as_float(q1[e]); }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = (uint16_t)(q0[e] & 0xffffu), hi = (uint16_t)(q0[e] >> 16);
      if constexpr (DT == kBF16) { v[2 * e] = bf16_to_f32(lo); v[2 * e + 1] = bf16_to_f32(hi); }
      else { v[2 * e] = f16_to_f32(lo); v[2 * e + 1] = f16_to_f32(hi); }
    }
  }
}

// Packed bytes of one 16-element slot of width B (2B bytes) at p; zeros
// when !ok (nothing is read).
template <int B>
__device__ __forceinline__ void load_slot(const uint8_t* p, bool ok, uint32_t out[4]) {
  out[0] = out[1] = out[2] = out[3] = 0u;
  if (!ok) return;
  if constexpr (B == 8) {
    const v4u q = *reinterpret_cast<const v4u*>(p);
    out[0] = q[0]; out[1] = q[1]; out[2] = q[2]; out[3] = q[3];
  } else if constexpr (B == 4) {
    const v2u q = *reinterpret_cast<const v2u*>(p);
    out[0] = q[0]; out[1] = q[1];
  } else {
    out[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

// Eight consecutive elements starting at element i (i % 8 == 0) as fp32,
// with 16-byte vector loads.
template <int DT>
__device__ __forceinline__ void load8(const void* p, long i, float v[8]) {
  if constexpr (DT == kF32) {
    const v4u a = reinterpret_cast<const v4u*>(p)[i / 4];
    const v4u b = reinterpret_cast<const v4u*>(p)[i / 4 + 1];
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = __uint_as_float(a[e]); v[e + 4] = __uint_as_float(b[e]); }
  } else {
    const v4u q = reinterpret_cast<const v4u*>(p)[i / 8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = (uint16_t)(q[e] & 0xffffu), hi = (uint16_t)(q[e] >> 16);
      if constexpr (DT == kBF16) { v[2 * e] = bf16_to_f32(lo); v[2 * e + 1] = bf16_to_f32(hi); }
      else { v[2 * e] = f16_to_f32(lo); v[2 * e + 1] = f16_to_f32(hi); }
    }
  }
}

// E consecutive elements starting at element i (i % E == 0) as fp32: load8
// for E = 8, one 4-, 8- or 16-byte load for E = 2 or 4.
template <int DT, int E>
__device__ __forceinline__ void load_n(const void* p, long i, float v[E]) {
  if constexpr (E == 8) {
    load8<DT>(p, i, v);
  } else {
    static_assert(E == 2 || E == 4, "2, 4 or 8 elements per lane");
    constexpr int ES = DT == kF32 ? 4 : 2;  // element bytes
    constexpr int NW = E * ES / 4;          // dwords
    uint32_t w[NW];
    const char* src = reinterpret_cast<const char*>(p) + i * ES;
    if constexpr (NW == 4) {
      const v4u q = *reinterpret_cast<const v4u*>(src);
      w[0] = q[0]; w[1] = q[1]; w[2] = q[2]; w[3] = q[3];
    } else if constexpr (NW == 2) {
      const v2u q = *reinterpret_cast<const v2u*>(src);
      w[0] = q[0]; w[1] = q[1];
    } else {
      w[0] = *reinterpret_cast<const uint32_t*>(src);
    }
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      if constexpr (DT == kF32) {
        v[j] = __uint_as_float(w[j]);
      } else {
        const uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
        if constexpr (DT == kBF16) { v[2 * j] = bf16_to_f32(lo); v[2 * j + 1] = bf16_to_f32(hi); }
        else { v[2 * j] = f16_to_f32(lo); v[2 * j + 1] = f16_to_f32(hi); }
      }
    }
  }
}

// Maximum of non-negative floats over an aligned L-lane segment (L = 8, 16
// or 32), in every lane of the segment: DPP moves (quad xor 1, quad xor 2,
// the mirror inside each 8-lane half row, then the mirror of the 16-lane
// row), for 32 lanes a swap of odd and even rows, and integer max on the
// bit patterns, which orders non-negative floats like their values; no LDS
// round trip. All 64 lanes must execute it.
template <int L>
__device__ __forceinline__ float seg_max(float a) {
  static_assert(L == 8 || L == 16 || L == 32, "8, 16 or 32 lanes");
  uint32_t u = __float_as_uint(a);
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, false));   // [1,0,3,2]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xF, 0xF, false));   // [2,3,0,1]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xF, 0xF, false));  // half-row mirror
  if constexpr (L >= 16) u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x140, 0xF, 0xF, false));  // row mirror
  if constexpr (L >= 32) {
    // rows 0/1 (and 2/3) exchanged: each lane sees its own row and the other
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    u = max((uint32_t)r[0], (uint32_t)r[1]);
  }
  return __uint_as_float(u);
}

// 1.5 * 2^23: adding it to a float q with |q| <= 2^22 rounds q to the nearest
// integer (ties to even, the default rounding mode), and the low byte of the
// sum's bit pattern is then that integer in two's complement.
constexpr float kRoundMagic = 12582912.0f;

// Group-64 codes of E elements held by one lane of a (64 / E)-lane segment
// group (8 elements and 8 lanes unless E says otherwise): amax over the group, s = fl(max(amax, 1e-8) / P) and c = clamp(rint(fl(v /
// s)), -P-1, P). For 16-bit inputs the quotient is x * y with y = fl(1/s)
// plus one FMA correction (Markstein), which gives the IEEE codes for every
// bf16 and f16 input (proved exhaustively by tests/exhaustive_division.c);
// fp32 inputs use the IEEE division itself. The quotient is clamped first
// (the bounds are integers, so clamp and round commute) and rounded by the
// magic add; cb[e] holds the sum's bits, whose low byte is code e. All 64
// lanes of the wave must call this together.
template <int A, int DT, int E = 8>
__device__ __forceinline__ float group_code_bits(const float v[E], uint32_t cb[E]) {
  constexpr int P = (1 << (A - 1)) - 1;
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(seg_max<64 / E>(amax), 1e-8f);
  float s;
  if constexpr (DT == kF32 || P == 1) {
    s = amax / (float)P;
  } else {
    // amax is a 16-bit float value or f32(1e-8): with yp = fl(1/P), the
    // product q0 = fl(amax * yp) and one FMA correction with the exact
    // residual give fl(amax / P) for every such amax and P in {7, 127}
    // (checked for all of them by tests/exhaustive_division.c), without the
    // IEEE division sequence on the quantizer's serial path
    constexpr float yp = 1.0f / (float)P;
    const float q0 = amax * yp;
    const float r = __builtin_fmaf(-q0, (float)P, amax);
    s = __builtin_fmaf(r, yp, q0);
  }
  const float y = 1.0f / s;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float q;
    if constexpr (DT == kF32) {
      q = v[e] / s;
    } else {
      const float q0 = v[e] * y;
      const float r = __builtin_fmaf(-q0, s, v[e]);
      q = __builtin_fmaf(r, y, q0);
    }
    q = fminf(fmaxf(q, (float)(-P - 1)), (float)P);
    cb[e] = __float_as_uint(q + kRoundMagic);
  }
  return s;
}

// Same codes as integers.
template <int A, int DT, int E = 8>
__device__ __forceinline__ float group_codes(const float v[E], int c[E]) {
  uint32_t cb[E];
  const float s = group_code_bits<A, DT, E>(v, cb);
#pragma unroll
  for (int e = 0; e < E; ++e) c[e] = (int)(int8_t)(cb[e] & 0xffu);
  return s;
}

// Byte offset of k-slot kb (16 elements) inside a group, after the weight
// exchange of gemm_smallm. W4 loads give each lane 32 consecutive k; the
// swap leaves lanes kb = 0..3 with slots 0, 2, 1, 3 (k offsets 0, 32, 16, 48).
template <int W>
__device__ __forceinline__ int smallm_slot_k(int kb) {
  if constexpr (W == 4) return ((kb & 1) << 5) | ((kb >> 1) << 4);
  else return kb << 4;
}

// Turn one 16-byte weight load per lane (lanes kb = 0..3 of a row hold 64
// consecutive bytes = 8/W groups) into one 16-element slot per group:
//   W8: no exchange, slot = the 4 dwords;
//   W4: lanes 0-31 hold group g, lanes 32-63 group g+1; swapping dwords 2,3
//       of the low half with dwords 0,1 of the high half leaves dwords 0,1 =
//       slot of g and dwords 2,3 = slot of g+1 in every lane;
//   W2: lane kb holds group g+kb; a 4x4 transpose of dwords across the four
//       lane rows (permlane32 then permlane16 swaps) leaves dword j = slot kb
//       of group g+j.
template <int W>
__device__ __forceinline__ void exchange(uint32_t v[4]) {
  if constexpr (W == 4) {
    auto r0 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    auto r1 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    v[0] = r0[0]; v[2] = r0[1]; v[1] = r1[0]; v[3] = r1[1];
  } else if constexpr (W == 2) {
    auto r0 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    auto r1 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    v[0] = r0[0]; v[2] = r0[1]; v[1] = r1[0]; v[3] = r1[1];
    auto r2 = __builtin_amdgcn_permlane16_swap(v[0], v[1], false, false);
    auto r3 = __builtin_amdgcn_permlane16_swap(v[2], v[3], false, false);
    v[0] = r2[0]; v[1] = r2[1]; v[2] = r3[0]; v[3] = r3[1];
  }
}

// Activation B-operand slot for token row arow at k offset koff, reordered to
// the weight width's element order.
template <int W, int A>
__device__ __forceinline__ void act_slot(const uint8_t* arow, bool ok, int koff, uint32_t d[4]) {
  uint32_t p[4];
  load_slot<A>(arow + (koff * A) / 8, ok, p);
  unpack_slot<A>(p, d);
  reorder_slot<A, W>(d);
}

// Low bytes of code bits (group_code_bits) a, b, c, d as one dword
// [a, b, c, d], with v_perm_b32.
__device__ __forceinline__ uint32_t code_quad(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint32_t lo = perm_b32(b, a, 0x0C0C0400u);  // [a, b, 0, 0]
  const uint32_t hi = perm_b32(d, c, 0x0C0C0400u);  // [c, d, 0, 0]
  return perm_b32(hi, lo, 0x05040100u);
}

// Shift every byte of d left by 8-A inside the byte (the code field moves to
// the top of its byte: c * 2^(8-A) as int8).
template <int A>
__device__ __forceinline__ uint32_t shift_bytes(uint32_t d) {
  if constexpr (A == 8) return d;
  else if constexpr (A == 4) return (d << 4) & 0xF0F0F0F0u;
  else return (d << 6) & 0xC0C0C0C0u;
}

// Store 8 consecutive codes (elements 8h..8h+7 of a 16-element slot, as
// code bits from group_code_bits) into the slot at `slot`, shifted to the top
// of their byte for width A, in the element order of weight width W
// (common.hpp, unpack_slot).
template <int W, int A>
__device__ __forceinline__ void store_half_slot(uint8_t* slot, int h, const uint32_t cb[8]) {
  if constexpr (W == 8) {
    *reinterpret_cast<v2u*>(slot + 8 * h) =
        v2u{shift_bytes<A>(code_quad(cb[0], cb[1], cb[2], cb[3])), shift_bytes<A>(code_quad(cb[4], cb[5], cb[6], cb[7]))};
  } else if constexpr (W == 4) {
    *reinterpret_cast<v2u*>(slot + 8 * h) =
        v2u{shift_bytes<A>(code_quad(cb[0], cb[2], cb[4], cb[6])), shift_bytes<A>(code_quad(cb[1], cb[3], cb[5], cb[7]))};
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<uint16_t*>(slot + 4 * r + 2 * h) = (uint16_t)shift_bytes<A>(perm_b32(cb[4 + r], cb[r], 0x0C0C0400u));
  }
}

}  // namespace actune
