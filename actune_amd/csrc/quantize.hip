// Group-64 activation quantizer for gfx950.
//
// Restates actune/kernels/grouped.py:55-71 (_quantize_groups) and the oracle
// form actune/calibration.py:12-14, with the optional channel-scale division
// of actune/layers.py:41-42 fused in front:
//   v = x (or dtype_round(x / input_scale)), p = 2^(A-1)-1,
//   s = fl32(max(max|v|, f32(1e-8)) / p)          (IEEE division)
//   c = clamp(rint_half_even(fl32(v / s)), -p-1, p)  (exact; see group_codes)
//   code k of row m -> byte m*(K*A/8) + k*A/8, bit (k % (8/A))*A.
//
// Layout: groups are 64 contiguous elements, and the M*K/64 groups of the
// row-major input are contiguous too. Each lane owns 8 consecutive elements
// (one 16-byte load for 16-bit inputs), 8 lanes own a group, a wave covers 8
// groups (1 KiB of bf16), and the group absmax is a 3-step DPP reduction
// inside the 8-lane segment. Stores are contiguous per wave:
// A8 writes 8 B/lane, A4 4 B/lane, A2 2 B/lane.
//
// The gated quantizer also has a narrow geometry for small inputs: 2
// elements per lane (4 for A2, so that a lane still stores whole bytes) and
// 32 (16) lanes per group. Its per-element work (the activation, two
// roundings and the product) is several times the plain quantizer's, and
// below 16384 groups the launch is too small to fill the chip: spreading a
// group over more lanes shortens each wave's serial work (M=50, K=4096,
// bf16 A4, in a hipGraph: 2.0 us against 2.9 us per launch). Above that,
// 8 elements per lane are as fast or faster (M=256, K=16384: 7.0 against
// 7.6 us with 2 per lane).
#include <math.h>

#include "../../include/actune_hip.h"
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

// One lane's E values v of group gi (segment seg, columns k0..k0+E-1): the
// channel-scale division when SCALE, the group's codes packed and stored
// (E*A bits at bit E*A*seg of the group's codes), and the scale stored by
// segment 0.
template <int A, int DT, bool SCALE, int E = 8>
__device__ __forceinline__ void quantize_lane(float (&v)[E], const void* __restrict__ input_scale, int k0,
                                              bool live, long gi, int seg, uint8_t* __restrict__ packed,
                                              float* __restrict__ scales) {
  static_assert(E * A >= 8, "a lane stores whole bytes");
  if constexpr (SCALE) {
    float d[E];
    load_n<DT, E>(input_scale, k0, d);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = round_to_dtype<DT>(v[e] / d[e]);
  }
  int c[E];
  const float s = group_codes<A, DT, E>(v, c);
  uint32_t bits[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t field = (uint32_t)c[e] & ((1u << A) - 1u);
    const int bit = e * A;  // bit position inside this lane's E*A-bit run
    bits[bit >> 5] |= field << (bit & 31);
  }
  if (!live) return;
  constexpr int B = E * A / 8;  // bytes per lane
  uint8_t* dst = packed + gi * (kGroup * A / 8) + seg * B;
  if constexpr (B == 8) {
    *reinterpret_cast<v2u*>(dst) = v2u{bits[0], bits[1]};
  } else if constexpr (B == 4) {
    *reinterpret_cast<uint32_t*>(dst) = bits[0];
  } else if constexpr (B == 2) {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)bits[0];
  } else {
    *dst = (uint8_t)bits[0];
  }
  if (seg == 0) scales[gi] = s;
}

// Lane geometry shared by the quantizers: E elements per lane, 64 / E lanes
// per group, 4 E groups per 256-thread workgroup; a lane past the last group
// works on the last group and stores nothing.
template <int E = 8>
struct LaneGroup {
  static constexpr int kLanes = kGroup / E;              // lanes per group
  static constexpr int kGroupsPerBlock = 256 / kLanes;
  long gi, e0;
  int seg, k0;
  bool live;
  __device__ LaneGroup(long groups, int G) {
    gi = (long)blockIdx.x * kGroupsPerBlock + threadIdx.x / kLanes;  // global group index m*G + g
    seg = threadIdx.x % kLanes;                                       // E-element segment in the group
    live = gi < groups;
    const long gsafe = live ? gi : groups - 1;
    e0 = gsafe * kGroup + seg * E;                                    // first element of this lane
    k0 = (int)(gsafe % G) * kGroup + seg * E;                         // its column (for input_scale)
  }
};

template <int A, int DT, bool SCALE>
__global__ __launch_bounds__(256) void quantize_groups_kernel(const void* __restrict__ x,
                                                              const void* __restrict__ input_scale,
                                                              long groups, int G,
                                                              uint8_t* __restrict__ packed,
                                                              float* __restrict__ scales) {
  const LaneGroup<> lg(groups, G);
  float v[8];
  load8<DT>(x, lg.e0, v);
  quantize_lane<A, DT, SCALE>(v, input_scale, lg.k0, lg.live, lg.gi, lg.seg, packed, scales);
}

// Gate activation of a gated MLP in fp32, as torch's GPU kernels compute it
// for torch.nn.functional.silu and gelu(approximate="tanh") (opmath float):
// SiLU x / (1 + e^-x); GELU 0.5 x (1 + tanh(b fma(k, x^3, x))) with
// b = sqrt(2) * 2/sqrt(pi) * 0.5 and k = 0.044715 rounded to fp32, the
// inner multiply-add fused as torch's build fuses it (checked against
// torch on MI355X for every fp32 value of an f16 input). The fp32 result is
// pinned in a register so that the rounding to f16 that follows stays a
// separate step: a multiply folded into the conversion (v_fma_mix) would
// round once from the exact product where torch rounds twice.
template <int ACT>
__device__ __forceinline__ float gate_act(float x) {
  float y;
  if constexpr (ACT == ACTUNE_ACT_SILU) {
    y = x / (1.0f + expf(-x));
  } else {
    constexpr float kBeta = (float)(M_SQRT2 * M_2_SQRTPI * 0.5);
    constexpr float kKappa = 0.044715f;
    const float cube = x * x * x;
    const float inner = kBeta * __builtin_fmaf(kKappa, cube, x);
    y = 0.5f * x * (1.0f + tanhf(inner));
  }
  asm volatile("" : "+v"(y));
  return y;
}

// Quantizer of the down projection's input p = act(gate) * up of a gated MLP:
// p is formed in the inputs' dtype as torch forms it (act rounded to the
// dtype, then the product rounded), then quantized exactly as
// quantize_groups_kernel quantizes a tensor holding p. E elements per lane.
template <int A, int DT, int ACT, bool SCALE, int E>
__global__ __launch_bounds__(256) void quantize_gated_kernel(const void* __restrict__ gate,
                                                             const void* __restrict__ up,
                                                             const void* __restrict__ input_scale,
                                                             long groups, int G,
                                                             uint8_t* __restrict__ packed,
                                                             float* __restrict__ scales) {
  const LaneGroup<E> lg(groups, G);
  float v[E], u[E];
  load_n<DT, E>(gate, lg.e0, v);
  load_n<DT, E>(up, lg.e0, u);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = round_to_dtype<DT>(round_to_dtype<DT>(gate_act<ACT>(v[e])) * u[e]);
  quantize_lane<A, DT, SCALE, E>(v, input_scale, lg.k0, lg.live, lg.gi, lg.seg, packed, scales);
}

// Elements per lane of the gated quantizer: the narrow geometry up to 16384
// groups, 8 above.
constexpr long kGatedNarrowMaxGroups = 16384;

template <int A, int DT>
static void launch_quantize_dt(const void* x, const void* sc, long M, long K, uint8_t* packed,
                               float* scales, hipStream_t stream) {
  const long groups = M * (K / kGroup);
  const dim3 grid((unsigned)((groups + 31) / 32));
  if (sc)
    quantize_groups_kernel<A, DT, true><<<grid, 256, 0, stream>>>(x, sc, groups, (int)(K / kGroup), packed, scales);
  else
    quantize_groups_kernel<A, DT, false><<<grid, 256, 0, stream>>>(x, sc, groups, (int)(K / kGroup), packed, scales);
}

template <int A>
static void launch_quantize_a(const void* x, int dt, const void* sc, long M, long K, uint8_t* packed,
                              float* scales, hipStream_t stream) {
  if (dt == kBF16) launch_quantize_dt<A, kBF16>(x, sc, M, K, packed, scales, stream);
  else if (dt == kF16) launch_quantize_dt<A, kF16>(x, sc, M, K, packed, scales, stream);
  else launch_quantize_dt<A, kF32>(x, sc, M, K, packed, scales, stream);
}

void launch_quantize(const void* x, int dt, const void* sc, long M, long K, int A, uint8_t* packed,
                     float* scales, hipStream_t stream) {
  if (A == 8) launch_quantize_a<8>(x, dt, sc, M, K, packed, scales, stream);
  else if (A == 4) launch_quantize_a<4>(x, dt, sc, M, K, packed, scales, stream);
  else launch_quantize_a<2>(x, dt, sc, M, K, packed, scales, stream);
}

template <int A, int DT, int ACT, int E>
static void launch_gated_e(const void* gate, const void* up, const void* sc, long groups, int G, uint8_t* packed,
                           float* scales, hipStream_t stream) {
  constexpr long per_block = LaneGroup<E>::kGroupsPerBlock;
  const dim3 grid((unsigned)((groups + per_block - 1) / per_block));
  if (sc)
    quantize_gated_kernel<A, DT, ACT, true, E><<<grid, 256, 0, stream>>>(gate, up, sc, groups, G, packed, scales);
  else
    quantize_gated_kernel<A, DT, ACT, false, E><<<grid, 256, 0, stream>>>(gate, up, sc, groups, G, packed, scales);
}

template <int A, int DT, int ACT>
static void launch_gated_t(const void* gate, const void* up, const void* sc, long M, long K, uint8_t* packed,
                           float* scales, hipStream_t stream) {
  const long groups = M * (K / kGroup);
  const int G = (int)(K / kGroup);
  if (groups <= kGatedNarrowMaxGroups)
    launch_gated_e<A, DT, ACT, A == 2 ? 4 : 2>(gate, up, sc, groups, G, packed, scales, stream);
  else
    launch_gated_e<A, DT, ACT, 8>(gate, up, sc, groups, G, packed, scales, stream);
}

template <int A, int DT>
static void launch_gated_dt(const void* gate, const void* up, int act, const void* sc, long M, long K,
                            uint8_t* packed, float* scales, hipStream_t stream) {
  if (act == ACTUNE_ACT_SILU) launch_gated_t<A, DT, ACTUNE_ACT_SILU>(gate, up, sc, M, K, packed, scales, stream);
  else launch_gated_t<A, DT, ACTUNE_ACT_GELU_TANH>(gate, up, sc, M, K, packed, scales, stream);
}

template <int A>
static void launch_gated_a(const void* gate, const void* up, int dt, int act, const void* sc, long M, long K,
                           uint8_t* packed, float* scales, hipStream_t stream) {
  if (dt == kBF16) launch_gated_dt<A, kBF16>(gate, up, act, sc, M, K, packed, scales, stream);
  else if (dt == kF16) launch_gated_dt<A, kF16>(gate, up, act, sc, M, K, packed, scales, stream);
  else launch_gated_dt<A, kF32>(gate, up, act, sc, M, K, packed, scales, stream);
}

void launch_quantize_gated(const void* gate, const void* up, int dt, int act, const void* sc, long M, long K, int A,
                           uint8_t* packed, float* scales, hipStream_t stream) {
  if (A == 8) launch_gated_a<8>(gate, up, dt, act, sc, M, K, packed, scales, stream);
  else if (A == 4) launch_gated_a<4>(gate, up, dt, act, sc, M, K, packed, scales, stream);
  else launch_gated_a<2>(gate, up, dt, act, sc, M, K, packed, scales, stream);
}

}  // namespace actune
