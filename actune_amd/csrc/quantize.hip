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
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

template <int A, int DT, bool SCALE>
__global__ __launch_bounds__(256) void quantize_groups_kernel(const void* __restrict__ x,
                                                              const void* __restrict__ input_scale,
                                                              long groups, int G,
                                                              uint8_t* __restrict__ packed,
                                                              float* __restrict__ scales) {
  const long gi = (long)blockIdx.x * 32 + (threadIdx.x >> 3);  // global group index m*G + g
  const int seg = threadIdx.x & 7;                               // 8-element segment in the group
  const bool live = gi < groups;
  const long gsafe = live ? gi : groups - 1;
  const long e0 = gsafe * kGroup + seg * 8;                      // first element of this lane
  const int k0 = (int)(gsafe % G) * kGroup + seg * 8;            // its column (for input_scale)

  float v[8];
  load8<DT>(x, e0, v);
  if constexpr (SCALE) {
    float d[8];
    load8<DT>(input_scale, k0, d);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = round_to_dtype<DT>(v[e] / d[e]);
  }
  int c[8];
  const float s = group_codes<A, DT>(v, c);
  uint32_t bits[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t field = (uint32_t)c[e] & ((1u << A) - 1u);
    const int bit = e * A;  // bit position inside this lane's 8*A-bit run
    bits[bit >> 5] |= field << (bit & 31);
  }
  if (!live) return;
  uint8_t* dst = packed + gi * (kGroup * A / 8) + seg * A;
  if constexpr (A == 8) {
    *reinterpret_cast<v2u*>(dst) = v2u{bits[0], bits[1]};
  } else if constexpr (A == 4) {
    *reinterpret_cast<uint32_t*>(dst) = bits[0];
  } else {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)bits[0];
  }
  if (seg == 0) scales[gi] = s;
}

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

}  // namespace actune
