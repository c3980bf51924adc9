// MFMA-tiled packed group-64 GEMM for gfx950 (any M; used for M > 64).
//
// Restates actune/kernels/grouped.py:74-94 / grouped_native.cu:42-88 with the
// canonical chunked fp32 order (common.hpp). Each wave owns TN x TM 16x16
// MFMA tiles of v_mfma_i32_16x16x64_i8 (weights as the A operand, tokens as
// the B operand); fragments are read straight from global memory.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

// ---------------------------------------------------------------------------
template <int W, int A, int TN, int TM, bool DOTS>
__global__ __launch_bounds__(256) void gemm_tiled(const LinearArgs args) {
  const uint8_t* __restrict__ a = args.a;
  const float* __restrict__ as = args.as;
  const uint8_t* __restrict__ w = args.prob[0].w;
  const float* __restrict__ ws = args.prob[0].ws;
  const void* __restrict__ bias = args.prob[0].bias;
  void* __restrict__ out = args.prob[0].out;
  int32_t* __restrict__ dots = args.dots;
  const int bias_dt = args.bias_dt, out_dt = args.out_dt;
  const int M = args.M, N = args.prob[0].N, K = args.K;
  constexpr int T = shift_of(W) + shift_of(A);
  const float fold = __builtin_ldexpf(1.0f, -T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int G = K / kGroup;
  const int nb = blockIdx.x * (2 * TN * 16) + (wave & 1) * (TN * 16);
  const int mb = blockIdx.y * (2 * TM * 16) + (wave >> 1) * (TM * 16);
  const uint32_t wrow_bytes = (uint32_t)K * W / 8, arow_bytes = (uint32_t)K * A / 8;
  const Rsrc wres = make_rsrc(w, (uint32_t)N * wrow_bytes);
  const Rsrc ares = make_rsrc(a, (uint32_t)M * arow_bytes);
  const Rsrc sres = make_rsrc(as, (uint32_t)M * G * 4);

  uint32_t wrow[TN];
  bool wok[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int n = nb + t * 16 + i;
    wok[t] = n < N;
    wrow[t] = (uint32_t)n * wrow_bytes;
  }
  uint32_t arow[TM];
  bool aok[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int m = mb + t * 16 + i;
    aok[t] = m < M;
    arow[t] = (uint32_t)m;
  }

  float acc[TN][TM][4];
#pragma unroll
  for (int x = 0; x < TN; ++x)
#pragma unroll
    for (int y = 0; y < TM; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[x][y][r] = 0.f;

  for (int c = 0; c < kChunks; ++c) {
    const int gb = chunk_begin(c, G), ge = chunk_begin(c + 1, G);
    float p[TN][TM][4];
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[x][y][r] = 0.f;
    for (int g = gb; g < ge; ++g) {
      const int koff = g * kGroup + kb * 16;
      uint32_t wd[TN][4], ad[TM][4];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        uint32_t raw[4];
        buffer_slot<W>(wres, wok[t] ? wrow[t] + (uint32_t)(koff * W) / 8 : kOff, raw);
        unpack_slot<W>(raw, wd[t]);
      }
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        uint32_t raw[4];
        buffer_slot<A>(ares, aok[t] ? arow[t] * arow_bytes + (uint32_t)(koff * A) / 8 : kOff, raw);
        unpack_slot<A>(raw, ad[t]);
        reorder_slot<A, W>(ad[t]);
      }
      float s[TM];
#pragma unroll
      for (int t = 0; t < TM; ++t) s[t] = DOTS ? 0.0f : buffer_f32(sres, aok[t] ? (arow[t] * G + g) * 4u : kOff) * fold;
#pragma unroll
      for (int x = 0; x < TN; ++x)
#pragma unroll
        for (int y = 0; y < TM; ++y) {
          const v4i D = mfma16x16x64(wd[x], ad[y], v4i{0, 0, 0, 0});
          if constexpr (DOTS) {
            const int m = mb + y * 16 + i;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int n = nb + x * 16 + 4 * kb + r;
              if (n < N && m < M) dots[((long)m * N + n) * G + g] = D[r] >> T;
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) p[x][y][r] = __builtin_fmaf((float)D[r], s[y], p[x][y][r]);
          }
        }
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int x = 0; x < TN; ++x)
#pragma unroll
        for (int y = 0; y < TM; ++y)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[x][y][r] = c == 0 ? p[x][y][r] : acc[x][y][r] + p[x][y][r];
    }
  }
  if constexpr (DOTS) return;
#pragma unroll
  for (int x = 0; x < TN; ++x)
#pragma unroll
    for (int y = 0; y < TM; ++y) {
      const int m = mb + y * 16 + i;
      if (m >= M) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nb + x * 16 + 4 * kb + r;
        if (n >= N) continue;
        const float v = finish(acc[x][y][r], ws[n], bias, bias_dt, n);
        const long o = (long)m * N + n;
        if (out_dt == kBF16) store_out<kBF16>(out, o, v);
        else if (out_dt == kF16) store_out<kF16>(out, o, v);
        else store_out<kF32>(out, o, v);
      }
    }
}

// Shapes (TN, TM): 0 = (2,2), 1 = (4,2), 2 = (2,4), 3 = (4,4); single problem.
template <int W, int A, bool DOTS>
static void launch_shape(int shape, const LinearArgs& g, hipStream_t st) {
#define TILED(TN, TM)                                                                           \
  gemm_tiled<W, A, TN, TM, DOTS><<<dim3((unsigned)((g.prob[0].N + 32 * TN - 1) / (32 * TN)),    \
                                        (unsigned)((g.M + 32 * TM - 1) / (32 * TM))),            \
                                   256, 0, st>>>(g)
  switch (shape) {
    case 0: TILED(2, 2); break;
    case 1: TILED(4, 2); break;
    case 2: TILED(2, 4); break;
    default: TILED(4, 4); break;
  }
#undef TILED
}

void launch_tiled(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB)                                                                \
  if (W == WB && A == AB) {                                                         \
    if (dots) launch_shape<WB, AB, true>(shape, g, st);                             \
    else launch_shape<WB, AB, false>(shape, g, st);                                 \
    return;                                                                         \
  }
  CASE(8, 8) CASE(8, 4) CASE(8, 2) CASE(4, 8) CASE(4, 4) CASE(4, 2) CASE(2, 8) CASE(2, 4) CASE(2, 2)
#undef CASE
}

}  // namespace actune
