// Packed W{2,4,8} x A{2,4,8} group-64 GEMMs for gfx950 (int8 MFMA).
//
// Restates the reference kernels actune/kernels/grouped.py:74-94 (_group_gemm)
// and actune/kernels/grouped_native.cu:42-88 (grouped<T,W,A>):
//   d[m,n,g] = sum_{k in g} a[m,k] * w[n,k]            int32, exact
//   y[m,n]   = (sum_g f32(d) * as[m,g]) * ws[n] (+ bias[n])  -> out dtype (RNE)
// with the fp32 sum taken in the canonical chunked order (common.hpp), so all
// kernels and tile configurations here give bit-identical outputs.
//
// MFMA mapping: v_mfma_i32_16x16x64_i8 with the weight tile as the A operand
// (16 output channels n x 64 k = one group) and the activation tile as the B
// operand (64 k x 16 tokens m). Lane l = 16*kb + i supplies A row i and B
// column i for the 16-k slot kb; D lane l holds rows n = 4*kb + r (r = 0..3)
// of column m = i, so each lane needs one activation scale per group.
//
// Kernels:
//  * gemm_smallm: M <= 16 (decode / action chunks). HBM-bound on the packed
//    weights. One workgroup owns 16 output channels over all of K; its waves
//    split K along the canonical chunks (split-K inside the workgroup), each
//    lane streams 16-byte weight loads (global_load_dwordx4) that cover
//    8/W groups, and v_permlane32/16_swap turn them into MFMA slots without
//    LDS. Chunk partials are combined through LDS in chunk order.
//  * gemm_tiled: any M. Each wave owns TN x TM 16x16 MFMA tiles; fragments
//    are read straight from global memory (L1/L2 serve the reuse).
#include "common.hpp"
#include "launch.hpp"

namespace actune {

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

// Packed bytes of one 16-element slot of width B (2B bytes) at p.
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

// Activation B-operand slot for token row arow at k offset koff, reordered to
// the weight width's element order.
template <int W, int A>
__device__ __forceinline__ void act_slot(const uint8_t* arow, bool ok, int koff, uint32_t d[4]) {
  uint32_t p[4];
  load_slot<A>(arow + (koff * A) / 8, ok, p);
  unpack_slot<A>(p, d);
  reorder_slot<A, W>(d);
}

// ---------------------------------------------------------------------------
template <int W, int A, int NW, bool DOTS>
__global__ __launch_bounds__(NW * 64) void gemm_smallm(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, const void* __restrict__ bias, int bias_dt, void* __restrict__ out,
    int out_dt, int32_t* __restrict__ dots, int M, int N, int K) {
  constexpr int GS = 8 / W;       // groups covered by one 16-byte weight load per lane
  constexpr int DG = 8;           // groups per load batch
  constexpr int DS = DG / GS;     // 16-byte weight loads per lane per batch
  constexpr int CPW = kChunks / NW;
  constexpr int T = shift_of(W) + shift_of(A);
  const float fold = __builtin_ldexpf(1.0f, -T);
  __shared__ float red[kChunks][16][17];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int G = K / kGroup;
  const int n0 = blockIdx.x * 16;
  const long wrow_bytes = (long)K * W / 8;
  const bool row_ok = n0 + i < N;
  const uint8_t* wrow = w + (long)(row_ok ? n0 + i : 0) * wrow_bytes;
  const bool m_ok = i < M;
  const uint8_t* arow = a + (long)(m_ok ? i : 0) * ((long)K * A / 8);
  const float* srow = as + (long)(m_ok ? i : 0) * G;
  const int slot_k = smallm_slot_k<W>(kb);

  for (int cc = 0; cc < CPW; ++cc) {
    const int c = wave * CPW + cc;
    const int gb = chunk_begin(c, G), ge = chunk_begin(c + 1, G);
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    // Batches of DG groups: every weight, activation and scale load of the
    // batch is issued before any of them is consumed, so a wave keeps
    // DS x 16 B of weights per lane in flight instead of one load at a time.
    for (int g0 = gb; g0 < ge; g0 += DG) {
      uint32_t wv[DS][4];
      uint32_t ap[DG][4];
      float sc[DG];
#pragma unroll
      for (int t = 0; t < DS; ++t) {
        const int g = g0 + t * GS;
        const long off = (long)g * 8 * W + kb * 16;
        load_slot<8>(wrow + off, row_ok && g < ge && off < wrow_bytes, wv[t]);
      }
#pragma unroll
      for (int j = 0; j < DG; ++j) {
        const int gg = g0 + j;
        const bool ok = m_ok && gg < ge;
        load_slot<A>(arow + ((gg * kGroup + slot_k) * A) / 8, ok, ap[j]);
        if constexpr (!DOTS) sc[j] = ok ? srow[gg] * fold : 0.0f;
      }
#pragma unroll
      for (int t = 0; t < DS; ++t) {
        exchange<W>(wv[t]);
#pragma unroll
        for (int j = 0; j < GS; ++j) {
          const int gg = g0 + t * GS + j;
          if (gg >= ge) break;
          uint32_t wd[4], ad[4];
          unpack_slot<W>(&wv[t][j * W / 2], wd);
          unpack_slot<A>(ap[t * GS + j], ad);
          reorder_slot<A, W>(ad);
          const v4i D = mfma16x16x64(wd, ad, v4i{0, 0, 0, 0});
          if constexpr (DOTS) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int n = n0 + 4 * kb + r;
              if (n < N && m_ok) dots[((long)i * N + n) * G + gg] = D[r] >> T;
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = __builtin_fmaf((float)D[r], sc[t * GS + j], p[r]);
          }
        }
      }
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[c][4 * kb + r][i] = p[r];
    }
  }
  if constexpr (DOTS) return;
  __syncthreads();
  if (threadIdx.x < 256) {
    const int nl = threadIdx.x >> 4, m = threadIdx.x & 15, n = n0 + nl;
    float acc = red[0][nl][m];
#pragma unroll
    for (int c = 1; c < kChunks; ++c) acc = acc + red[c][nl][m];
    if (n < N && m < M) {
      const float y = finish(acc, ws[n], bias, bias_dt, n);
      const long o = (long)m * N + n;
      if (out_dt == kBF16) store_out<kBF16>(out, o, y);
      else if (out_dt == kF16) store_out<kF16>(out, o, y);
      else store_out<kF32>(out, o, y);
    }
  }
}

// ---------------------------------------------------------------------------
template <int W, int A, int TN, int TM, bool DOTS>
__global__ __launch_bounds__(256) void gemm_tiled(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, const void* __restrict__ bias, int bias_dt, void* __restrict__ out,
    int out_dt, int32_t* __restrict__ dots, int M, int N, int K) {
  constexpr int T = shift_of(W) + shift_of(A);
  const float fold = __builtin_ldexpf(1.0f, -T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int G = K / kGroup;
  const int nb = blockIdx.x * (2 * TN * 16) + (wave & 1) * (TN * 16);
  const int mb = blockIdx.y * (2 * TM * 16) + (wave >> 1) * (TM * 16);
  const long wrow_bytes = (long)K * W / 8, arow_bytes = (long)K * A / 8;

  const uint8_t* wrow[TN];
  bool wok[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int n = nb + t * 16 + i;
    wok[t] = n < N;
    wrow[t] = w + (long)(wok[t] ? n : 0) * wrow_bytes;
  }
  const uint8_t* arow[TM];
  const float* srow[TM];
  bool aok[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int m = mb + t * 16 + i;
    aok[t] = m < M;
    arow[t] = a + (long)(aok[t] ? m : 0) * arow_bytes;
    srow[t] = as + (long)(aok[t] ? m : 0) * G;
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
        load_slot<W>(wrow[t] + (koff * W) / 8, wok[t], raw);
        unpack_slot<W>(raw, wd[t]);
      }
#pragma unroll
      for (int t = 0; t < TM; ++t) act_slot<W, A>(arow[t], aok[t], koff, ad[t]);
      float s[TM];
#pragma unroll
      for (int t = 0; t < TM; ++t) s[t] = aok[t] ? srow[t][g] * fold : 0.0f;
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

// ---------------------------------------------------------------------------
// Launch table. Config ids (stable, part of the ABI; see actune_hip.h):
//   0,1,2  gemm_smallm with 4, 8, 16 waves (M <= 16 only)
//   3..6   gemm_tiled with (TN,TM) = (2,2), (4,2), (2,4), (4,4)
template <int W, int A, bool DOTS>
static void launch_wa(int config, const GemmArgs& g, hipStream_t st) {
#define ACT_ARGS g.a, g.as, g.w, g.ws, g.bias, g.bias_dt, g.out, g.out_dt, g.dots, g.M, g.N, g.K
  const dim3 gs((unsigned)((g.N + 15) / 16));
  switch (config) {
    case 0: gemm_smallm<W, A, 4, DOTS><<<gs, 256, 0, st>>>(ACT_ARGS); break;
    case 1: gemm_smallm<W, A, 8, DOTS><<<gs, 512, 0, st>>>(ACT_ARGS); break;
    case 2: gemm_smallm<W, A, 16, DOTS><<<gs, 1024, 0, st>>>(ACT_ARGS); break;
#define TILED(TN, TM)                                                                         \
  gemm_tiled<W, A, TN, TM, DOTS><<<dim3((unsigned)((g.N + 32 * TN - 1) / (32 * TN)),           \
                                        (unsigned)((g.M + 32 * TM - 1) / (32 * TM))),          \
                                   256, 0, st>>>(ACT_ARGS)
    case 3: TILED(2, 2); break;
    case 4: TILED(4, 2); break;
    case 5: TILED(2, 4); break;
    case 6: TILED(4, 4); break;
#undef TILED
  }
#undef ACT_ARGS
}

template <bool DOTS>
static void launch_dispatch(int W, int A, int config, const GemmArgs& g, hipStream_t st) {
#define CASE(WB, AB) if (W == WB && A == AB) return launch_wa<WB, AB, DOTS>(config, g, st)
  CASE(8, 8); CASE(8, 4); CASE(8, 2);
  CASE(4, 8); CASE(4, 4); CASE(4, 2);
  CASE(2, 8); CASE(2, 4); CASE(2, 2);
#undef CASE
}

void launch_gemm(int W, int A, int config, const GemmArgs& g, hipStream_t st) {
  launch_dispatch<false>(W, A, config, g, st);
}

void launch_dots(int W, int A, int config, const GemmArgs& g, hipStream_t st) {
  launch_dispatch<true>(W, A, config, g, st);
}

}  // namespace actune
