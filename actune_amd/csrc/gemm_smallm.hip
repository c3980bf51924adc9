// Small-M packed group-64 GEMM for gfx950 (decode and action-chunk shapes,
// M <= 64): HBM-bound on the packed weights.
//
// Restates the per-call math of actune/kernels/grouped.py:74-94 and
// actune/kernels/grouped_native.cu:42-88 (exact int32 dot per 64-group,
// fp32 rescale by the activation scale, weight-scale epilogue), reduced in
// the canonical chunked order of common.hpp.
//
// Structure:
//  * One workgroup owns 16 output channels of one problem (a problem is one
//    linear; up to kMaxProblems linears that share the same input run in one
//    launch) and one block of 16*MT tokens (blockIdx.y) over all of K, and NW
//    waves split K along the 16 canonical chunks (split-K inside the
//    workgroup, no global scratch).
//  * Each lane streams 16-byte weight loads (global_load_dwordx4): lanes
//    kb = 0..3 of a row fetch 64 consecutive bytes = 8/W groups, and
//    v_permlane32/16_swap turn them into MFMA slots without LDS.
//  * Loads are batched: every activation, scale and weight load of DG groups
//    is issued before the batch is consumed, activations first (loads
//    complete in issue order, so the activation work waits only for the
//    activations). The epilogue's weight scale and bias are fetched at entry.
//  * v_mfma_i32_16x16x64_i8 with the weight rows as the A operand and up to
//    16 tokens per column tile (MT tiles) as the B operand; one fp32 FMA per
//    (row, token, group).
//  * MODE_FUSED (M <= 4): each wave quantizes the activation groups of its
//    own K-range straight from x (the group-64 quantizer of
//    grouped.py:55-71, optionally dividing by the channel scale of
//    layers.py:41-42) into a per-wave LDS slab laid out as MFMA B slots, while
//    its weight loads are in flight; no separate quantizer launch.
//  * Chunk partials meet in LDS and are added in chunk order.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

template <int W, int A, int NW, int MT, int MODE, int DT, bool SCALE>
__global__ __launch_bounds__(NW * 64) void gemm_smallm(const LinearArgs args) {
  constexpr int GS = 8 / W;                        // groups per 16-byte weight load per lane
  constexpr int DG = (8 / MT) > GS ? (8 / MT) : GS;  // groups per load batch
  constexpr int DS = DG / GS;                      // weight loads per lane per batch
  constexpr int CPW = kChunks / NW;                // canonical chunks per wave
  constexpr int T = shift_of(W) + shift_of(A);
  constexpr bool FUSED = MODE == kModeFused;
  constexpr bool DOTS = MODE == kModeDots;
  constexpr int COLS = 16 * MT;
  constexpr int EPT = (16 * COLS + NW * 64 - 1) / (NW * 64);  // epilogue outputs per thread
  constexpr int XL = DT == kF32 ? 2 : 1;           // 16-byte loads per 8 elements of x
  constexpr uint32_t ESZ = DT == kF32 ? 4 : 2;
  constexpr int FM = 4;                            // largest M of the fused mode
  static_assert(!FUSED || (MT == 1 && DG == 8), "fused quantization serves M <= 4");

  __shared__ float red[DOTS ? 1 : kChunks][16][COLS + 1];
  __shared__ __align__(16) uint8_t slab[FUSED ? NW : 1][FUSED ? DG * FM * kGroup : 16];
  __shared__ float sslab[FUSED ? NW : 1][FUSED ? DG * FM : 1];

  const float fold = __builtin_ldexpf(1.0f, -T);
  const Problem pr = select_problem(args, blockIdx.x);
  const int M = args.M, K = args.K, N = pr.N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int G = K / kGroup;
  const int n0 = ((int)blockIdx.x - pr.tile0) * 16;
  const int m_base = (int)blockIdx.y * COLS;  // first token of this workgroup's token block
  const uint32_t wrow_bytes = (uint32_t)K * W / 8;
  const bool row_ok = n0 + i < N;
  const Rsrc wres = make_rsrc(pr.w, (uint32_t)N * wrow_bytes);
  const uint32_t wrow = (uint32_t)(n0 + i) * wrow_bytes;
  const int slot_k = smallm_slot_k<W>(kb);

  // Epilogue constants of the outputs this thread finishes, fetched first.
  ChannelConst cc_out[DOTS ? 1 : EPT];
  if constexpr (!DOTS) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int e = (int)threadIdx.x + j * NW * 64;
      cc_out[j] = fetch_channel(pr.ws, pr.bias, args.bias_dt, N, n0 + e / COLS, e < 16 * COLS);
    }
  }

  // activation row offsets (bytes) of this lane's tokens, kOff when m >= M
  const uint32_t arow_bytes = (uint32_t)K * A / 8;
  Rsrc ares, sres, xres, xsres;
  if constexpr (FUSED) {
    xres = make_rsrc(args.x, (uint32_t)M * K * ESZ);
    xsres = make_rsrc(SCALE ? args.xscale : args.x, (uint32_t)K * ESZ);
  } else {
    ares = make_rsrc(args.a, (uint32_t)M * arow_bytes);
    sres = make_rsrc(args.as, (uint32_t)M * G * 4);
  }
  uint32_t arow[MT];
  bool aok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m_base + 16 * t + i;
    aok[t] = m < M;
    arow[t] = (uint32_t)m;
  }

  for (int cc = 0; cc < CPW; ++cc) {
    const int c = wave * CPW + cc;
    const int gb = chunk_begin(c, G), ge = chunk_begin(c + 1, G);
    float p[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[t][r] = 0.f;

    for (int g0 = gb; g0 < ge; g0 += DG) {
      // 1. Activation operands first: loads complete in issue order, so
      //    consuming them waits only for them, not for the weights below.
      //    Fused: lane (j = lane/8, seg = lane%8) reads elements seg*8..+7 of
      //    group g0+j of every token m < M.
      v4u xr[FUSED ? FM : 1][XL], dr[FUSED && SCALE ? FM : 1][XL];
      uint32_t ap[FUSED ? 1 : DG][MT][4];
      float sc[FUSED ? 1 : DG][MT];
      const int fj = lane >> 3, seg = lane & 7;
      if constexpr (FUSED) {
        const int g = g0 + fj;
        const uint32_t k0 = (uint32_t)(g * kGroup + seg * 8);
#pragma unroll
        for (int m = 0; m < FM; ++m) {
          const bool live = m < M && g < ge;
          const uint32_t xo = live ? ((uint32_t)m * K + k0) * ESZ : kOff;
#pragma unroll
          for (int h = 0; h < XL; ++h)
            xr[m][h] = __builtin_amdgcn_raw_buffer_load_b128(xres, xo == kOff ? kOff : xo + 16 * h, 0, 0);
          if constexpr (SCALE) {
            const uint32_t so = live ? k0 * ESZ : kOff;
#pragma unroll
            for (int h = 0; h < XL; ++h)
              dr[m][h] = __builtin_amdgcn_raw_buffer_load_b128(xsres, so == kOff ? kOff : so + 16 * h, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < DG; ++j) {
          const int gg = g0 + j;
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const bool ok = aok[t] && gg < ge;
            const uint32_t aoff = arow[t] * arow_bytes + (uint32_t)((gg * kGroup + slot_k) * A) / 8;
            buffer_slot<A>(ares, ok ? aoff : kOff, ap[j][t]);
            if constexpr (!DOTS) sc[j][t] = buffer_f32(sres, ok ? (arow[t] * G + gg) * 4u : kOff) * fold;
          }
        }
      }
      // Keep the scheduler from hoisting weight loads above the activation
      // loads (the point of the order above).
      __builtin_amdgcn_sched_barrier(0);
      // 2. Weights of the batch.
      uint32_t wv[DS][4];
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const int g = g0 + s * GS;
        const uint32_t off = (uint32_t)g * 8 * W + kb * 16;
        buffer_slot<8>(wres, row_ok && g < ge && off < wrow_bytes ? wrow + off : kOff, wv[s]);
      }
      // 3. Fused: quantize into the wave's slab (as MFMA B slots, row j*FM+m)
      //    while the weights are in flight, then read the slots back.
      uint32_t bq[FUSED ? DG : 1][4];
      float bs[FUSED ? DG : 1];
      if constexpr (FUSED) {
        uint8_t* my_slab = slab[wave];
        const bool glive = g0 + fj < ge;
#pragma unroll
        for (int m = 0; m < FM; ++m) {
          if (m < M) {  // wave-uniform
            float v[8];
            unpack8<DT>(xr[m][0], xr[m][XL - 1], v);
            if constexpr (SCALE) {
              float d[8];
              unpack8<DT>(dr[m][0], dr[m][XL - 1], d);
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] = glive ? round_to_dtype<DT>(v[e] / d[e]) : 0.0f;
            }
            uint32_t cq[8];
            const float s = group_code_bits<A, DT>(v, cq);
            if (glive) {
              store_half_slot<W, A>(my_slab + (fj * FM + m) * kGroup + (seg >> 1) * 16, seg & 1, cq);
              if (seg == 0) sslab[wave][fj * FM + m] = s * fold;
            }
          }
        }
        // LDS operations of one wave complete in order; keep the compiler from
        // moving the slab reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const bool ok = i < M;
#pragma unroll
        for (int j = 0; j < DG; ++j) {
          v4u q = v4u{0u, 0u, 0u, 0u};
          if (ok) q = *reinterpret_cast<const v4u*>(my_slab + (j * FM + i) * kGroup + slot_k);
          bq[j][0] = q[0]; bq[j][1] = q[1]; bq[j][2] = q[2]; bq[j][3] = q[3];
          bs[j] = ok ? sslab[wave][j * FM + i] : 0.0f;
        }
      }
      // 4. Exchange, unpack, MFMA, rescale.
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        exchange<W>(wv[s]);
#pragma unroll
        for (int jj = 0; jj < GS; ++jj) {
          const int j = s * GS + jj, gg = g0 + j;
          if (gg >= ge) break;
          uint32_t wd[4];
          unpack_slot<W>(&wv[s][jj * W / 2], wd);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            uint32_t bd[4];
            float scale;
            if constexpr (FUSED) {
              bd[0] = bq[j][0]; bd[1] = bq[j][1]; bd[2] = bq[j][2]; bd[3] = bq[j][3];
              scale = bs[j];
            } else {
              unpack_slot<A>(ap[j][t], bd);
              reorder_slot<A, W>(bd);
              scale = DOTS ? 0.0f : sc[j][t];
            }
            const v4i D = mfma16x16x64(wd, bd, v4i{0, 0, 0, 0});
            if constexpr (DOTS) {
              const int m = m_base + 16 * t + i;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int n = n0 + 4 * kb + r;
                if (n < N && m < M) args.dots[((long)m * N + n) * G + gg] = D[r] >> T;
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) p[t][r] = __builtin_fmaf((float)D[r], scale, p[t][r]);
            }
          }
        }
      }
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[c][4 * kb + r][16 * t + i] = p[t][r];
    }
  }
  if constexpr (DOTS) return;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = (int)threadIdx.x + j * NW * 64;
    if (e >= 16 * COLS) break;
    const int nl = e / COLS, mc = e % COLS, n = n0 + nl, m = m_base + mc;
    float acc = red[0][nl][mc];
#pragma unroll
    for (int c = 1; c < kChunks; ++c) acc = acc + red[c][nl][mc];
    if (n < N && m < M) {
      const float y = finish_const(acc, cc_out[j], pr.bias != nullptr, args.bias_dt);
      const long o = (long)m * N + n;
      if (args.out_dt == kBF16) store_out<kBF16>(pr.out, o, y);
      else if (args.out_dt == kF16) store_out<kF16>(pr.out, o, y);
      else store_out<kF32>(pr.out, o, y);
    }
  }
}

// ---------------------------------------------------------------------------
template <int W, int A, int NW, int MT>
static void launch_nw_mt(int mode, const LinearArgs& g, hipStream_t st) {
  const dim3 grid((unsigned)g.tiles, (unsigned)((g.M + 16 * MT - 1) / (16 * MT))), block(NW * 64);
  if (mode == kModeDots) {
    gemm_smallm<W, A, NW, MT, kModeDots, kBF16, false><<<grid, block, 0, st>>>(g);
  } else if (mode == kModePacked) {
    gemm_smallm<W, A, NW, MT, kModePacked, kBF16, false><<<grid, block, 0, st>>>(g);
  } else if constexpr (MT == 1) {
#define FUSED_DT(DTV)                                                                               \
  if (g.xscale) gemm_smallm<W, A, NW, 1, kModeFused, DTV, true><<<grid, block, 0, st>>>(g);        \
  else gemm_smallm<W, A, NW, 1, kModeFused, DTV, false><<<grid, block, 0, st>>>(g)
    if (g.x_dt == kBF16) { FUSED_DT(kBF16); }
    else if (g.x_dt == kF16) { FUSED_DT(kF16); }
    else { FUSED_DT(kF32); }
#undef FUSED_DT
  }
}

// Few row tiles: one 16-token block per workgroup, over a second grid
// dimension, so that the workgroups cover the GPU (the weight rows are then
// re-read per token block, from L2). Many row tiles: all tokens in one
// workgroup, so each weight row is read once.
template <int W, int A, int NW>
static void launch_nw(int mode, const LinearArgs& g, hipStream_t st) {
  if (g.M <= 16 || g.tiles < 512) launch_nw_mt<W, A, NW, 1>(mode, g, st);
  else if (g.M <= 32) launch_nw_mt<W, A, NW, 2>(mode, g, st);
  else launch_nw_mt<W, A, NW, 4>(mode, g, st);
}

template <int W, int A>
static void launch_wa(int nw, int mode, const LinearArgs& g, hipStream_t st) {
  if (nw == 4) launch_nw<W, A, 4>(mode, g, st);
  else if (nw == 8) launch_nw<W, A, 8>(mode, g, st);
  else launch_nw<W, A, 16>(mode, g, st);
}

void launch_smallm(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB) if (W == WB && A == AB) return launch_wa<WB, AB>(nw, mode, g, st)
  CASE(8, 8); CASE(8, 4); CASE(8, 2);
  CASE(4, 8); CASE(4, 4); CASE(4, 2);
  CASE(2, 8); CASE(2, 4); CASE(2, 2);
#undef CASE
}

}  // namespace actune
