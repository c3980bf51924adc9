// Persistent streaming small-M GEMM for gfx950 (M <= 16), the default decode
// kernel. Same arithmetic as gemm_smallm (exact int32 group dots, fp32
// canonical chunked order) with a different schedule:
//
//  * Stage once: each wave owns the same K-range (NW of the 16 canonical
//    chunks) in every row tile, so it writes the MFMA B operands of its
//    K-range into LDS once per kernel: quantized from x (fused mode, M <= 4;
//    the group-64 quantizer of grouped.py:55-71 with the optional channel
//    scale of layers.py:41-42) or unpacked and reordered from the packed
//    activations (packed mode). Rows M..15 read a zero row.
//  * Stream: the grid is sized to the resident capacity and each workgroup
//    walks row tiles with a stride of gridDim.x. A wave's work per tile is a
//    short list of items of DSB 16-byte weight loads per lane; the loads of
//    item q+1 (possibly of the next tile) are issued before item q is
//    consumed, so the weights of the next tile are in flight while the
//    current one finishes its MFMAs and its cross-wave reduction.
//  * Reduce: per tile, chunk partials meet in LDS and are added in chunk
//    order (same as gemm_smallm), then scaled and stored.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

__device__ __forceinline__ void tile_problem(const LinearArgs& args, int tile, const uint8_t*& w,
                                             const float*& ws, const void*& bias, void*& out, int& N,
                                             int& tile0) {
  w = args.prob[0].w; ws = args.prob[0].ws; bias = args.prob[0].bias; out = args.prob[0].out;
  N = args.prob[0].N; tile0 = args.prob[0].tile0;
#pragma unroll
  for (int q = 1; q < kMaxProblems; ++q) {
    if (q < args.nprob && tile >= args.prob[q].tile0) {
      w = args.prob[q].w; ws = args.prob[q].ws; bias = args.prob[q].bias; out = args.prob[q].out;
      N = args.prob[q].N; tile0 = args.prob[q].tile0;
    }
  }
}

// LDS layout (dynamic): per wave a slab [GW][ROWS][64 B] of B slots and a
// scale slab [GW][ROWS] (fp32, already multiplied by 2^-(sW+sA)), one 64-byte
// zero row, and the chunk-partial arrays red[2][16][16][17] (one per parity of
// the workgroup's tile counter, so one barrier per tile suffices).
template <int W, int A, int NW, int MODE, int DT, bool SCALE>
__global__ __launch_bounds__(NW * 64) void gemm_stream(const LinearArgs args, int GW, int ROWS) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int GS = 8 / W;        // groups per 16-byte weight load per lane
  constexpr int DSB = 4;           // weight loads per lane per item
  constexpr int GB = DSB * GS;     // groups per item
  constexpr int CPW = kChunks / NW;
  constexpr int T = shift_of(W) + shift_of(A);
  constexpr bool FUSED = MODE == kModeFused;

  const float fold = __builtin_ldexpf(1.0f, -T);
  const int M = args.M, K = args.K, G = K / kGroup;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int c_first = wave * CPW;
  const int wg0 = chunk_begin(c_first, G), wg1 = chunk_begin(c_first + CPW, G);

  uint8_t* slab = smem + (size_t)wave * GW * ROWS * kGroup;
  float* sslab = reinterpret_cast<float*>(smem + (size_t)NW * GW * ROWS * kGroup) + (size_t)wave * GW * ROWS;
  uint8_t* zero_row = reinterpret_cast<uint8_t*>(sslab - (size_t)wave * GW * ROWS + (size_t)NW * GW * ROWS);
  float (*red2)[kChunks][16][17] = reinterpret_cast<float (*)[kChunks][16][17]>(zero_row + kGroup);

  // ---------------------------------------------------------------- stage
  // The activation loads of up to kPass passes are issued together, then
  // converted into B slots; passes beyond kPass run load-then-convert. No
  // weight load is issued before the staging is complete (see below).
  constexpr int kPass = 4;
  constexpr int ESZ = DT == kF32 ? 4 : 2;
  constexpr int LPR = FUSED ? 8 : 4;             // lanes per group-row
  constexpr int RPP = 64 / LPR;                  // group-rows per pass
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(zero_row)[threadIdx.x] = 0u;
  const int rows_here = (wg1 - wg0) * M;         // group-rows of this wave
  const int npass = (rows_here + RPP - 1) / RPP;
  const uint32_t arow_bytes = (uint32_t)K * A / 8;
  Rsrc xres, xsres, ares, sres;
  if constexpr (FUSED) {
    xres = make_rsrc(args.x, (uint32_t)M * K * ESZ);
    xsres = make_rsrc(SCALE ? args.xscale : args.x, (uint32_t)K * ESZ);
  } else {
    ares = make_rsrc(args.a, (uint32_t)M * arow_bytes);
    sres = make_rsrc(args.as, (uint32_t)M * G * 4);
  }
  // group-row of this lane in pass p, and its load offsets
  auto row_of = [&](int pass, int& gl, int& m, bool& live) {
    const int idx = pass * RPP + lane / LPR;
    live = idx < rows_here;
    gl = live ? idx / M : 0;
    m = live ? idx % M : 0;
  };
  struct Raw { v4u x0, x1, s0, s1; uint32_t p[4]; float sc; };
  auto issue = [&](int pass, Raw& r) {
    int gl, m; bool live;
    row_of(pass, gl, m, live);
    const int g = wg0 + gl;
    if constexpr (FUSED) {
      const int seg = lane & 7;
      const uint32_t k0 = (uint32_t)(g * kGroup + seg * 8);
      const uint32_t xo = live ? ((uint32_t)m * K + k0) * ESZ : kOff;
      r.x0 = __builtin_amdgcn_raw_buffer_load_b128(xres, xo, 0, 0);
      if constexpr (DT == kF32) r.x1 = __builtin_amdgcn_raw_buffer_load_b128(xres, xo == kOff ? kOff : xo + 16, 0, 0);
      if constexpr (SCALE) {
        const uint32_t so = live ? k0 * ESZ : kOff;
        r.s0 = __builtin_amdgcn_raw_buffer_load_b128(xsres, so, 0, 0);
        if constexpr (DT == kF32) r.s1 = __builtin_amdgcn_raw_buffer_load_b128(xsres, so == kOff ? kOff : so + 16, 0, 0);
      }
    } else {
      const int q = lane & 3;
      buffer_slot<A>(ares, live ? (uint32_t)m * arow_bytes + (uint32_t)((g * kGroup + q * 16) * A) / 8 : kOff, r.p);
      r.sc = buffer_f32(sres, live && q == 0 ? ((uint32_t)m * G + g) * 4u : kOff);
    }
  };
  auto convert = [&](int pass, const Raw& r) {
    int gl, m; bool live;
    row_of(pass, gl, m, live);
    if constexpr (FUSED) {
      const int seg = lane & 7;
      float v[8];
      unpack8<DT>(r.x0, r.x1, v);
      if constexpr (SCALE) {
        float d[8];
        unpack8<DT>(r.s0, r.s1, d);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = live ? round_to_dtype<DT>(v[e] / d[e]) : 0.0f;
      }
      uint32_t cq[8];
      const float s = group_code_bits<A, DT>(v, cq);
      if (live) {
        store_half_slot<W, A>(slab + (gl * ROWS + m) * kGroup + (seg >> 1) * 16, seg & 1, cq);
        if (seg == 0) sslab[gl * ROWS + m] = s * fold;
      }
    } else {
      const int q = lane & 3;
      uint32_t d[4];
      unpack_slot<A>(r.p, d);
      reorder_slot<A, W>(d);
      if (live) {
        *reinterpret_cast<v4u*>(slab + (gl * ROWS + m) * kGroup + q * 16) = v4u{d[0], d[1], d[2], d[3]};
        if (q == 0) sslab[gl * ROWS + m] = r.sc * fold;
      }
    }
  };
  Raw early[kPass];
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (p < npass) issue(p, early[p]);

  // ---------------------------------------------------------------- stream
  const int slot_k = smallm_slot_k<W>(kb);
  const int tiles = args.tiles;
  const int my_tiles = ((int)blockIdx.x < tiles) ? (tiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int nb = wg1 > wg0 ? (wg1 - wg0 + GB - 1) / GB : 1;  // items per tile (1 empty item if no groups)
  const int items = my_tiles * nb;
  const uint32_t wrow_bytes = (uint32_t)K * W / 8;

  // Each item load also fetches the epilogue constants of its tile for the
  // thread that finishes channel threadIdx.x / 16 (threads < 256), so the
  // per-tile epilogue never waits on a fresh memory round trip.
  auto load_item = [&](int q, uint32_t (&buf)[DSB][4], ChannelConst& cc) {
    const int tile = (int)blockIdx.x + (q / nb) * (int)gridDim.x;
    const int gs = wg0 + (q % nb) * GB;
    const uint8_t* w; const float* ws; const void* bias; void* out; int N, tile0;
    tile_problem(args, tile, w, ws, bias, out, N, tile0);
    const int n = (tile - tile0) * 16 + i;
    const Rsrc wres = make_rsrc(w, (uint32_t)N * wrow_bytes);
#pragma unroll
    for (int s = 0; s < DSB; ++s) {
      const int g = gs + s * GS;
      const uint32_t off = (uint32_t)g * 8 * W + kb * 16;
      const bool ok = n < N && g < wg1 && off < wrow_bytes;
      buffer_slot<8>(wres, ok ? (uint32_t)n * wrow_bytes + off : kOff, buf[s]);
    }
    cc = fetch_channel(ws, bias, args.bias_dt, N, (tile - tile0) * 16 + ((int)threadIdx.x >> 4), threadIdx.x < 256);
  };

  uint32_t cur[DSB][4], nxt[DSB][4];
  ChannelConst cur_cc{0.0f, 0u}, nxt_cc{0.0f, 0u};
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (p < npass) convert(p, early[p]);
  for (int p = kPass; p < npass; ++p) {
    Raw r;
    issue(p, r);
    convert(p, r);
  }
  __syncthreads();  // slabs and the zero row are visible to their readers
  // The weight stream starts only now: issued earlier, the first items of all
  // workgroups (tens of MB) would sit in front of the small activation loads
  // in the memory system and hold the staging, and so every tile, back by
  // several microseconds.
  if (items > 0) load_item(0, cur, cur_cc);

  float p[4] = {0.f, 0.f, 0.f, 0.f};
  int par = 0;                                // parity of the workgroup's current tile
  int c = c_first;                            // chunk being accumulated
  int cend = chunk_begin(c + 1, G);
  for (int q = 0; q < items; ++q) {
    const bool more = q + 1 < items;
    if (more) load_item(q + 1, nxt, nxt_cc);
    const int b = q % nb;
    const int gs = wg0 + b * GB;
#pragma unroll
    for (int s = 0; s < DSB; ++s) {
      exchange<W>(cur[s]);
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        const int gg = gs + s * GS + jj;
        if (gg >= wg1) break;
        while (gg >= cend) {  // close finished (possibly empty) chunks
#pragma unroll
          for (int r = 0; r < 4; ++r) { red2[par][c][4 * kb + r][i] = p[r]; p[r] = 0.f; }
          ++c;
          cend = chunk_begin(c + 1, G);
        }
        uint32_t wd[4];
        unpack_slot<W>(&cur[s][jj * W / 2], wd);
        const int gl = gg - wg0;
        const uint8_t* brow = i < M ? slab + (gl * ROWS + i) * kGroup + slot_k : zero_row;
        const v4u bq = *reinterpret_cast<const v4u*>(brow);
        const uint32_t bd[4] = {bq[0], bq[1], bq[2], bq[3]};
        const float scale = sslab[gl * ROWS + (i < M ? i : 0)];
        const v4i D = mfma16x16x64(wd, bd, v4i{0, 0, 0, 0});
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = __builtin_fmaf((float)D[r], scale, p[r]);
      }
    }
    if (b == nb - 1) {
      // end of this tile for the wave: close its remaining chunks, reduce
      for (; c < c_first + CPW; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) { red2[par][c][4 * kb + r][i] = p[r]; p[r] = 0.f; }
      }
      c = c_first;
      cend = chunk_begin(c + 1, G);
      __syncthreads();
      if (threadIdx.x < 256) {
        const int tile = (int)blockIdx.x + (q / nb) * (int)gridDim.x;
        const uint8_t* w; const float* ws; const void* bias; void* out; int N, tile0;
        tile_problem(args, tile, w, ws, bias, out, N, tile0);
        const int nl = threadIdx.x >> 4, m = threadIdx.x & 15, n = (tile - tile0) * 16 + nl;
        float acc = red2[par][0][nl][m];
#pragma unroll
        for (int cc = 1; cc < kChunks; ++cc) acc = acc + red2[par][cc][nl][m];
        if (n < N && m < M) {
          const float y = finish_const(acc, cur_cc, bias != nullptr, args.bias_dt);
          const long o = (long)m * N + n;
          if (args.out_dt == kBF16) store_out<kBF16>(out, o, y);
          else if (args.out_dt == kF16) store_out<kF16>(out, o, y);
          else store_out<kF32>(out, o, y);
        }
      }
      // No second barrier: the next tile writes red2[par ^ 1], and the one
      // after it writes red2[par] only after the next tile's barrier, which
      // the epilogue threads reach after finishing this epilogue.
      par ^= 1;
    }
    if (more) {
#pragma unroll
      for (int s = 0; s < DSB; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) cur[s][e] = nxt[s][e];
      cur_cc = nxt_cc;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: LDS sizing, resident-capacity grid, dispatch.
static int max_wave_groups(int G, int nw) {
  const int cpw = kChunks / nw;
  int gw = 0;
  for (int w = 0; w < nw; ++w) {
    const int d = chunk_begin((w + 1) * cpw, G) - chunk_begin(w * cpw, G);
    gw = d > gw ? d : gw;
  }
  return gw > 0 ? gw : 1;
}

size_t stream_lds_bytes(int K, int M, int nw) {
  const int G = K / kGroup, rows = (M + 3) & ~3;
  const size_t gw = (size_t)max_wave_groups(G, nw);
  return (size_t)nw * gw * rows * (kGroup + 4) + kGroup + 2 * sizeof(float) * kChunks * 16 * 17;
}

template <typename Kern>
static int resident_grid(Kern kern, int threads, size_t lds, int tiles) {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  int per_cu = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int cap = cus * per_cu;
  return tiles < cap ? tiles : cap;
}

template <int W, int A, int NW, int MODE, int DT, bool SCALE>
static void launch_one(const LinearArgs& g, hipStream_t st) {
  const size_t lds = stream_lds_bytes(g.K, g.M, NW);
  auto kern = gemm_stream<W, A, NW, MODE, DT, SCALE>;
  allow_dynamic_lds<gemm_stream<W, A, NW, MODE, DT, SCALE>>();
  const int grid = resident_grid(kern, NW * 64, lds, g.tiles);
  const int gw = max_wave_groups(g.K / kGroup, NW);
  kern<<<grid, NW * 64, lds, st>>>(g, gw, (g.M + 3) & ~3);
}

template <int W, int A, int NW>
static void launch_stream_nw(int mode, const LinearArgs& g, hipStream_t st) {
  if (mode == kModePacked) {
    launch_one<W, A, NW, kModePacked, kBF16, false>(g, st);
    return;
  }
#define FUSED_DT(DTV)                                                         \
  if (g.xscale) launch_one<W, A, NW, kModeFused, DTV, true>(g, st);          \
  else launch_one<W, A, NW, kModeFused, DTV, false>(g, st)
  if (g.x_dt == kBF16) { FUSED_DT(kBF16); }
  else if (g.x_dt == kF16) { FUSED_DT(kF16); }
  else { FUSED_DT(kF32); }
#undef FUSED_DT
}

template <int W, int A>
static void launch_stream_wa(int nw, int mode, const LinearArgs& g, hipStream_t st) {
  if (nw == 4) launch_stream_nw<W, A, 4>(mode, g, st);
  else if (nw == 8) launch_stream_nw<W, A, 8>(mode, g, st);
  else launch_stream_nw<W, A, 16>(mode, g, st);
}

void launch_stream(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB) if (W == WB && A == AB) return launch_stream_wa<WB, AB>(nw, mode, g, st)
  CASE(8, 8); CASE(8, 4); CASE(8, 2);
  CASE(4, 8); CASE(4, 4); CASE(4, 2);
  CASE(2, 8); CASE(2, 4); CASE(2, 2);
#undef CASE
}

}  // namespace actune
