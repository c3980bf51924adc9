// MFMA-tiled packed group-64 GEMM for gfx950 (prefill shapes, M > 64).
//
// Restates actune/kernels/grouped.py:74-94 / grouped_native.cu:42-88 with the
// canonical chunked fp32 order (common.hpp), bit-identical to the small-M
// kernels.
//
// Structure (one workgroup = 4 waves in a WN x WM = 2 x 2 arrangement; each
// wave owns TN x TM 16x16 MFMA tiles, so the workgroup tile is
// BN = 32*TN weight rows by BM = 32*TM tokens):
//  * Staging: every stage covers KG = 2 groups. The packed weight and
//    activation bytes of the stage are fetched with 16-byte buffer loads
//    (coalesced along K), unpacked to shifted int8 and reordered to the
//    weight width's element order ONCE per workgroup, and written to LDS as
//    16-byte MFMA slots; activation scales go to LDS with the 2^-(sW+sA)
//    fold applied. Slot positions are XOR-swizzled by row so that the 16 rows
//    read by one ds_read_b128 spread over the banks.
//  * Pipeline: LDS is double-buffered; the global loads of stage s+1 are in
//    flight while stage s is multiplied, and are unpacked into the other
//    buffer afterwards (one barrier per stage).
//  * Math: per group, TN + TM ds_read_b128 fragments feed TN x TM
//    v_mfma_i32_16x16x64_i8 (weights = A operand, tokens = B operand), then
//    one cvt + one fma per output element with the token's group scale.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

constexpr int kTileKG = 2;    // groups per stage
constexpr int kTileRing = 3;  // stages whose global loads are in flight (register ring)

// LDS byte offset of slot `slot` of row `row` of group `gl` in a [KG][rows][4]
// slot array. Rows are 64 bytes, so rows r and r+2 start in the same 16-byte
// bank group; XOR-ing the slot with (row >> 1) & 3 gives the 8 consecutive
// rows read by 8 lanes of one ds_read_b128 cycle 8 distinct bank groups.
__device__ __forceinline__ int slot_addr(int gl, int row, int rows, int slot) {
  return ((gl * rows + row) * 4 + (slot ^ ((row >> 1) & 3))) * 16;
}

template <int W, int A, int TN, int TM, bool DOTS>
__global__ __launch_bounds__(256) void gemm_tiled(const LinearArgs args) {
  constexpr int R = TN * TM >= 16 ? 2 : kTileRing;  // the 128x128 tile keeps 2 for registers
  constexpr int BN = 32 * TN, BM = 32 * TM, KG = kTileKG;
  constexpr int T = shift_of(W) + shift_of(A);
  // bytes of packed data per row per stage, and 16-byte chunks per stage
  constexpr int WROW = KG * 8 * W, AROW = KG * 8 * A;
  constexpr int WCH = BN * WROW / 16, ACH = BM * AROW / 16;
  constexpr int WPT = (WCH + 255) / 256, APT = (ACH + 255) / 256;  // chunks per thread
  constexpr int SPT = (BM * KG + 255) / 256;                        // scales per thread
  constexpr int WBYTES = KG * BN * 64, ABYTES = KG * BM * 64, SBYTES = KG * BM * 4;
  constexpr int STAGE = WBYTES + ABYTES + SBYTES;
  __shared__ __align__(16) uint8_t lds[2][STAGE];

  const float fold = __builtin_ldexpf(1.0f, -T);
  const int M = args.M, K = args.K, N = args.prob[0].N, G = K / kGroup;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int n_blk = blockIdx.x * BN, m_blk = blockIdx.y * BM;
  const int wn = (wave & 1) * TN * 16, wm = (wave >> 1) * TM * 16;  // wave origin inside the tile

  const uint32_t wrow_bytes = (uint32_t)K * W / 8, arow_bytes = (uint32_t)K * A / 8;
  const Rsrc wres = make_rsrc(args.prob[0].w, (uint32_t)N * wrow_bytes);
  const Rsrc ares = make_rsrc(args.a, (uint32_t)M * arow_bytes);
  const Rsrc sres = make_rsrc(args.as, DOTS ? 4u : (uint32_t)M * G * 4);

  uint32_t wraw_r[R][WPT][4], araw_r[R][APT][4];
  float sraw_r[R][SPT];

  auto fetch = [&](int g0, uint32_t (&wraw)[WPT][4], uint32_t (&araw)[APT][4], float (&sraw)[SPT]) {
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int ch = tid + t * 256, row = ch / (WROW / 16), cc = ch % (WROW / 16);
      const int n = n_blk + row;
      const uint32_t off = (uint32_t)g0 * 8 * W + cc * 16;
      const bool ok = ch < WCH && n < N && off < wrow_bytes;
      buffer_slot<8>(wres, ok ? (uint32_t)n * wrow_bytes + off : kOff, wraw[t]);
    }
#pragma unroll
    for (int t = 0; t < APT; ++t) {
      const int ch = tid + t * 256, row = ch / (AROW / 16), cc = ch % (AROW / 16);
      const int m = m_blk + row;
      const uint32_t off = (uint32_t)g0 * 8 * A + cc * 16;
      const bool ok = ch < ACH && m < M && off < arow_bytes;
      buffer_slot<8>(ares, ok ? (uint32_t)m * arow_bytes + off : kOff, araw[t]);
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int t = 0; t < SPT; ++t) {
        const int e = tid + t * 256, row = e / KG, gl = e % KG;
        const int m = m_blk + row, g = g0 + gl;
        const bool ok = e < BM * KG && m < M && g < G;
        sraw[t] = buffer_f32(sres, ok ? ((uint32_t)m * G + g) * 4u : kOff);
      }
    }
  };

  auto store = [&](uint8_t* buf, const uint32_t (&wraw)[WPT][4], const uint32_t (&araw)[APT][4],
                   const float (&sraw)[SPT]) {
    uint8_t* wl = buf;
    uint8_t* al = buf + WBYTES;
    float* sl = reinterpret_cast<float*>(buf + WBYTES + ABYTES);
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int ch = tid + t * 256;
      if (ch >= WCH) break;
      const int row = ch / (WROW / 16), cc = ch % (WROW / 16);
      // a 16-byte chunk holds 8/W slots: elements [cc*128/W, +128/W) of the stage
      constexpr int SPC = 8 / W;
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const int slot_all = cc * SPC + q, gl = slot_all / 4, slot = slot_all % 4;
        uint32_t d[4];
        unpack_slot<W>(const_cast<uint32_t*>(&wraw[t][q * W / 2]), d);
        *reinterpret_cast<v4u*>(wl + slot_addr(gl, row, BN, slot)) = v4u{d[0], d[1], d[2], d[3]};
      }
    }
#pragma unroll
    for (int t = 0; t < APT; ++t) {
      const int ch = tid + t * 256;
      if (ch >= ACH) break;
      const int row = ch / (AROW / 16), cc = ch % (AROW / 16);
      constexpr int SPC = 8 / A;
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const int slot_all = cc * SPC + q, gl = slot_all / 4, slot = slot_all % 4;
        uint32_t d[4];
        unpack_slot<A>(const_cast<uint32_t*>(&araw[t][q * A / 2]), d);
        reorder_slot<A, W>(d);
        *reinterpret_cast<v4u*>(al + slot_addr(gl, row, BM, slot)) = v4u{d[0], d[1], d[2], d[3]};
      }
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int t = 0; t < SPT; ++t) {
        const int e = tid + t * 256;
        if (e < BM * KG) sl[(e % KG) * BM + e / KG] = sraw[t] * fold;
      }
    }
  };

  float acc[TN][TM][4], p[TN][TM][4];
#pragma unroll
  for (int x = 0; x < TN; ++x)
#pragma unroll
    for (int y = 0; y < TM; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[x][y][r] = p[x][y][r] = 0.f;

  const int stages = (G + KG - 1) / KG;
  int c = 0, cend = chunk_begin(1, G);
  // acc += p in chunk order (acc starts at +0 and p is never -0, so the first
  // add is exact and matches acc = p_0)
  auto close_chunk = [&]() {
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y)
#pragma unroll
        for (int r = 0; r < 4; ++r) { acc[x][y][r] = acc[x][y][r] + p[x][y][r]; p[x][y][r] = 0.f; }
    ++c;
    cend = chunk_begin(c + 1, G);
  };
  // Prologue: loads of stages 0 .. R-1 in flight, stage 0 unpacked to LDS.
#pragma unroll
  for (int u = 0; u < R; ++u)
    if (u < stages) fetch(u * KG, wraw_r[u], araw_r[u], sraw_r[u]);
  store(lds[0], wraw_r[0], araw_r[0], sraw_r[0]);
  __syncthreads();
  // Stage s: compute from lds[s & 1]; refill ring slot s % R with stage s+R;
  // unpack stage s+1 (ring slot (s+1) % R, fetched R-1 stages ago) into the
  // other LDS buffer.
  for (int s0 = 0; s0 < stages; s0 += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int s = s0 + u;
      if (s >= stages) break;
      if (s + R < stages) fetch((s + R) * KG, wraw_r[u], araw_r[u], sraw_r[u]);
      const uint8_t* buf = lds[s & 1];
      const uint8_t* wl = buf;
      const uint8_t* al = buf + WBYTES;
      const float* sl = reinterpret_cast<const float*>(buf + WBYTES + ABYTES);
      // fragments of group gl are read one group ahead; all TN x TM MFMAs of
      // a group are issued before its epilogue so their latency overlaps
      uint32_t wf[TN][4], af[TM][4];
      float sc[TM];
      auto read_frags = [&](int gl) {
#pragma unroll
        for (int x = 0; x < TN; ++x) {
          const v4u q = *reinterpret_cast<const v4u*>(wl + slot_addr(gl, wn + x * 16 + i, BN, kb));
          wf[x][0] = q[0]; wf[x][1] = q[1]; wf[x][2] = q[2]; wf[x][3] = q[3];
        }
#pragma unroll
        for (int y = 0; y < TM; ++y) {
          const v4u q = *reinterpret_cast<const v4u*>(al + slot_addr(gl, wm + y * 16 + i, BM, kb));
          af[y][0] = q[0]; af[y][1] = q[1]; af[y][2] = q[2]; af[y][3] = q[3];
          if constexpr (!DOTS) sc[y] = sl[gl * BM + wm + y * 16 + i];
        }
      };
      read_frags(0);
#pragma unroll
      for (int gl = 0; gl < KG; ++gl) {
        const int g = s * KG + gl;
        if (g >= G) break;
        if constexpr (!DOTS) {
          while (g >= cend) close_chunk();  // finished (possibly empty) chunks before group g
        }
        v4i D[TN][TM];
#pragma unroll
        for (int x = 0; x < TN; ++x)
#pragma unroll
          for (int y = 0; y < TM; ++y) D[x][y] = mfma16x16x64(wf[x], af[y], v4i{0, 0, 0, 0});
        float scg[TM];
#pragma unroll
        for (int y = 0; y < TM; ++y) scg[y] = sc[y];
        if (gl + 1 < KG) read_frags(gl + 1);
#pragma unroll
        for (int x = 0; x < TN; ++x)
#pragma unroll
          for (int y = 0; y < TM; ++y) {
            if constexpr (DOTS) {
              const int m = m_blk + wm + y * 16 + i;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int n = n_blk + wn + x * 16 + 4 * kb + r;
                if (n < N && m < M) args.dots[((long)m * N + n) * G + g] = D[x][y][r] >> T;
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) p[x][y][r] = __builtin_fmaf((float)D[x][y][r], scg[y], p[x][y][r]);
            }
          }
      }
      if (s + 1 < stages) store(lds[(s + 1) & 1], wraw_r[(u + 1) % R], araw_r[(u + 1) % R], sraw_r[(u + 1) % R]);
      __syncthreads();
    }
  }
  if constexpr (DOTS) return;
  while (c < kChunks) close_chunk();
#pragma unroll
  for (int x = 0; x < TN; ++x)
#pragma unroll
    for (int y = 0; y < TM; ++y) {
      const int m = m_blk + wm + y * 16 + i;
      if (m >= M) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n_blk + wn + x * 16 + 4 * kb + r;
        if (n >= N) continue;
        const float v = finish(acc[x][y][r], args.prob[0].ws[n], args.prob[0].bias, args.bias_dt, n);
        const long o = (long)m * N + n;
        if (args.out_dt == kBF16) store_out<kBF16>(args.prob[0].out, o, v);
        else if (args.out_dt == kF16) store_out<kF16>(args.prob[0].out, o, v);
        else store_out<kF32>(args.prob[0].out, o, v);
      }
    }
}

// Shapes (TN, TM): 0 = (2,2) 64x64, 1 = (4,2) 128x64, 2 = (2,4) 64x128,
// 3 = (4,4) 128x128; single problem.
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
