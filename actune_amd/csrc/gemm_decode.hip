// Decode packed group-64 GEMM for gfx950, single-width launches: the
// kernel body and its structure are in decode_body.hpp; this file holds the
// host-side sizing (LDS, row tiles per workgroup, fit) and the launches.
#include "decode_body.hpp"

namespace actune {

// Dynamic LDS: per wave a slab [GW groups][M tokens][64 B] and a scale slab
// [GW][MT] (fp32, 2^-(sW+sA) folded in; entries of absent tokens unused), the
// zero region, and the chunk partials red[16][16 * tr][MT] (cmp:
// red[chunk_slots(G)][16 * tr][MT]).
size_t decode_lds_bytes(int K, int M, int nw, int tr, bool cmp) {
  M = M > 16 ? 16 : M;  // tokens of one 16-token block
  const int gw = decode_groups_per_wave(K, nw), MT = decode_token_tile(M);
  const int slots = cmp ? chunk_slots(K / kGroup) : kChunks;
  return (size_t)nw * gw * (M * kGroup + MT * sizeof(float)) + kDecodeZeroBytes +
         sizeof(float) * slots * 16 * tr * MT;
}

// At least this many workgroups when several row tiles share one (measured
// on MI355X, W4A8 M=8: 256 row tiles run best one per workgroup, 688-1376
// with four).
constexpr int kDecodeMinGroups = 160;
constexpr size_t kCuLds = 160 * 1024;  // LDS of one gfx950 CU

// Row tiles per workgroup for M > 1: the most (up to 4) whose weight slots
// still fit the ring, keeping at least kDecodeMinGroups workgroups over the
// nprob problems of `tiles` row tiles each. With 16-token tiles, four row
// tiles' chunk partials (64 KiB) can leave room for one workgroup per CU;
// where two row tiles still fit two workgroups per CU and their grid fills
// two per CU, two are taken (measured on MI355X, W4A4 gate/up 2 x 4096 x 1024
// at M = 50, four waves: 13.2 -> 10.6 us; at M = 24, 11008 x 4096, where two
// tiles also leave one workgroup per CU, four stay faster: 19.1 against
// 28.2 us for one).
int decode_row_tiles(int K, int M, int W, int nw, int tiles, int nprob, bool compact) {
  if (M < 2) return 1;
  const int slots = (decode_groups_per_wave(K, nw) + 8 / W - 1) / (8 / W);
  int tr = 1;
  for (int c = 2; c <= 4; c *= 2)
    if (slots * c <= decode_ring(W) && (tiles + c - 1) / c * nprob >= kDecodeMinGroups &&
        decode_lds_bytes(K, M, nw, c) <= kStreamLdsMax)
      tr = c;
  if (tr == 4 && M > 8 && compact && nw == 4 && chunk_slots(K / kGroup) < kChunks) {
    // a launch that can take compact partials (decode_compact) keeps four
    // tiles, x quantized once per four, while that grid still gives every
    // CU two workgroups (W4A4 2 x 4096 x 1024 at M = 50: 10.8 -> 10.2 us;
    // 16384 x 2048 at M = 24: 15.0 -> 12.3 us; with half that grid, 8192 x
    // 1024 at M = 17, four tiles were 12% slower than two)
    if ((tiles + 3) / 4 * nprob < 2 * 256 && (tiles + 1) / 2 * nprob >= 2 * 256) tr = 2;
  } else if (tr == 4 && M > 8 && 2 * decode_lds_bytes(K, M, nw, 4) > kCuLds &&
             2 * decode_lds_bytes(K, M, nw, 2) <= kCuLds && (tiles + 1) / 2 * nprob >= 2 * 256) {
    tr = 2;
  }
  return tr;
}

// Workgroups of a decode launch resident at once: the CU's LDS and 16 waves
// per CU (the M > 1 decode kernels take 100-128 VGPRs, four waves per SIMD),
// over 256 CUs.
long decode_resident(int nw, size_t lds) {
  return 256L * std::min<long>(16 / nw, (long)(kCuLds / lds));
}

// Compact chunk partials for a 4-wave launch of 16-token blocks with two or
// four row tiles per workgroup, below kChunks quads: taken where the grid
// needs more than one round of resident workgroups and the smaller LDS lets
// more of them be resident (W4A4 2 x 4096 x 1024 at M = 50, two tiles:
// 50 -> 26 KB, three to four workgroups per CU for 1024 workgroups).
bool decode_compact(int K, int M, int nw, int tr, long groups) {
  if (nw != 4 || tr < 2 || M <= 8 || chunk_slots(K / kGroup) >= kChunks) return false;
  const long full = decode_resident(nw, decode_lds_bytes(K, M, nw, tr)),
             cmp = decode_resident(nw, decode_lds_bytes(K, M, nw, tr, true));
  return groups > full && cmp > full;
}

bool decode_fits(int K, int M, int W, int nw, bool packed, int x_dt) {
  if (!packed && x_dt != kBF16) return false;  // fused mode: bf16 x
  if (M < 1 || M > kDecodeMaxM || (nw != 4 && nw != 8 && nw != 16)) return false;
  const int gw = decode_groups_per_wave(K, nw), gps = 8 / W;
  if ((gw + gps - 1) / gps > decode_ring(W)) return false;
  const int per = packed ? 16 : 8, mb = M > 16 ? 16 : M;  // tokens of one 16-token block
  // group-row indices gl * M + m are divided by M through LinearArgs::m_div,
  // which is exact below kDecodeMaxGroupRows
  if (gw * mb > kDecodeMaxGroupRows) return false;
  if ((gw * mb + per - 1) / per > decode_passes(decode_token_tile(M), packed)) return false;
  return decode_lds_bytes(K, M, nw, 1) <= kStreamLdsMax;
}

// ---------------------------------------------------------------------------
template <int W, int A, int NW, int RING, int MT, bool PACKED, bool SCALE, bool ONE, bool FULL, int TR, bool CMP>
__global__ __launch_bounds__(NW * 64) void gemm_decode(const LinearArgs args, int GW) {
  extern __shared__ __align__(16) uint8_t smem[];
  decode_tile<W, A, NW, RING, MT, PACKED, SCALE, ONE, FULL, TR, CMP>(args, GW, smem);
}

template <int W, int A, int NW, int MT, bool PACKED, bool SCALE, bool ONE, bool FULL, int TR = 1, bool CMP = false>
static void launch_decode_one(const LinearArgs& g, hipStream_t st) {
  constexpr int RING = decode_ring(W) / TR;
  const size_t lds = decode_lds_bytes(g.K, g.M, NW, TR, CMP);
  auto kern = gemm_decode<W, A, NW, RING, MT, PACKED, SCALE, ONE, FULL, TR, CMP>;
  allow_dynamic_lds<gemm_decode<W, A, NW, RING, MT, PACKED, SCALE, ONE, FULL, TR, CMP>>();
  const int groups = (decode_max_tiles(g) + TR - 1) / TR, blocks = MT == 16 ? (g.M + 15) / 16 : 1;
  kern<<<dim3((unsigned)groups, (unsigned)g.nprob, (unsigned)blocks), NW * 64, lds, st>>>(g, decode_groups_per_wave(g.K, NW));
}

// M > 1: TR row tiles per workgroup (decode_row_tiles), compact partials
// where decode_compact takes them (4 waves, 16-token blocks)
template <int W, int A, int NW, int MT, bool PACKED, bool SCALE>
static void launch_decode_tr(const LinearArgs& g, hipStream_t st) {
  const int blocks = MT == 16 ? (g.M + 15) / 16 : 1;
  const int tr = decode_row_tiles(g.K, g.M, W, NW, decode_max_tiles(g), g.nprob * blocks);
  const bool full = decode_full(g.K, W, NW, tr);
#define DEC_TR(TRV, CMPV)                                                                      \
  if (full) launch_decode_one<W, A, NW, MT, PACKED, SCALE, false, true, TRV, CMPV>(g, st);     \
  else launch_decode_one<W, A, NW, MT, PACKED, SCALE, false, false, TRV, CMPV>(g, st)
  if constexpr (MT == 16 && NW == 4) {
    const long groups = (long)((decode_max_tiles(g) + tr - 1) / tr) * g.nprob * blocks;
    if (tr >= 2 && decode_compact(g.K, g.M, NW, tr, groups)) {
      if (tr == 4) { DEC_TR(4, true); }
      else { DEC_TR(2, true); }
      return;
    }
  }
  if (tr == 4) { DEC_TR(4, false); }
  else if (tr == 2) { DEC_TR(2, false); }
  else { DEC_TR(1, false); }
#undef DEC_TR
}

template <int W, int A, int NW>
static void launch_decode_nw(bool packed, const LinearArgs& g, hipStream_t st) {
  const bool full = decode_full(g.K, W, NW), scale = g.xscale != nullptr;
  if (packed) {
    if (g.M == 1) launch_decode_one<W, A, NW, 4, true, false, true, false>(g, st);
    else if (g.M <= 4) launch_decode_tr<W, A, NW, 4, true, false>(g, st);
    else if (g.M <= 8) launch_decode_tr<W, A, NW, 8, true, false>(g, st);
    else launch_decode_tr<W, A, NW, 16, true, false>(g, st);
    return;
  }
#define DEC_FULL(MTV, SC, ONEV)                                                 \
  if (full) launch_decode_one<W, A, NW, MTV, false, SC, ONEV, true>(g, st);     \
  else launch_decode_one<W, A, NW, MTV, false, SC, ONEV, false>(g, st)
  if (g.M == 1) {
    if (scale) { DEC_FULL(4, true, true); }
    else { DEC_FULL(4, false, true); }
  } else if (g.M <= 4) {
    if (scale) launch_decode_tr<W, A, NW, 4, false, true>(g, st);
    else launch_decode_tr<W, A, NW, 4, false, false>(g, st);
  } else if (g.M <= 8) {
    if (scale) launch_decode_tr<W, A, NW, 8, false, true>(g, st);
    else launch_decode_tr<W, A, NW, 8, false, false>(g, st);
  } else {
    if (scale) launch_decode_tr<W, A, NW, 16, false, true>(g, st);
    else launch_decode_tr<W, A, NW, 16, false, false>(g, st);
  }
#undef DEC_FULL
}

template <int W, int A>
static void launch_decode_wa(int nw, bool packed, const LinearArgs& g, hipStream_t st) {
  if (nw == 4) launch_decode_nw<W, A, 4>(packed, g, st);
  else if (nw == 8) launch_decode_nw<W, A, 8>(packed, g, st);
  else launch_decode_nw<W, A, 16>(packed, g, st);
}

void launch_decode(int W, int A, int nw, bool packed, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB) if (W == WB && A == AB) return launch_decode_wa<WB, AB>(nw, packed, g, st)
  CASE(8, 8); CASE(8, 4); CASE(8, 2);
  CASE(4, 8); CASE(4, 4); CASE(4, 2);
  CASE(2, 8); CASE(2, 4); CASE(2, 2);
#undef CASE
}

}  // namespace actune
