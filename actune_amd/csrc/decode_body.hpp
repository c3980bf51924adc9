// Body of the decode packed group-64 GEMM (one workgroup's tiles), shared by
// the single-width kernels (gemm_decode.hip) and the mixed-width kernel
// (gemm_decode_mixed.hip), with the host-side sizing helpers both use.
//
// Decode packed group-64 GEMM for gfx950 (M <= 1024 tokens in 16-token
// blocks; the default up to 64 and for narrow problems): the launch is bound
// by the HBM read of the packed weights, so the kernel is shaped to start
// that read early and keep all of it in flight.
//
// Restates the per-call math of actune/kernels/grouped.py:55-94 (group-64
// quantizer, exact int32 dot per group, fp32 rescale, weight-scale epilogue;
// the optional channel scale of layers.py:41-42 is divided in first), in the
// canonical chunked order of common.hpp.
//
// Structure:
//  * A workgroup is NW waves and owns TR (1, 2 or 4; 1 at M = 1) consecutive
//    16-row tiles of one problem (up to kMaxProblems linears that read the
//    same activations share a launch; the problem is blockIdx.y, so each
//    workgroup reads only its own problem's kernel arguments, in one batch of
//    scalar loads before its first memory load). The waves split K along the
//    16 canonical chunks; the tiles share the activation slab.
//  * Each wave issues all its loads at entry: its activation passes, then its
//    whole K-range of weights as RING 16-byte loads per lane at constant
//    offsets (lanes of a row fetch 64 consecutive bytes; passes and slots
//    past the wave's range are switched off and read zeros without memory
//    traffic). Straight-line loads let every use wait for exactly its own
//    load (in-order memory counter). It then fills a wave-private LDS slab
//    with its K-range of the activations as MFMA operand rows while the
//    weights arrive: bf16 x is quantized in place (fused), packed codes from
//    the quantizer launch are unpacked (packed).
//  * The wave walks its slots in a software pipeline: slot s+1's
//    v_permlane32/16_swap exchange, register unpack and MFMAs are issued
//    before slot s's results are rescaled. The tokens are the MFMA A operand
//    (token m of weight row c lands in lane 16*(m/4) + c, register m%4); one
//    fp32 FMA per (row, token, group) rescales the exact int32 dot.
//  * Chunk partials meet in LDS [16 chunks][16 * TR rows][MT tokens] (CMP:
//    one slot per chunk that holds groups) and are added in chunk order after
//    one barrier (wave t finishes tile t).
#pragma once
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

constexpr int kDecodeMaxM = 1024;  // 16-token blocks on grid z
// zero region: a wave's widest K-range (16 groups) of 64-byte zero rows
constexpr int kDecodeZeroBytes = 16 * kGroup;

// 16-byte weight loads per lane: 16 groups of W2 / W4, 8 groups of W8
__host__ __device__ constexpr int decode_ring(int W) { return W == 2 ? 4 : 8; }
// token tile: tokens 4j..4j+3 land in lanes 16j..16j+15
inline int decode_token_tile(int M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }
// activation passes a wave issues up front: fused passes quantize 8
// group-rows, packed passes unpack 16
__host__ __device__ constexpr int decode_passes(int MT, bool packed) {
  return packed ? (MT < 8 ? MT : 8) : (MT == 4 ? 4 : 8);
}

// Largest groups per wave of a K split over nw waves.
inline int decode_groups_per_wave(int K, int nw) {
  const int G = K / kGroup, cpw = kChunks / nw;
  int gw = 1;
  for (int w = 0; w < nw; ++w) {
    const int d = chunk_begin((w + 1) * cpw, G) - chunk_begin(w * cpw, G);
    gw = d > gw ? d : gw;
  }
  return gw;
}

// true when every one of nw waves gets exactly a full ring of weight slots
// (decode_ring(W) / tr slots per row tile)
inline bool decode_full(int K, int W, int nw, int tr = 1) {
  const int G = K / kGroup, cpw = kChunks / nw, per = decode_ring(W) / tr * (8 / W);
  for (int w = 0; w < nw; ++w)
    if (chunk_begin((w + 1) * cpw, G) - chunk_begin(w * cpw, G) != per) return false;
  return true;
}

// chunk_begin in unsigned arithmetic (c, G >= 0): shifts instead of the
// signed-division sequences, for the slot loop's scalar chunk tracking
__device__ __forceinline__ int chunk_begin_u(int c, int G) {
  const uint32_t Q = ((uint32_t)G + 3u) >> 2;
  const uint32_t b = (((uint32_t)c * Q) >> 4) << 2;
  return b < (uint32_t)G ? (int)b : G;
}

// MT: token tile (4, 8 or 16). PACKED: activations come as packed codes +
// scales (args.a, args.as); otherwise bf16 x (and the bf16 channel scale
// when SCALE) is quantized here. ONE: M == 1 (only register 0 of a lane's
// MFMA result can be nonzero); its launches read token operands at constant
// LDS offsets and keep the group scales in scalar registers. FULL: every
// wave's K-range is exactly RING slots (decode_full), so the slot pipeline
// runs without bounds tests (and a fused ONE launch issues exactly the x
// passes of the range). TR: 16-row tiles per workgroup (M > 1): the tiles share
// the workgroup's activation slab, so x is read and quantized once per TR
// tiles; RING is then the weight slots per tile. CMP (K below kChunks quads,
// M > 1): the chunk partials keep one slot per nonempty chunk (chunk_slots),
// which shrinks the workgroup's LDS where it limits how many are resident.
template <int W, int A, int NW, int RING, int MT, bool PACKED, bool SCALE, bool ONE, bool FULL, int TR,
          bool CMP = false>
__device__ __forceinline__ void decode_tile(const LinearArgs& args, int GW, uint8_t* smem) {
  static_assert(!CMP || !ONE, "compact partials are for the M > 1 slot loop");
  constexpr int GS = 8 / W;                // groups per 16-byte weight load per lane
  constexpr int CPW = kChunks / NW;        // canonical chunks per wave
  constexpr int T = shift_of(W) + shift_of(A);
  constexpr int DT = kBF16;
  constexpr int ESZ = 2;
  constexpr bool FAST = ONE;
  constexpr int PR = PACKED ? 16 : 8;      // group-rows per activation pass
  constexpr int NPX = FULL && ONE && !PACKED ? (RING * GS + 7) / 8 : decode_passes(MT, PACKED);
  static_assert(MT == 4 || MT == 8 || MT == 16, "token tiles of 4, 8 or 16");
  static_assert(!ONE || MT == 4, "M == 1 uses the 4-token tile");
  static_assert(!ONE || TR == 1, "M == 1 launches own one row tile per workgroup");
  static_assert(TR <= NW, "waves 0..TR-1 finish one tile each");

  const float fold = __builtin_ldexpf(1.0f, -T);
  // Every kernel argument the prologue needs is read here, in one batch of
  // scalar loads with one wait: the empty asm takes the values as operands
  // it may change, so none of them is reloaded later (a reload would put a
  // scalar round trip between entry and the first weight load).
  // The problem is blockIdx.y: its fields sit at an offset known at entry.
  Problem pr = args.prob[blockIdx.y];
  int M = args.M, K = args.K, bias_dt = args.bias_dt, out_dt = args.out_dt;
  uint32_t m_inv = args.m_div;  // r / M == (r * m_inv) >> 16 for the row indices here
  const void* xsrc = PACKED ? static_cast<const void*>(args.a) : args.x;
  const void* xaux = PACKED ? static_cast<const void*>(args.as) : args.xscale;
  asm volatile("" : "+s"(M), "+s"(K), "+s"(bias_dt), "+s"(out_dt), "+s"(m_inv), "+s"(xsrc), "+s"(xaux), "+s"(GW),
                    "+s"(pr.w), "+s"(pr.ws), "+s"(pr.bias), "+s"(pr.out), "+s"(pr.N));
  const int N = pr.N, G = K / kGroup;
  if constexpr (MT == 16) {
    // 16-token block blockIdx.z: its tokens, x rows or codes and scales, and
    // output rows (the channel scale of the fused mode is per column)
    const int m0 = 16 * (int)blockIdx.z;
    const bool last = m0 + 16 >= M;
    m_inv = last ? args.m_div_tail : 4096u;
    M = last ? M - m0 : 16;
    if constexpr (PACKED) {
      xsrc = static_cast<const uint8_t*>(xsrc) + (size_t)m0 * (K / 8) * A;
      xaux = static_cast<const float*>(xaux) + (size_t)m0 * G;
    } else {
      xsrc = static_cast<const uint8_t*>(xsrc) + (size_t)m0 * K * ESZ;
    }
    pr.out = static_cast<uint8_t*>(pr.out) + (size_t)m0 * N * (out_dt == kF32 ? 4 : 2);
  }
  const int n0 = (int)blockIdx.x * 16 * TR;
  // blockIdx.x spans the widest problem of the launch; a narrower one's
  // workgroups past its rows leave at once (whole workgroup, before any
  // barrier)
  if (n0 >= N) return;
  // wave is read into a scalar register so that every K-range bound below is
  // wave-uniform: the step loop then branches on scalars and the memory
  // counter waits stay per slot.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int c_first = wave * CPW;
  const int wg0 = chunk_begin(c_first, G), wg1 = chunk_begin(c_first + CPW, G);
  const int ng = wg1 - wg0;                 // groups of this wave
  const int ns = (ng + GS - 1) / GS;        // weight steps of this wave
  // A FULL launch holds G = NW * RING * GS groups (every wave a full ring).
  // When G is a multiple of 4 * kChunks every chunk has GPC = G / kChunks
  // groups, so the slot loop closes chunk c_first + j after slot
  // (j + 1) * GPC / GS - 1 with no scalar chunk tracking.
  constexpr int GF = NW * RING * GS;
  constexpr bool SC = FULL && GF % (4 * kChunks) == 0;
  constexpr int GPC = SC ? GF / kChunks : 4;

  uint8_t* slab = smem + (size_t)wave * GW * M * kGroup;
  float* sslab = reinterpret_cast<float*>(smem + (size_t)NW * GW * M * kGroup) + (size_t)wave * GW * MT;
  uint8_t* zero_row = reinterpret_cast<uint8_t*>(reinterpret_cast<float*>(smem + (size_t)NW * GW * M * kGroup) +
                                                 (size_t)NW * GW * MT);
  float* red = reinterpret_cast<float*>(zero_row + kDecodeZeroBytes);  // [chunk][row][MT]

  // Wave 0 finishes output row lane / 4 for tokens lane % 4 + 4j.
  const int e_row = lane >> 2, e_m = lane & 3;

  // ---------------------------------------------------------------- activation loads
  // Group-row r = gl * M + m (gl: group of the wave's range, m: token).
  const int rows_here = ng * M;
  const int npass = (rows_here + PR - 1) / PR;
  struct Raw { v4u x, s; uint32_t q[4]; float sc; };
  // fused: a pass covers 8 group-rows, 8 lanes each, 8 consecutive elements
  // per lane
  const Rsrc xres = make_rsrc(xsrc, PACKED ? (uint32_t)M * K * A / 8 : (uint32_t)M * K * ESZ);
  const Rsrc xsres = make_rsrc(PACKED || SCALE ? xaux : xsrc, PACKED ? (uint32_t)(M * G) * 4u : (uint32_t)K * ESZ);
  const int seg = lane & 7;
  // M == 1: lane l of pass p reads elements wg0*64 + p*512 + 8l.. of x (the
  // rows past the wave's range read neighbouring elements or zeros and are
  // not stored); the pass is a constant offset, passes past npass are
  // switched off through the scalar offset.
  const uint32_t xbase1 = ((uint32_t)wg0 * kGroup + (uint32_t)lane * 8) * ESZ;
  // packed: a pass covers 16 group-rows; lane (row lane / 4, k-slot lane % 4)
  constexpr int CB = 16 * A / 8;            // bytes of one 16-code slot
  const uint32_t arow_bytes = (uint32_t)K * A / 8;
  auto row_of = [&](int r, int& gl, int& m) {
    gl = ONE ? r : (int)(((uint32_t)r * m_inv) >> 16);
    m = ONE ? 0 : r - gl * M;
  };
  auto issue_x = [&](int pass, Raw& raw) {
    if constexpr (PACKED) {
      const int r = pass * 16 + (lane >> 2), j = lane & 3;
      const bool live = r < rows_here;
      int gl, m;
      row_of(live ? r : 0, gl, m);
      buffer_slot<A>(xres, live ? (uint32_t)m * arow_bytes + (uint32_t)((wg0 + gl) * 4 + j) * CB : kOff, raw.q);
      raw.sc = buffer_f32(xsres, live && j == 0 ? ((uint32_t)m * G + wg0 + gl) * 4u : kOff);
    } else if constexpr (ONE) {
      const uint32_t soff = pass < npass ? 0u : kOff;
      raw.x = __builtin_amdgcn_raw_buffer_load_b128(xres, xbase1 + (uint32_t)(pass * 512 * ESZ), soff, 0);
      if constexpr (SCALE) raw.s = __builtin_amdgcn_raw_buffer_load_b128(xsres, xbase1 + (uint32_t)(pass * 512 * ESZ), soff, 0);
    } else {
      const int r = pass * 8 + (lane >> 3);
      const bool live = r < rows_here;
      int gl, m;
      row_of(live ? r : 0, gl, m);
      const uint32_t k0 = (uint32_t)((wg0 + gl) * kGroup + seg * 8);
      raw.x = __builtin_amdgcn_raw_buffer_load_b128(xres, live ? ((uint32_t)m * K + k0) * ESZ : kOff, 0, 0);
      if constexpr (SCALE) raw.s = __builtin_amdgcn_raw_buffer_load_b128(xsres, live ? k0 * ESZ : kOff, 0, 0);
    }
  };
  // Slab row r gets its operand slots; returns the group scale s * 2^-T (the
  // same in the lanes of a group-row).
  auto convert_x = [&](int pass, const Raw& raw) -> float {
    if constexpr (PACKED) {
      const int r = pass * 16 + (lane >> 2), j = lane & 3;
      const float sf = raw.sc * fold;
      if (r < rows_here) {
        int gl, m;
        row_of(r, gl, m);
        uint32_t d[4];
        unpack_slot<A>(raw.q, d);
        reorder_slot<A, W>(d);
        *reinterpret_cast<v4u*>(slab + (size_t)r * kGroup + 16 * j) = v4u{d[0], d[1], d[2], d[3]};
        if (!FAST && j == 0) sslab[gl * MT + m] = sf;
      }
      return sf;
    } else {
      const int r = pass * 8 + (lane >> 3);
      const bool live = r < rows_here;
      float v[8];
      unpack8<DT>(raw.x, raw.x, v);
      if constexpr (SCALE) {
        float d[8];
        unpack8<DT>(raw.s, raw.s, d);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = live ? round_to_dtype<DT>(v[e] / d[e]) : 0.0f;
      }
      // every lane joins the group max, live or not
      uint32_t cq[8];
      const float s = group_code_bits<A, DT>(v, cq);
      if (live) {
        int gl, m;
        row_of(r, gl, m);
        store_half_slot<W, A>(slab + (size_t)r * kGroup + (seg >> 1) * 16, seg & 1, cq);
        if (!FAST && seg == 0) sslab[gl * MT + m] = s * fold;
      }
      return s * fold;
    }
  };
  Raw early[NPX];
#pragma unroll
  for (int p = 0; p < NPX; ++p) issue_x(p, early[p]);

  // ---------------------------------------------------------------- weight loads
  const uint32_t wrow_bytes = (uint32_t)K * W / 8;
  const Rsrc wres = make_rsrc(pr.w, (uint32_t)N * wrow_bytes);
  // Slot st of the wave is 64 bytes past slot st-1: a constant offset. Rows
  // past N lie past the buffer's range and read zeros; slots past the wave's
  // range are switched off through the scalar offset (the vector offset
  // stays below 2^31, so the sum cannot wrap).
  const uint32_t wbase = (uint32_t)(n0 + i) * wrow_bytes + kb * 16 + (uint32_t)wg0 * 8 * W;
  // the host guarantees ns <= RING and npass <= NPX (decode_fits)
  uint32_t ring[TR][RING][4];
#pragma unroll
  for (int t = 0; t < TR; ++t)
#pragma unroll
  for (int st = 0; st < RING; ++st) {
    // (a runtime test also where every slot is live: with a constant offset
    // the compiler schedules the loads differently and the launch measured
    // 0.4 us slower at one workgroup per CU)
    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(wres, wbase + (uint32_t)(16 * t) * wrow_bytes + (uint32_t)st * 64,
                                                        st < ns ? 0u : kOff, 0);
    ring[t][st][0] = q[0]; ring[t][st][1] = q[1]; ring[t][st][2] = q[2]; ring[t][st][3] = q[3];
  }
  // epilogue constants, behind the weights: they are needed last, by wave 0.
  // Every wave issues the two loads (switched off outside wave 0) so that all
  // waves have the same loads in flight: behind a branch, the compiler's
  // waits for the activation passes would count from the shorter path and
  // make wave 0 wait for weight slots before quantizing.
  const ChannelConst cc = fetch_channel(pr.ws, pr.bias, bias_dt, N, n0 + 16 * (wave % TR) + e_row, wave / TR < MT / 4);

  // ---------------------------------------------------------------- activation slab
  // the zero region: one dword per thread of the first four waves
  if (threadIdx.x < kDecodeZeroBytes / 4) reinterpret_cast<uint32_t*>(zero_row)[threadIdx.x] = 0u;
  // FAST: the wave's group scales (s * 2^-T, wave-uniform) move from the
  // lanes that computed or loaded them into scalar registers
  float gsc[FAST ? RING * GS : 1];
#pragma unroll
  for (int p = 0; p < NPX; ++p) {
    if ((FULL && ONE && !PACKED) || p < npass) {
      const float sf = convert_x(p, early[p]);
      if constexpr (FAST) {
        // a group past the wave's range (the tail of its last slot, whose
        // weights are the next row's bytes and whose slab row is unwritten
        // LDS) gets scale 0 and adds fma(d, 0, p) = p exactly; a FULL
        // launch has none (every wave holds RING * GS groups)
#pragma unroll
        for (int j = 0; j < PR; ++j)
          if (p * PR + j < RING * GS)
            gsc[p * PR + j] = FULL || p * PR + j < ng
                                  ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sf), (64 / PR) * j))
                                  : 0.0f;
      }
    }
  }
  // the zero region and the slabs are written across waves
  __syncthreads();

  // ---------------------------------------------------------------- stream the K-range
  float p[TR][4];
#pragma unroll
  for (int t = 0; t < TR; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) p[t][q] = 0.f;
  int c = c_first;
  // partials: lane l holds rows l % 16 of tokens 4*(l/16)..+3 of each tile;
  // the lanes of the token tile write them to red[chunk][tile row][token]
  constexpr int RS = 16 * TR * MT;  // floats per chunk of red
  const bool writer = lane < 16 * (MT / 4);
  float* red_lane = red + (size_t)(lane & 15) * MT + 4 * ((lane >> 4) & (MT / 4 - 1));
  auto write_partials = [&](int cc_) {
    // CMP: the chunk's quad is its slot; a chunk without groups stores
    // nothing (its partial is +0)
    int sl = cc_;
    if constexpr (CMP) {
      const int b0 = chunk_begin_u(cc_, G), b1 = chunk_begin_u(cc_ + 1, G);
      sl = b1 > b0 ? b0 >> 2 : -1;
    }
#pragma unroll
    for (int t = 0; t < TR; ++t) {
      if (writer && (!CMP || sl >= 0))
        *reinterpret_cast<v4f*>(red_lane + (size_t)sl * RS + 16 * t * MT) = v4f{p[t][0], p[t][1], p[t][2], p[t][3]};
#pragma unroll
      for (int q = 0; q < 4; ++q) p[t][q] = 0.f;
    }
  };
  if constexpr (FAST) {
    // M == 1: lanes of token 0 (i == 0) read the wave's slab, the others the
    // zero region, both with stride 64 per group, so every token operand
    // read is one LDS load at a constant offset (reads past the wave's range
    // stay inside LDS; their groups have scale 0); the rescale takes its
    // scale from a scalar register. Same pipeline and order as the general
    // loop below.
    constexpr int RA = 3;
    const uint8_t* tbase = (i == 0 ? slab : zero_row) + smallm_slot_k<W>(kb);
    v4u bq[RING][GS];
    v4i D[RING][GS];
    auto read_q = [&](int st) {
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) bq[st][jj] = *reinterpret_cast<const v4u*>(tbase + (st * GS + jj) * kGroup);
    };
#pragma unroll
    for (int st = 0; st < RA && st < RING; ++st) read_q(st);
    auto mfma_slot = [&](int st) {
      exchange<W>(ring[0][st]);
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        uint32_t wd[4];
        unpack_slot<W>(&ring[0][st][jj * W / 2], wd);
        const uint32_t bd[4] = {bq[st][jj][0], bq[st][jj][1], bq[st][jj][2], bq[st][jj][3]};
        D[st][jj] = mfma16x16x64(bd, wd, v4i{0, 0, 0, 0});
      }
    };
    int cend = chunk_begin_u(c + 1, G);
    const int c_last = c_first + CPW - 1;
    mfma_slot(0);
#pragma unroll
    for (int st = 0; st < RING; ++st) {
      if constexpr (!FULL) {
        if (st >= ns) break;
      }
      if (st + 1 < RING && (FULL || st + 1 < ns)) {
        if (st + RA < RING) read_q(st + RA);
        mfma_slot(st + 1);
      }
      if constexpr (SC) {
        if (st > 0 && (st * GS) % GPC == 0) {  // the chunk ending before this slot
          if (lane < 16)
            *reinterpret_cast<v4f*>(red_lane + (size_t)(c_first + st * GS / GPC - 1) * RS) = v4f{p[0][0], 0.f, 0.f, 0.f};
          p[0][0] = 0.f;
        }
      } else {
        const int g0 = wg0 + st * GS;
        while (g0 >= cend && c < c_last) {  // close finished (possibly empty) chunks
          if (lane < 16) *reinterpret_cast<v4f*>(red_lane + (size_t)c * RS) = v4f{p[0][0], 0.f, 0.f, 0.f};
          p[0][0] = 0.f;
          ++c;
          cend = chunk_begin_u(c + 1, G);
        }
      }
      if constexpr (GS == 1) {  // see the general loop
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 1");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) p[0][0] = __builtin_fmaf((float)D[st][jj][0], gsc[st * GS + jj], p[0][0]);
    }
  } else {
    // The GS MFMAs of a slot are issued together (for every tile) and folded
    // in group order.
    const int slot_k = smallm_slot_k<W>(kb);
    // Lanes of absent tokens (i >= M) read the zero row with stride 0. A group
    // past the wave's range (the tail of its last slot, or a slot read ahead
    // and never used) reads a clamped slab row and a zero scale, so it adds
    // exactly nothing. Lane l rescales tokens 4*(l/16) + q; lanes past the
    // token tile read the first tokens' scales against zero MFMA rows.
    const bool tok = i < M;
    const uint8_t* bbase = tok ? slab + i * kGroup + slot_k : zero_row;
    const uint32_t bstride = tok ? (uint32_t)M * kGroup : 0u;
    const float* sbase = sslab + 4 * ((lane >> 4) & (MT / 4 - 1));
    auto read_b = [&](int st, v4u (&bq)[GS], v4f (&bs)[GS]) {
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        const int gl = max(0, min(st * GS + jj, ng - 1));
        bq[jj] = *reinterpret_cast<const v4u*>(bbase + __umul24((uint32_t)gl, bstride));
        const float* srow = st * GS + jj < ng ? sbase + gl * MT : reinterpret_cast<const float*>(zero_row);
        bs[jj] = *reinterpret_cast<const v4f*>(srow);
      }
    };
    // Software pipeline over the wave's ns slots: slot st+1's MFMAs are issued
    // before slot st's results are rescaled, so MFMA latency hides under that
    // work. Token operands are read three slots ahead (one for W2 at 16
    // waves, whose 4-group slots would not fit 128 registers three deep).
    // (Slot 0's MFMAs run even when the wave has no slot: its weights and
    // scales are zero.)
    constexpr int RA = GS == 4 && NW == 16 ? 1 : 3;
    v4u bq[RING][GS];
    v4f bs[RING][GS];
    v4i D[TR][RING][GS];
#pragma unroll
    for (int st = 0; st < RA && st < RING; ++st) read_b(st, bq[st], bs[st]);
    auto mfma_slot = [&](int st) {
#pragma unroll
      for (int t = 0; t < TR; ++t) {
        exchange<W>(ring[t][st]);
#pragma unroll
        for (int jj = 0; jj < GS; ++jj) {
          uint32_t wd[4];
          unpack_slot<W>(&ring[t][st][jj * W / 2], wd);
          const uint32_t bd[4] = {bq[st][jj][0], bq[st][jj][1], bq[st][jj][2], bq[st][jj][3]};
          D[t][st][jj] = mfma16x16x64(bd, wd, v4i{0, 0, 0, 0});
        }
      }
    };
    int cend = chunk_begin(c + 1, G);
    const int c_last = c_first + CPW - 1;
    mfma_slot(0);
#pragma unroll
    for (int st = 0; st < RING; ++st) {
      if constexpr (!FULL) {
        if (st >= ns) break;
      }
      if (st + 1 < RING && (FULL || st + 1 < ns)) {
        if (st + RA < RING) read_b(st + RA, bq[st + RA], bs[st + RA]);
        mfma_slot(st + 1);
      }
      // Chunk boundaries are multiples of 4 groups and a slot's GS groups
      // start at a multiple of GS, so chunks close only at slot starts.
      if constexpr (SC) {
        if (st > 0 && (st * GS) % GPC == 0) write_partials(c_first + st * GS / GPC - 1);
      } else {
        const int g0 = wg0 + st * GS;
        while (g0 >= cend && c < c_last) {  // close finished (possibly empty) chunks
          write_partials(c);
          ++c;
          cend = chunk_begin(c + 1, G);
        }
      }
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        // registers of absent tokens hold zeros (their scale entries are
        // unset and their partials never read)
        const v4f sc = bs[st][jj];
#pragma unroll
        for (int t = 0; t < TR; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) p[t][q] = __builtin_fmaf((float)D[t][st][jj][q], sc[q], p[t][q]);
      }
    }
  }
  if constexpr (SC) write_partials(c_first + CPW - 1);  // the wave's last chunk
  else for (; c < c_first + CPW; ++c) write_partials(c);
  __syncthreads();

  // ---------------------------------------------------------------- epilogue
  // wave w finishes tile w % TR, tokens 4j .. 4j + 3 for j = w / TR, w / TR +
  // NW / TR, ... (the 4-token groups of an 8- or 16-token tile are finished
  // by different waves at once)
  if (MT == 4 ? wave < TR : true) {
    const int et = wave % TR, n = n0 + 16 * et + e_row;
    for (int jt = wave / TR; jt < MT / 4; jt += NW / TR) {
      const int m = e_m + 4 * jt;
      if (m < M && n < N) {
        const float* rr = red + (size_t)(16 * et + e_row) * MT + m;
        float acc = rr[0];
        if constexpr (CMP) {
          // the slots in chunk order, all reads issued together (indices
          // clamped to the last slot), then added
          const int ns = chunk_slots(G);
          float v[kChunks];
#pragma unroll
          for (int q = 1; q < kChunks; ++q) v[q] = rr[(size_t)(q < ns ? q : ns - 1) * RS];
#pragma unroll
          for (int q = 1; q < kChunks; ++q)
            if (q < ns) acc = acc + v[q];
        } else {
#pragma unroll
          for (int q = 1; q < kChunks; ++q) acc = acc + rr[(size_t)q * RS];
        }
        const float y = finish_const(acc, cc, pr.bias != nullptr, bias_dt);
        const long o = (long)m * N + n;
        if (out_dt == kBF16) store_out<kBF16>(pr.out, o, y);
        else if (out_dt == kF16) store_out<kF16>(pr.out, o, y);
        else store_out<kF32>(pr.out, o, y);
      }
    }
  }
}

// grid x: the TR-tile groups of the widest problem; grid y: the problems
inline int decode_max_tiles(const LinearArgs& g) {
  int row_tiles = 1;
  for (int q = 0; q < g.nprob; ++q) row_tiles = std::max(row_tiles, (g.prob[q].N + 15) / 16);
  return row_tiles;
}

}  // namespace actune
