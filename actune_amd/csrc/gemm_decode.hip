// Decode packed group-64 GEMM for gfx950 (M <= 4 tokens, quantizer fused):
// the launch is bound by the HBM read of the packed weights, so the kernel is
// shaped for memory-level parallelism.
//
// Restates the per-call math of actune/kernels/grouped.py:55-94 (group-64
// quantizer, exact int32 dot per group, fp32 rescale, weight-scale epilogue;
// the optional channel scale of layers.py:41-42 is divided in first), in the
// canonical chunked order of common.hpp.
//
// Structure:
//  * A workgroup is NW waves and owns one 16-row tile of one problem (up to
//    kMaxProblems linears that read the same x share a launch; the problem
//    is blockIdx.y, so each workgroup reads only its own problem's kernel
//    arguments, in the one batch of scalar loads before its first memory
//    load). The waves
//    split K along the 16 canonical chunks. Workgroups are light (small LDS,
//    no per-tile staging), so several are resident per CU and nearly every
//    tile of a decode-size problem is in flight at once.
//  * Each wave issues all its loads at entry, unconditionally (lanes and
//    passes with nothing to read load out of range and get zeros without
//    memory traffic): kPass x passes, then its whole K-range of weights as
//    RING 16-byte loads per lane. It then quantizes its K-range of x into a
//    wave-private LDS slab while the weights arrive. Straight-line loads let
//    every use wait for exactly its own load (in-order memory counter);
//    shapes whose K-range per wave needs more loads run the small-M kernel
//    (decode_fits).
//  * Weight slots reach MFMA A-operand form with v_permlane32/16_swap and
//    register unpacking (the small-M kernel's load pattern: lanes of a row
//    fetch 64 consecutive bytes); the tokens are the B operand, read from the
//    slab. One fp32 FMA per (row, token, group).
//  * Chunk partials meet in a small LDS array [16 chunks][16 rows][4 tokens]
//    and are added in chunk order after one barrier.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

constexpr int kDecodeMaxM = 4;

// Dynamic LDS: per wave a slab [GW groups][M tokens][64 B] and a scale slab
// [GW][4] (fp32, 2^-(sW+sA) folded in; entries of absent tokens unused), one
// 64-byte zero row, and the chunk partials red[16][16][kDecodeMaxM].
// Largest groups per wave of a K split over nw waves.
static int decode_groups_per_wave(int K, int nw) {
  const int G = K / kGroup, cpw = kChunks / nw;
  int gw = 1;
  for (int w = 0; w < nw; ++w) {
    const int d = chunk_begin((w + 1) * cpw, G) - chunk_begin(w * cpw, G);
    gw = d > gw ? d : gw;
  }
  return gw;
}

// 16-byte weight loads per lane: 16 groups of W2 / W4, 8 groups of W8
__host__ __device__ constexpr int decode_ring(int W) { return W == 2 ? 4 : 8; }
constexpr int kDecodePass = 4;   // x passes of 8 group-rows

bool decode_fits(int K, int M, int W, int nw) {
  const int gw = decode_groups_per_wave(K, nw);
  return M <= kDecodeMaxM && (gw + 8 / W - 1) / (8 / W) <= decode_ring(W) && gw * M <= 8 * kDecodePass &&
         decode_lds_bytes(K, M, nw) <= kStreamLdsMax;
}

// true when every one of nw waves gets exactly a full ring of weight slots
static bool decode_full(int K, int W, int nw) {
  const int G = K / kGroup, cpw = kChunks / nw, per = decode_ring(W) * (8 / W);
  for (int w = 0; w < nw; ++w)
    if (chunk_begin((w + 1) * cpw, G) - chunk_begin(w * cpw, G) != per) return false;
  return true;
}

// zero region: a wave's widest K-range (16 groups) of 64-byte zero rows
constexpr int kDecodeZeroBytes = 16 * kGroup;

size_t decode_lds_bytes(int K, int M, int nw) {
  const int gw = decode_groups_per_wave(K, nw);
  return (size_t)nw * gw * (M * kGroup + 4 * sizeof(float)) + kDecodeZeroBytes +
         sizeof(float) * kChunks * 16 * kDecodeMaxM;
}

// chunk_begin in unsigned arithmetic (c, G >= 0): shifts instead of the
// signed-division sequences, for the slot loop's scalar chunk tracking
__device__ __forceinline__ int chunk_begin_u(int c, int G) {
  const uint32_t Q = ((uint32_t)G + 3u) >> 2;
  const uint32_t b = (((uint32_t)c * Q) >> 4) << 2;
  return b < (uint32_t)G ? (int)b : G;
}

// ONE: M == 1 (only register 0 of the MFMA result is rescaled). FULL: every
// wave's K-range is exactly RING slots (decode_full), so the slot pipeline
// runs without bounds tests. ONE launches read token operands at constant
// LDS offsets and keep the group scales in scalar registers; with FULL they
// also issue exactly the x passes of the K-range.
template <int W, int A, int NW, int RING, int DT, bool SCALE, bool ONE, bool FULL>
__global__ __launch_bounds__(NW * 64) void gemm_decode(const LinearArgs args, int GW) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int GS = 8 / W;                // groups per 16-byte weight load per lane
  constexpr int CPW = kChunks / NW;        // canonical chunks per wave
  constexpr int T = shift_of(W) + shift_of(A);
  constexpr int ESZ = DT == kF32 ? 4 : 2;
  constexpr int XL = DT == kF32 ? 2 : 1;   // 16-byte loads per 8 elements of x
  constexpr int kPass = kDecodePass;      // x passes (8 group-rows each) loaded before the weights
  constexpr bool FAST = ONE;
  constexpr int NPX = FULL && ONE ? (RING * GS + 7) / 8 : kPass;  // x passes issued

  const float fold = __builtin_ldexpf(1.0f, -T);
  // Every kernel argument the prologue needs is read here, in one batch of
  // scalar loads with one wait: the empty asm takes the values as operands
  // it may change, so none of them is reloaded later (a reload would put a
  // scalar round trip between entry and the first weight load).
  // The problem is blockIdx.y: its fields sit at an offset known at entry.
  Problem pr = args.prob[blockIdx.y];
  int M = args.M, K = args.K, bias_dt = args.bias_dt, out_dt = args.out_dt;
  uint32_t m_inv = args.m_div;  // idx / M == (idx * m_inv) >> 16 here
  const void* xsrc = args.x;
  const void* xscale = args.xscale;
  asm volatile("" : "+s"(M), "+s"(K), "+s"(bias_dt), "+s"(out_dt), "+s"(m_inv), "+s"(xsrc), "+s"(xscale), "+s"(GW),
                    "+s"(pr.w), "+s"(pr.ws), "+s"(pr.bias), "+s"(pr.out), "+s"(pr.N));
  const int N = pr.N, G = K / kGroup;
  const int n0 = (int)blockIdx.x * 16;
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

  uint8_t* slab = smem + (size_t)wave * GW * M * kGroup;
  float* sslab = reinterpret_cast<float*>(smem + (size_t)NW * GW * M * kGroup) + (size_t)wave * GW * 4;
  uint8_t* zero_row = reinterpret_cast<uint8_t*>(reinterpret_cast<float*>(smem + (size_t)NW * GW * M * kGroup) +
                                                 (size_t)NW * GW * 4);
  float (*red)[16][kDecodeMaxM] = reinterpret_cast<float (*)[16][kDecodeMaxM]>(zero_row + kDecodeZeroBytes);

  // The output this thread finishes in the epilogue (wave 0: row lane / 4,
  // token lane % 4).
  const int e_row = lane >> 2, e_m = lane & 3;

  // ---------------------------------------------------------------- x loads
  // Group-row r = gl * M + m (gl: group of the wave's range, m: token); a
  // pass covers 8 group-rows, 8 lanes each, 8 consecutive elements per lane.
  const int rows_here = ng * M;
  const int npass = (rows_here + 7) / 8;
  const Rsrc xres = make_rsrc(xsrc, (uint32_t)M * K * ESZ);
  const Rsrc xsres = make_rsrc(SCALE ? xscale : xsrc, (uint32_t)K * ESZ);
  const int seg = lane & 7;
  struct Raw { v4u x[XL], s[XL]; };
  // M == 1: lane l of pass p reads elements wg0*64 + p*512 + 8l.. of x (the
  // rows past the wave's range read neighbouring elements or zeros and are
  // not stored); the pass is a constant offset, passes past npass are
  // switched off through the scalar offset.
  const uint32_t xbase1 = ((uint32_t)wg0 * kGroup + (uint32_t)lane * 8) * ESZ;
  auto issue_x = [&](int pass, Raw& r) {
    if constexpr (ONE) {
      const uint32_t soff = pass < npass ? 0u : kOff;
#pragma unroll
      for (int h = 0; h < XL; ++h) {
        r.x[h] = __builtin_amdgcn_raw_buffer_load_b128(xres, xbase1 + (uint32_t)(pass * 512 * ESZ + 16 * h), soff, 0);
        if constexpr (SCALE)
          r.s[h] = __builtin_amdgcn_raw_buffer_load_b128(xsres, xbase1 + (uint32_t)(pass * 512 * ESZ + 16 * h), soff, 0);
      }
      return;
    }
    const int idx = pass * 8 + (lane >> 3);
    const bool live = idx < rows_here;
    const int q = ONE ? idx : (int)(((uint32_t)idx * m_inv) >> 16);
    const int gl = live ? q : 0, m = ONE || !live ? 0 : idx - q * M;
    const uint32_t k0 = (uint32_t)((wg0 + gl) * kGroup + seg * 8);
    const uint32_t xo = live ? ((uint32_t)m * K + k0) * ESZ : kOff;
#pragma unroll
    for (int h = 0; h < XL; ++h) r.x[h] = __builtin_amdgcn_raw_buffer_load_b128(xres, xo == kOff ? kOff : xo + 16 * h, 0, 0);
    if constexpr (SCALE) {
      const uint32_t so = live ? k0 * ESZ : kOff;
#pragma unroll
      for (int h = 0; h < XL; ++h) r.s[h] = __builtin_amdgcn_raw_buffer_load_b128(xsres, so == kOff ? kOff : so + 16 * h, 0, 0);
    }
  };
  auto convert_x = [&](int pass, const Raw& r) {
    const int idx = pass * 8 + (lane >> 3);
    const bool live = idx < rows_here;
    const int q = ONE ? idx : (int)(((uint32_t)idx * m_inv) >> 16);
    const int gl = live ? q : 0, m = ONE || !live ? 0 : idx - q * M;
    float v[8];
    unpack8<DT>(r.x[0], r.x[XL - 1], v);
    if constexpr (SCALE) {
      float d[8];
      unpack8<DT>(r.s[0], r.s[XL - 1], d);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = live ? round_to_dtype<DT>(v[e] / d[e]) : 0.0f;
    }
    uint32_t cq[8];
    const float s = group_code_bits<A, DT>(v, cq);
    if (live) {
      store_half_slot<W, A>(slab + (gl * M + m) * kGroup + (seg >> 1) * 16, seg & 1, cq);
      if (!FAST && seg == 0) sslab[gl * 4 + m] = s * fold;
    }
    return s * fold;  // the same in the 8 lanes of a group
  };
  Raw early[kPass];
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
  // the host guarantees ns <= RING and npass <= kPass (decode_fits)
  uint32_t ring[RING][4];
#pragma unroll
  for (int st = 0; st < RING; ++st) {
    // (a runtime test also where every slot is live: with a constant offset
    // the compiler schedules the loads differently and the launch measured
    // 0.4 us slower at one workgroup per CU)
    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(wres, wbase + (uint32_t)st * 64, st < ns ? 0u : kOff, 0);
    ring[st][0] = q[0]; ring[st][1] = q[1]; ring[st][2] = q[2]; ring[st][3] = q[3];
  }
  // epilogue constants, behind the weights: they are needed last, by wave 0.
  // Every wave issues the two loads (switched off outside wave 0) so that all
  // waves have the same loads in flight: behind a branch, the compiler's
  // waits for the x passes would count from the shorter path and make wave 0
  // wait for weight slots before quantizing.
  const ChannelConst cc = fetch_channel(pr.ws, pr.bias, bias_dt, N, n0 + e_row, wave == 0 && e_m < M);

  // ---------------------------------------------------------------- quantize x
  // the zero region: one dword per thread of the first four waves
  if (threadIdx.x < kDecodeZeroBytes / 4) reinterpret_cast<uint32_t*>(zero_row)[threadIdx.x] = 0u;
  // FAST: the wave's group scales (s * 2^-T, wave-uniform) move from the
  // quantizing lanes into scalar registers
  float gsc[FAST ? RING * GS : 1];
#pragma unroll
  for (int p = 0; p < NPX; ++p) {
    if ((FULL && ONE) || p < npass) {
      const float sf = convert_x(p, early[p]);
      if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (p * 8 + j < RING * GS) gsc[p * 8 + j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sf), 8 * j));
      }
    }
  }
  // the zero region and the slabs are written across waves
  __syncthreads();

  // ---------------------------------------------------------------- stream the K-range
  float p[4] = {0.f, 0.f, 0.f, 0.f};
  int c = c_first;
  if constexpr (FAST) {
    // M == 1: lanes of token 0 (i == 0) read the wave's slab, the others the
    // zero region, both with stride 64 per group, so every token operand
    // read is one LDS load at a constant offset (reads past the wave's range
    // stay inside LDS and are never used); the rescale takes its scale from
    // a scalar register. Same pipeline and order as the general loop below.
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
      exchange<W>(ring[st]);
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        uint32_t wd[4];
        unpack_slot<W>(&ring[st][jj * W / 2], wd);
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
      const int g0 = wg0 + st * GS;
      while (g0 >= cend && c < c_last) {  // close finished (possibly empty) chunks
        if (lane < 16) *reinterpret_cast<v4f*>(&red[c][lane][0]) = v4f{p[0], 0.f, 0.f, 0.f};
        p[0] = 0.f;
        ++c;
        cend = chunk_begin_u(c + 1, G);
      }
      if constexpr (GS == 1) {  // see the general loop
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 1");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) p[0] = __builtin_fmaf((float)D[st][jj][0], gsc[st * GS + jj], p[0]);
    }
  } else {
    // The tokens are the MFMA A operand and the weight rows the B operand, so
    // token m of weight row c lands in lane c, register m: only M registers of
    // lanes 0..15 carry results and only those are rescaled. The GS MFMAs of a
    // slot are issued together and folded in group order.
    const int slot_k = smallm_slot_k<W>(kb);
    // Lanes of absent tokens (i >= M) read the zero row with stride 0. A group
    // past the wave's range (the tail of its last slot, or a slot read ahead
    // and never used) reads a clamped slab row and a zero scale, so it adds
    // exactly nothing.
    const bool tok = i < M;
    const uint8_t* bbase = tok ? slab + i * kGroup + slot_k : zero_row;
    const uint32_t bstride = tok ? (uint32_t)M * kGroup : 0u;
    auto read_b = [&](int st, v4u (&bq)[GS], v4f (&bs)[GS]) {
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        const int gl = max(0, min(st * GS + jj, ng - 1));
        bq[jj] = *reinterpret_cast<const v4u*>(bbase + __umul24((uint32_t)gl, bstride));
        const float* srow = st * GS + jj < ng ? sslab + gl * 4 : reinterpret_cast<const float*>(zero_row);
        bs[jj] = *reinterpret_cast<const v4f*>(srow);  // same address in every lane
      }
    };
    // Software pipeline over the wave's ns slots: slot st+1's MFMAs are issued
    // before slot st's results are rescaled, so MFMA latency hides under that
    // work. Token operands are read three slots ahead. (Slot 0's MFMAs run
    // even when the wave has no slot: its weights and scales are zero.)
    constexpr int RA = 3;
    v4u bq[RING][GS];
    v4f bs[RING][GS];
    v4i D[RING][GS];
#pragma unroll
    for (int st = 0; st < RA && st < RING; ++st) read_b(st, bq[st], bs[st]);
    auto mfma_slot = [&](int st) {
      exchange<W>(ring[st]);
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        uint32_t wd[4];
        unpack_slot<W>(&ring[st][jj * W / 2], wd);
        const uint32_t bd[4] = {bq[st][jj][0], bq[st][jj][1], bq[st][jj][2], bq[st][jj][3]};
        D[st][jj] = mfma16x16x64(bd, wd, v4i{0, 0, 0, 0});
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
      const int g0 = wg0 + st * GS;
      while (g0 >= cend && c < c_last) {  // close finished (possibly empty) chunks
        if (lane < 16) *reinterpret_cast<v4f*>(&red[c][lane][0]) = v4f{p[0], p[1], p[2], p[3]};
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = 0.f;
        ++c;
        cend = chunk_begin(c + 1, G);
      }
      // With one MFMA and one FMA per slot (W8, M == 1) the last slot's
      // result would be read 7 instructions after its MFMA across branches,
      // one short of the wait states the compiler keeps in straight-line
      // code; two more are added here, fenced so the scheduler keeps them in
      // front of the rescale.
      if constexpr (GS == 1 && ONE) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 1");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int jj = 0; jj < GS; ++jj) {
        // registers of absent tokens hold zeros (their scale entries are
        // unset and their partials never read)
        const v4f sc = bs[st][jj];
#pragma unroll
        for (int q = 0; q < (ONE ? 1 : 4); ++q) p[q] = __builtin_fmaf((float)D[st][jj][q], sc[q], p[q]);
      }
    }
  }
  // lane c < 16 holds row c of tokens 0..3 (zero for absent tokens)
  for (; c < c_first + CPW; ++c) {
    if (lane < 16) *reinterpret_cast<v4f*>(&red[c][lane][0]) = v4f{p[0], p[1], p[2], p[3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = 0.f;
  }
  __syncthreads();

  // ---------------------------------------------------------------- epilogue
  if (wave == 0 && e_m < M) {
    const int n = n0 + e_row;
    float acc = red[0][e_row][e_m];
#pragma unroll
    for (int q = 1; q < kChunks; ++q) acc = acc + red[q][e_row][e_m];
    if (n < N) {
      const float y = finish_const(acc, cc, pr.bias != nullptr, bias_dt);
      const long o = (long)e_m * N + n;
      if (out_dt == kBF16) store_out<kBF16>(pr.out, o, y);
      else if (out_dt == kF16) store_out<kF16>(pr.out, o, y);
      else store_out<kF32>(pr.out, o, y);
    }
  }
}

// ---------------------------------------------------------------------------
template <int W, int A, int NW, int DT, bool SCALE, bool ONE, bool FULL>
static void launch_decode_one(const LinearArgs& g, hipStream_t st) {
  constexpr int RING = decode_ring(W);
  const size_t lds = decode_lds_bytes(g.K, g.M, NW);
  auto kern = gemm_decode<W, A, NW, RING, DT, SCALE, ONE, FULL>;
  static bool attr_set = false;  // allow dynamic LDS beyond the default per-launch limit
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kStreamLdsMax);
    attr_set = true;
  }
  int row_tiles = 1;  // grid x: the row tiles of the widest problem; grid y: the problems
  for (int q = 0; q < g.nprob; ++q) row_tiles = std::max(row_tiles, (g.prob[q].N + 15) / 16);
  kern<<<dim3((unsigned)row_tiles, (unsigned)g.nprob), NW * 64, lds, st>>>(g, decode_groups_per_wave(g.K, NW));
}

template <int W, int A, int NW>
static void launch_decode_nw(const LinearArgs& g, hipStream_t st) {
#define DEC_ONE(DTV, SC)                                                        \
  if (g.M == 1) launch_decode_one<W, A, NW, DTV, SC, true, false>(g, st);       \
  else launch_decode_one<W, A, NW, DTV, SC, false, false>(g, st)
  // bf16 activations of shapes whose waves each fill the ring exactly take
  // the bound-free pipeline
  if (g.x_dt == kBF16 && decode_full(g.K, W, NW)) {
    if (g.xscale) {
      if (g.M == 1) launch_decode_one<W, A, NW, kBF16, true, true, true>(g, st);
      else launch_decode_one<W, A, NW, kBF16, true, false, true>(g, st);
    } else {
      if (g.M == 1) launch_decode_one<W, A, NW, kBF16, false, true, true>(g, st);
      else launch_decode_one<W, A, NW, kBF16, false, false, true>(g, st);
    }
    return;
  }
#define DEC_DT(DTV)                                                             \
  if (g.xscale) { DEC_ONE(DTV, true); }                                         \
  else { DEC_ONE(DTV, false); }
  if (g.x_dt == kBF16) { DEC_DT(kBF16); }
  else if (g.x_dt == kF16) { DEC_DT(kF16); }
  else { DEC_DT(kF32); }
#undef DEC_DT
#undef DEC_ONE
}

template <int W, int A>
static void launch_decode_wa(int nw, const LinearArgs& g, hipStream_t st) {
  if (nw == 4) launch_decode_nw<W, A, 4>(g, st);
  else if (nw == 8) launch_decode_nw<W, A, 8>(g, st);
  else launch_decode_nw<W, A, 16>(g, st);
}

void launch_decode(int W, int A, int nw, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB) if (W == WB && A == AB) return launch_decode_wa<WB, AB>(nw, g, st)
  CASE(8, 8); CASE(8, 4); CASE(8, 2);
  CASE(4, 8); CASE(4, 4); CASE(4, 2);
  CASE(2, 8); CASE(2, 4); CASE(2, 2);
#undef CASE
}

}  // namespace actune
