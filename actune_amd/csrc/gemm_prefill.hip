// Prefill packed group-64 GEMM for gfx950 (M > 64): int8 MFMA with the
// per-group fp32 rescale, organised around the VALU budget.
//
// Restates actune/kernels/grouped.py:74-94 / grouped_native.cu:42-88 with the
// canonical chunked fp32 order (common.hpp), bit-identical to every other
// kernel of the library.
//
// Cost model. Each 16x16x64 int8 MFMA (16 cycles of the matrix pipe) needs 4
// v_cvt_f32_i32 + 4 v_fma_f32 per lane for the per-group rescale (32 cycles
// of the vector pipe): the vector pipe is the bottleneck and any other VALU
// work comes straight out of MFMA throughput. The layout below keeps the
// remaining VALU work near one instruction per MFMA:
//  * A workgroup is 4 waves, one per SIMD. Wave w owns TN 16-row weight tiles
//    (rows n_blk + 16*TN*w ...) and all TM 16-token tiles of the workgroup, so
//    the workgroup tile is (64*TN) x (16*TM).
//  * Weights bypass LDS: each wave streams its own rows straight into MFMA
//    A-operand registers (lane (i, kb) loads 16 bytes of row i; the lanes of a
//    row fetch 64 consecutive bytes), swaps halves across lanes with
//    v_permlane32/16_swap and unpacks sub-byte codes in registers; every
//    unpacked slot feeds TM MFMAs.
//  * Activations are staged once per workgroup per stage (KG = 4 or 8
//    groups) into LDS as 16-byte MFMA B slots, unpacked and reordered to the
//    weight width's element order, with their group scales (2^-(sW+sA)
//    folded in). LDS is double-buffered: one barrier per stage.
//  * The MFMAs of group g are issued in the same block as the rescale of
//    group g-1, so the matrix and vector pipes of a SIMD run side by side.
//  * Weight loads run DW = 2 stages of 4 groups ahead in a register ring,
//    activation loads DA = 1 stage ahead of their LDS store (a stage takes
//    over a microsecond: enough lead for loads that miss L2). Shallow rings
//    keep the 64x64 tile at 162 VGPRs, three waves per SIMD; measured on
//    MI355X, the deeper rings (4 / 2 stages, 204 VGPRs, two waves per SIMD)
//    were 3-11% slower.
//  * Tiles are ordered so that the workgroups of one XCD (workgroup ids are
//    dealt to the 8 XCDs round-robin) cover a contiguous range of weight row
//    blocks with all of their token blocks: each XCD's L2 holds the rows it
//    re-reads.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

constexpr int kXcds = 8;
// 64x32-tile launches of at most this many workgroups (one per CU) split K
// in two inside the workgroup and stage 8 groups per barrier; measured on
// MI355X (W4A8): 2048x16384 at M=256 45.2 -> 29.4 us, 2048x11008 32.3 -> 22.2
// us, 4096x4096 at M=128 14.1 -> 11.9 us; slower with more tiles
constexpr int kPrefillSplitTiles = 256;

// LDS byte offset of B slot `slot` of token row `row` of group `gl` of a
// stage of KG groups: each row holds its stage's 4*KG slots (64*KG bytes)
// with the slot index XORed by row % 16, so that both the 16 rows read by
// one ds_read_b128 and the 16 slots of one row written by 16 lanes fall on
// distinct 16-byte bank groups (measured 2-4% faster than a
// [group][row][slot] array swizzled by row / 2).
template <int KG>
__device__ __forceinline__ int pf_slot_addr(int gl, int row, int slot) {
  return (row * (4 * KG) + ((gl * 4 + slot) ^ (row & 15))) * 16;
}

// Outputs i .. i+3 of one token in one store; element i is aligned to four
// elements (8 bytes for 16-bit outputs, 16 for f32).
template <int DT>
__device__ __forceinline__ void store_out4(void* out, long i, const float (&v)[4]) {
  if constexpr (DT == kF32) {
    *reinterpret_cast<v4f*>((float*)out + i) = v4f{v[0], v[1], v[2], v[3]};
  } else {
    uint32_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) h[r] = DT == kBF16 ? f32_to_bf16(v[r]) : f32_to_f16(v[r]);
    *reinterpret_cast<v2u*>((uint16_t*)out + i) = v2u{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  }
}

// KS > 1 splits K inside the workgroup: KS groups of 4 waves each take
// kChunks / KS consecutive canonical chunks of the same output tile. Group 0
// accumulates its chunks as usual; the other groups leave each chunk's
// partial in LDS, and group 0 adds them in chunk order at the end, so the
// result is the canonical one bit for bit. Shapes with few tiles use it to
// shorten each wave's serial walk over K.
//
// CPS (one chunk per stage): with Q = ceil(G/4) <= kChunks every canonical
// chunk holds at most one quad, so with KS = 1 and KG = 4 each stage is
// exactly one chunk. The stage's first group then starts the chunk partial
// with p = d * s, which equals fmaf(d, s, +0) bit for bit, and closing the
// chunk is acc += p with no zeroing of p.
template <int W, int A, int TN, int TM, int KS, int KG, bool DOTS, bool CPS>
__global__ __launch_bounds__(256 * KS) void gemm_prefill(const LinearArgs args, int tiles_m) {
  constexpr int T = shift_of(W) + shift_of(A);
  constexpr int BN = 64 * TN, BM = 16 * TM;
  static_assert(KG == 4 || KG == 8, "a stage is one or two quads (KG groups)");
  constexpr int GS = 8 / W;                   // groups per 16-byte weight load per lane
  constexpr int WST = KG / GS;                // weight load steps per stage
  constexpr int AROW = KG * 8 * A;            // packed activation bytes per token per stage
  constexpr int ACH = BM * AROW / 16;         // 16-byte activation chunks per stage
  constexpr int APT = (ACH + 255) / 256;      // per thread
  constexpr int SPT = (BM * KG + 255) / 256;  // activation scales per thread per stage
  constexpr int ABYTES = KG * BM * 64, SBYTES = BM * KG * 4;
  static_assert(KG % GS == 0, "a weight load never straddles a stage");
  // ring depths (stages) and stage unroll
  constexpr int DW = KG == 8 ? 1 : 2, DA = 1, UQ = KG == 8 ? 2 : 4;
  static_assert(UQ % DW == 0 && UQ % DA == 0 && UQ % 2 == 0, "static ring indices");
  constexpr int NC = kChunks / KS;            // canonical chunks per K group
  // chunk partials of K groups 1..KS-1: [group - 1][wave][chunk][tile][lane] x 4
  constexpr int CPART = KS > 1 && !DOTS ? (KS - 1) * 4 * NC * TN * TM * 64 * 4 : 1;
  static_assert(KS == 1 || KS * 2 * (ABYTES + SBYTES) + CPART * 4 <= 150 * 1024, "LDS");
  static_assert(!CPS || (KS == 1 && KG == 4 && !DOTS), "one chunk per stage: one K group of quad stages");

  __shared__ __align__(16) uint8_t alds[KS][2][ABYTES + SBYTES];
  __shared__ __align__(16) float cpart[CPART];
  __shared__ float wsl[DOTS ? 1 : BN], bsl[DOTS ? 1 : BN];

  const float fold = __builtin_ldexpf(1.0f, -T);
  const int M = args.M, K = args.K, N = args.prob[0].N, G = K / kGroup;
  const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3;
  const int kgrp = __builtin_amdgcn_readfirstlane(tid >> 8), ltid = tid & 255;  // K group, thread in it
  const int i = lane & 15, kb = lane >> 4;
  // This K group's groups [g_lo, g_hi) in Qk stages of KG groups from g_lo
  // (stage v: groups g_lo + v*KG ...). Groups of the last stage past g_hi
  // belong to the next K group or lie past K: their activation scales are
  // loaded as 0, so they add fma(d, 0, p) = p exactly (and the dots mode skips
  // them). Qmax: the most stages of any K group (every wave runs that many
  // barrier rounds).
  auto k_range = [&](int k, int& glo, int& ghi, int& qk) {
    glo = chunk_begin(k * NC, G);
    ghi = chunk_begin((k + 1) * NC, G);
    qk = glo < ghi ? (ghi - glo + KG - 1) / KG : 0;
  };
  int g_lo, g_hi, Qk, Qmax = 0;
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    int a, b, d;
    k_range(k, a, b, d);
    Qmax = d > Qmax ? d : Qmax;
  }
  k_range(kgrp, g_lo, g_hi, Qk);

  // XCD-aware tile order: XCD x = id % 8 takes tiles [x*per + min(x, rem), ...)
  // in n-major order (consecutive tiles share a weight row block).
  const int ntiles = (int)gridDim.x, id = (int)blockIdx.x;
  const int xcd = id % kXcds, per = ntiles / kXcds, rem = ntiles % kXcds;
  const int tile = xcd * per + (xcd < rem ? xcd : rem) + id / kXcds;
  const int n_blk = (tile / tiles_m) * BN, m_blk = (tile % tiles_m) * BM;
  const int n_wave = n_blk + wave * 16 * TN;

  const uint32_t wrow_bytes = (uint32_t)K * W / 8, arow_bytes = (uint32_t)K * A / 8;
  const Rsrc wres = make_rsrc(args.prob[0].w, (uint32_t)N * wrow_bytes);
  const Rsrc ares = make_rsrc(args.a, (uint32_t)M * arow_bytes);
  const Rsrc sres = make_rsrc(args.as, DOTS ? 4u : (uint32_t)M * G * 4);
  const int slot_b = smallm_slot_k<W>(kb) >> 4;  // B slot matching this lane's weight slot

  // epilogue constants of the workgroup's rows, through LDS
  if constexpr (!DOTS) {
    for (int t = tid; t < BN; t += 256 * KS) {
      const ChannelConst cc = fetch_channel(args.prob[0].ws, args.prob[0].bias, args.bias_dt, N, n_blk + t, true);
      wsl[t] = cc.ws;
      bsl[t] = bias_from_bits(cc.bias_bits, args.bias_dt);
    }
  }

  // ---------------------------------------------------------------- operand movers
  // Register rings: the weight loads of stage v sit in wring[v % DW] (issued DW
  // stages ahead), the activation chunks of stage v in araw[v % DA] (issued DA
  // stages ahead of their LDS store). The stage loop is unrolled by UQ so every
  // ring index is a constant.
  uint32_t wring[DW][WST][TN][4];
  uint32_t araw[DA][APT][4];
  float sraw[DA][SPT];

  // Load offsets = a per-lane base (kOff for rows/tokens past the end, so the
  // sum stays out of range) + a uniform per-stage offset. Bytes past the end
  // of K (tail stage, prefetch past the last stage) read the following row, or
  // zeros past the buffer; their groups have activation scale 0, so they add
  // fma(d, 0, p) = p exactly (and the dots mode skips them).
  uint32_t wbase[TN];
#pragma unroll
  for (int x = 0; x < TN; ++x) {
    const int n = n_wave + x * 16 + i;
    wbase[x] = n < N ? (uint32_t)n * wrow_bytes + kb * 16 : kOff;
  }
  auto load_weights = [&](int q, int st, uint32_t (&buf)[TN][4]) {
    const uint32_t off = (uint32_t)(g_lo + q * KG + st * GS) * 8 * W;
#pragma unroll
    for (int x = 0; x < TN; ++x) buffer_slot<8>(wres, wbase[x] + off, buf[x]);
  };
  uint32_t abase[APT];
#pragma unroll
  for (int t = 0; t < APT; ++t) {
    const int ch = ltid + t * 256, row = ch / (AROW / 16), cc = ch % (AROW / 16);
    const int m = m_blk + row;
    abase[t] = ch < ACH && m < M ? (uint32_t)m * arow_bytes + cc * 16 : kOff;
  }
  auto load_acts = [&](int q, int rs) {  // stage q into ring slot rs
#pragma unroll
    for (int t = 0; t < APT; ++t) buffer_slot<8>(ares, abase[t] + (uint32_t)(g_lo + q * KG) * 8 * A, araw[rs][t]);
    if constexpr (!DOTS) {
#pragma unroll
      for (int t = 0; t < SPT; ++t) {
        const int e = ltid + t * 256, row = e / KG, gl = e % KG;
        const int m = m_blk + row, g = g_lo + q * KG + gl;
        const bool ok = e < BM * KG && m < M && g < g_hi;
        sraw[rs][t] = buffer_f32(sres, ok ? ((uint32_t)m * G + g) * 4u : kOff);
      }
    }
  };
  auto store_acts = [&](uint8_t* buf, int rs) {  // ring slot rs into LDS buffer buf
    float* sl = reinterpret_cast<float*>(buf + ABYTES);
#pragma unroll
    for (int t = 0; t < APT; ++t) {
      const int ch = ltid + t * 256;
      if (ch >= ACH) break;
      const int row = ch / (AROW / 16), cc = ch % (AROW / 16);
      constexpr int SPC = 8 / A;  // slots per 16-byte chunk
#pragma unroll
      for (int u = 0; u < SPC; ++u) {
        const int slot_all = cc * SPC + u, gl = slot_all / 4, slot = slot_all % 4;
        uint32_t d[4];
        unpack_slot<A>(&araw[rs][t][u * A / 2], d);
        reorder_slot<A, W>(d);
        *reinterpret_cast<v4u*>(buf + pf_slot_addr<KG>(gl, row, slot)) = v4u{d[0], d[1], d[2], d[3]};
      }
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int t = 0; t < SPT; ++t) {
        const int e = ltid + t * 256;
        if (e < BM * KG) sl[e] = sraw[rs][t] * fold;  // [token][group of the stage]
      }
    }
  };

  // ---------------------------------------------------------------- accumulators
  float acc[TN][TM][4], p[TN][TM][4];
#pragma unroll
  for (int x = 0; x < TN; ++x)
#pragma unroll
    for (int y = 0; y < TM; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[x][y][r] = p[x][y][r] = 0.f;
  // MFMA results of group g live in D[g & 1] until the block of group g+1
  // rescales them (no register copies: stages have an even number of groups,
  // so the parity of g is that of its index in the stage). D[1] starts at zero,
  // so the rescale in the block of group 0 adds fma(0, 0, +0) = +0.
  v4i D[2][TN][TM];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y) D[b][x][y] = v4i{0, 0, 0, 0};
  float scl[TM];  // token scales of the last group of the previous stage
#pragma unroll
  for (int y = 0; y < TM; ++y) scl[y] = 0.0f;
  int c = kgrp * NC, cend = chunk_begin(kgrp * NC + 1, G);  // chunk being accumulated, and its end
  // p += D[par] * scale for group gq, or p = D[par] * scale for the first
  // group of a chunk under CPS (dots mode: store the dots of gq instead)
  auto rescale = [&](int par, const float (&sc)[TM], int gq, bool first) {
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y) {
        if constexpr (DOTS) {
          if (gq < g_lo || gq >= g_hi) continue;  // the groups of this K group
          const int m = m_blk + y * 16 + i;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = n_wave + x * 16 + 4 * kb + r;
            if (n < N && m < M) args.dots[((long)m * N + n) * G + gq] = D[par][x][y][r] >> T;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            p[x][y][r] = first ? (float)D[par][x][y][r] * sc[y] : __builtin_fmaf((float)D[par][x][y][r], sc[y], p[x][y][r]);
        }
      }
  };
  // acc += p in chunk order (acc starts at +0 and p is never -0, so closing an
  // empty chunk adds +0 and changes nothing); K groups past the first leave
  // the chunk's partial in LDS for group 0 instead
  auto cpart_at = [&](int k, int cl, int x, int y) {
    return cpart + (((((k - 1) * 4 + wave) * NC + cl) * TN + x) * TM + y) * 256 + lane * 4;
  };
  auto close_chunk = [&]() {
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y) {
        if constexpr (KS > 1 && !DOTS) {
          if (kgrp != 0) {
            *reinterpret_cast<v4f*>(cpart_at(kgrp, c - kgrp * NC, x, y)) = v4f{p[x][y][0], p[x][y][1], p[x][y][2], p[x][y][3]};
#pragma unroll
            for (int r = 0; r < 4; ++r) p[x][y][r] = 0.f;
            continue;
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) { acc[x][y][r] = acc[x][y][r] + p[x][y][r]; p[x][y][r] = 0.f; }
      }
    ++c;
    cend = chunk_begin(c + 1, G);
  };
  // CPS: the chunk of the stage just rescaled ends here; p is overwritten by
  // the next stage's first rescale, so it is not cleared
  auto close_stage = [&]() {
#pragma unroll
    for (int x = 0; x < TN; ++x)
#pragma unroll
      for (int y = 0; y < TM; ++y)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[x][y][r] = acc[x][y][r] + p[x][y][r];
  };

  // ---------------------------------------------------------------- prologue
#pragma unroll
  for (int v = 0; v < DA; ++v) load_acts(v, v);
#pragma unroll
  for (int v = 0; v < DW; ++v)
#pragma unroll
    for (int st = 0; st < WST; ++st) load_weights(v, st, wring[v][st]);
  store_acts(alds[kgrp][0], 0);
  load_acts(DA, 0);
  __syncthreads();

  // ---------------------------------------------------------------- main loop
  // Branch-free per group: groups past G (the tail of the last stage) have
  // activation scale 0, so their rescale fma(d, 0, p) leaves p unchanged.
  // Every wave runs Qmax barrier rounds; a K group with fewer stages idles
  // through the last ones.
  for (int v0 = 0; v0 < Qmax; v0 += UQ) {
#pragma unroll
  for (int u = 0; u < UQ; ++u) {
    const int v = v0 + u;
    if (v < Qmax) {  // uniform: false only in the last pass
    if (v < Qk) {    // uniform
    const int q = v;  // stage of this K group
    const int ws_slot = u % DW, as_next = (u + 1) % DA;
    const uint8_t* buf = alds[kgrp][u & 1];
    const float* sl = reinterpret_cast<const float*>(buf + ABYTES);
    float sq[TM][KG];
    if constexpr (!DOTS) {
#pragma unroll
      for (int y = 0; y < TM; ++y) {
#pragma unroll
        for (int h = 0; h < KG / 4; ++h) {
          const v4u s4 = *reinterpret_cast<const v4u*>(sl + (y * 16 + i) * KG + 4 * h);
#pragma unroll
          for (int gl = 0; gl < 4; ++gl) sq[y][4 * h + gl] = __uint_as_float(s4[gl]);
        }
      }
    }
    // B fragments of the current group and (read one block ahead) the next
    uint32_t bf[2][TM][4];
    auto read_b = [&](int gl, uint32_t (&dst)[TM][4]) {
#pragma unroll
      for (int y = 0; y < TM; ++y) {
        const v4u b = *reinterpret_cast<const v4u*>(buf + pf_slot_addr<KG>(gl, y * 16 + i, slot_b));
        dst[y][0] = b[0]; dst[y][1] = b[1]; dst[y][2] = b[2]; dst[y][3] = b[3];
      }
    };
    read_b(0, bf[0]);
#pragma unroll
    for (int gl = 0; gl < KG; ++gl) {
      const int g = g_lo + q * KG + gl;
      const int st = gl / GS, jj = gl % GS;
      if (jj == 0) {
#pragma unroll
        for (int x = 0; x < TN; ++x) exchange<W>(wring[ws_slot][st][x]);
      }
      uint32_t wd[TN][4];
#pragma unroll
      for (int x = 0; x < TN; ++x) unpack_slot<W>(&wring[ws_slot][st][x][jj * W / 2], wd[x]);
      if (jj == GS - 1) load_weights(q + DW, st, wring[ws_slot][st]);
      if (gl + 1 < KG) read_b(gl + 1, bf[(gl + 1) & 1]);
#pragma unroll
      for (int x = 0; x < TN; ++x)
#pragma unroll
        for (int y = 0; y < TM; ++y) D[gl & 1][x][y] = mfma16x16x64(wd[x], bf[gl & 1][y], v4i{0, 0, 0, 0});
      {
        float sp[TM];  // scales of group g-1
#pragma unroll
        for (int y = 0; y < TM; ++y) sp[y] = gl > 0 ? sq[y][gl > 0 ? gl - 1 : 0] : scl[y];
        rescale((gl + 1) & 1, sp, g - 1, CPS && gl == 1);
      }
      if constexpr (!DOTS) {
        // one MFMA of group g, then 8 VALU of the rescale of group g-1
#pragma unroll
        for (int k = 0; k < TN * TM; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
        }
        if constexpr (CPS) {
          // the previous stage's chunk (at the first stage: p = acc = +0);
          // the use of acc keeps the sums in this block, before the next
          // group's products overwrite p (sunk past them, the old and new p
          // would both be live and the loop would copy one into the other)
          if (gl == 0) {
            close_stage();
#pragma unroll
            for (int x = 0; x < TN; ++x)
#pragma unroll
              for (int y = 0; y < TM; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) asm volatile("" ::"v"(acc[x][y][r]));
          }
        } else if (gl % 4 == 0) {  // chunks start on quads
          // chunks that end before group g (the group's own last chunk closes
          // after the loop: groups past g_hi belong to no chunk of this group)
          while (g >= cend && c < (kgrp + 1) * NC - 1) close_chunk();
        }
      }
      if constexpr (!DOTS) {
        // Keep the rescale of group g-1 in this block: without a use here the
        // compiler sinks it to the end of the stage, away from the MFMAs it is
        // meant to overlap.
#pragma unroll
        for (int x = 0; x < TN; ++x)
#pragma unroll
          for (int y = 0; y < TM; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) asm volatile("" ::"v"(p[x][y][r]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!DOTS) {
#pragma unroll
      for (int y = 0; y < TM; ++y) scl[y] = sq[y][KG - 1];
    }
    store_acts(alds[kgrp][(u + 1) & 1], as_next);
    load_acts(q + 1 + DA, as_next);
    }
    __syncthreads();
    }
  }
  }
  rescale((KG - 1) & 1, scl, g_lo + Qk * KG - 1, false);  // the last group
  if constexpr (DOTS) return;
  if constexpr (CPS) close_stage();  // the remaining chunks are empty
  else while (c < (kgrp + 1) * NC) close_chunk();
  if constexpr (KS > 1) {
    // group 0 adds the other groups' chunk partials in chunk order
    __syncthreads();
    if (kgrp != 0) return;
    for (int k = 1; k < KS; ++k)
      for (int cl = 0; cl < NC; ++cl)
#pragma unroll
        for (int x = 0; x < TN; ++x)
#pragma unroll
          for (int y = 0; y < TM; ++y) {
            const v4f pv = *reinterpret_cast<const v4f*>(cpart_at(k, cl, x, y));
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[x][y][r] = acc[x][y][r] + pv[r];
          }
  }

  // ---------------------------------------------------------------- epilogue
  const bool has_bias = args.prob[0].bias != nullptr;
  // a lane's 4 rows are 4 consecutive outputs of one token: one vector store
  // when N and the output pointer keep them aligned (rows past N excepted);
  // measured 2-8% faster than four 2-byte stores on the M = 512 shapes
  const int ebytes = args.out_dt == kF32 ? 4 : 2;
  void* const out = args.prob[0].out;
  const bool vec_out = N % 4 == 0 && ((uintptr_t)out % (4 * ebytes)) == 0;
#pragma unroll
  for (int x = 0; x < TN; ++x) {
    const int nl = wave * 16 * TN + x * 16 + 4 * kb;  // first of this lane's 4 rows in the tile
#pragma unroll
    for (int y = 0; y < TM; ++y) {
      const int m = m_blk + y * 16 + i;
      if (m >= M) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float a = acc[x][y][r];
        v[r] = has_bias ? __builtin_fmaf(a, wsl[nl + r], bsl[nl + r]) : a * wsl[nl + r];
      }
      const int n0 = n_blk + nl;
      const long o = (long)m * N + n0;
      if (vec_out && n0 + 3 < N) {
        if (args.out_dt == kBF16) store_out4<kBF16>(out, o, v);
        else if (args.out_dt == kF16) store_out4<kF16>(out, o, v);
        else store_out4<kF32>(out, o, v);
        continue;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (n0 + r >= N) break;
        if (args.out_dt == kBF16) store_out<kBF16>(out, o + r, v[r]);
        else if (args.out_dt == kF16) store_out<kF16>(out, o + r, v[r]);
        else store_out<kF32>(out, o + r, v[r]);
      }
    }
  }
}

// Shapes (TN, TM): 0 = (2, 4) 128x64, 1 = (2, 2) 128x32, 2 = (1, 4) 64x64, 3 = (1, 2) 64x32.
template <int W, int A, bool DOTS>
static void launch_prefill_shape(int shape, const LinearArgs& g, hipStream_t st) {
#define PREFILL(TN, TM, KS, KG, CPS)                                                          \
  gemm_prefill<W, A, TN, TM, KS, KG, DOTS, CPS><<<dim3((unsigned)(tn * tm)), 256 * KS, 0, st>>>(g, tm)
// one K group of quad stages: one chunk per stage when ceil(G/4) <= kChunks
#define PREFILL4(TN, TM)                                  \
  if (!DOTS && (g.K / kGroup + 3) / 4 <= kChunks)         \
    PREFILL(TN, TM, 1, 4, !DOTS);                         \
  else                                                    \
    PREFILL(TN, TM, 1, 4, false)
  const int TN_ = shape < 2 ? 2 : 1, TM_ = (shape & 1) ? 2 : 4;
  const int tn = (g.prob[0].N + 64 * TN_ - 1) / (64 * TN_), tm = (g.M + 16 * TM_ - 1) / (16 * TM_);
  switch (shape) {
    case 0: PREFILL4(2, 4); break;
    case 1: PREFILL4(2, 2); break;
    case 2: PREFILL4(1, 4); break;
    default:
      if (tn * tm <= kPrefillSplitTiles) PREFILL(1, 2, 2, 8, false);
      else PREFILL4(1, 2);
      break;
  }
#undef PREFILL4
#undef PREFILL
}

void launch_prefill(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st) {
#define CASE(WB, AB)                                                                \
  if (W == WB && A == AB) {                                                         \
    if (dots) launch_prefill_shape<WB, AB, true>(shape, g, st);                     \
    else launch_prefill_shape<WB, AB, false>(shape, g, st);                         \
    return;                                                                         \
  }
  CASE(8, 8) CASE(8, 4) CASE(8, 2) CASE(4, 8) CASE(4, 4) CASE(4, 2) CASE(2, 8) CASE(2, 4) CASE(2, 2)
#undef CASE
}

}  // namespace actune
