// Tokenwise (per-row) packed-integer linears for gfx950: the per-row dynamic
// A8 / A4 quantizer and one int8-MFMA GEMM for every weight layout of the
// reference's tokenwise family, with exact full-K int32 accumulation and an
// optional exact split-K across workgroups.
//
// Restates (zanehpn/Actune):
//   per-row A8 quantizer  actune/kernels/w4a8_triton.py:161-201 (also
//                         decode_w4a8_triton.py:21-28, resident_a8_triton.py:13-21)
//   per-row A4 quantizer  actune/kernels/wxa4_native.py:28-65
//   W4A8  K-major nibble pairs     w4a8_triton.py:57-114, 380-383
//   W8A8  K-major int8             w8a8_triton.py:21-77, 100-107
//   W2A8  K-major quarters         w2a8_triton.py:24-112, 149-159
//   W4A4 / W2A4 row-major S4 / S2  native_s4_extension_kernel.cu:239-481
//   W8A4  K-major nested int8 x A4 wxa4_native.py:315-391
//   exact split-K, integer reduce  decode_w4a8_triton.py:31-110
//
// Arithmetic. Codes of width b are held as int8 c * 2^(8-b) (the field at the
// top of its byte), so an int8 MFMA returns 2^T times the true dot, T = the
// two operands' shifts; |every product| <= 2^14, so the int32 sum over K is
// exact for K < 2^17 and the arithmetic shift by T recovers the true
// accumulator. Integer sums do not depend on order: split-K partials are
// added in any order and the result is still bit-exact. The fp32 epilogue
// is then one fixed sequence per output (tokenwise_oracle.c):
//   A8 family: t = f32(acc) * as[m]; y = bias ? fmaf(t, ws[n], bias[n]) : t * ws[n]
//   native A4: q = as[m] * ws[n];    y = bias ? fmaf(f32(acc), q, bias[n]) : f32(acc) * q
//
// MFMA operands (v_mfma_i32_16x16x64_i8): tokens are the A operand, output
// channels the B operand; lane l holds row l % 16 and the 16 k-slots of
// group kb = l / 16. The k index behind each slot only has to be the same
// for both operands, so each weight layout uses the slot order its bytes
// give cheapest:
//   K-major layouts (rows of the buffer run along K, columns along N): the
//     weight tile is staged in LDS as buffer rows and read back transposed
//     with ds_read_b64_tr_b8 (in each 16-lane group, lane 2i + h points at
//     row i, bytes 8h..8h+7 of 16 columns; lane c receives column c of the
//     8 rows). One read gives a lane 8 consecutive buffer rows of its column:
//     8 k (W8), 16 k (nibble pairs: k = j and j + K/2) or 32 k (quarters:
//     j + f K/4 for f = 0..3, two MFMAs).
//   row-major S4 / S2 (the group-64 packing): a lane's 16 k-slots are one
//     8- (S4) or 4-byte (S2) run of its row, unpacked in the width's native
//     element order (common.hpp), and the activation slot is reordered to it.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <climits>

#include "../../include/actune_hip.h"
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {
namespace {

constexpr int kThreads = 256;
// longest row the fused-quantization launch takes (8 passes of 8 elements per thread)
constexpr int kTwFusedMaxK = 16384;
// rows the fused-quantization launch takes: up to 8 (16-bit x), with
// 256 / P threads per row for the row counts padded to P = 2, 4, 8 and 16
// passes of 8 elements each, so K <= 32768 / P
constexpr int kTwFusedMaxRows = 8;
constexpr int kTwFusedRowPasses = 16;
inline int tw_fused_rows_pad(int64_t M) { return M <= 2 ? 2 : M <= 4 ? 4 : 8; }
inline int64_t tw_fused_max_k(int64_t M) {
  return M == 1 ? kTwFusedMaxK : (int64_t)kTwFusedRowPasses * 8 * (256 / tw_fused_rows_pad(M));
}

template <int WL> struct WTraits;
// U: MFMAs per K-step (64 k each); TW: shift of the weight codes;
// rows(TN): rows of the staged weight tile; row_bytes(TN): bytes per staged row
template <> struct WTraits<ACTUNE_TW_KMAJOR_W8> {
  static constexpr int U = 1, TW = 0;
  static constexpr bool KM = true;
  static constexpr int rows(int) { return 64; }
  static constexpr int row_bytes(int tn) { return tn; }
};
template <> struct WTraits<ACTUNE_TW_KMAJOR_W4> {
  static constexpr int U = 1, TW = 4;
  static constexpr bool KM = true;
  static constexpr int rows(int) { return 32; }
  static constexpr int row_bytes(int tn) { return tn; }
};
template <> struct WTraits<ACTUNE_TW_KMAJOR_W2> {
  static constexpr int U = 2, TW = 6;
  static constexpr bool KM = true;
  static constexpr int rows(int) { return 32; }
  static constexpr int row_bytes(int tn) { return tn; }
};
// nibble-pair q4 rows (staged rows 0-31) and the residual r4 rows of the
// same K (staged rows 32-63); codes formed as int8 16 q4 + r4
template <> struct WTraits<ACTUNE_TW_KMAJOR_W4R4> {
  static constexpr int U = 1, TW = 0;
  static constexpr bool KM = true;
  static constexpr int rows(int) { return 64; }
  static constexpr int row_bytes(int tn) { return tn; }
};
template <> struct WTraits<ACTUNE_TW_ROWS_S4> {
  static constexpr int U = 1, TW = 4;
  static constexpr bool KM = false;
  static constexpr int rows(int tn) { return tn; }
  static constexpr int row_bytes(int) { return 32; }
};
template <> struct WTraits<ACTUNE_TW_ROWS_S2> {
  static constexpr int U = 1, TW = 6;
  static constexpr bool KM = false;
  static constexpr int rows(int tn) { return tn; }
  static constexpr int row_bytes(int) { return 16; }
};

// Padded LDS row strides: the transposed reads of 8 weight rows and the
// 16-row activation reads each touch distinct banks.
constexpr bool kmajor(int wl) { return wl <= ACTUNE_TW_KMAJOR_W2 || wl == ACTUNE_TW_KMAJOR_W4R4; }
// nibble-pair layouts: a buffer row holds codes j and j + K/2
constexpr bool nibble_pairs(int wl) { return wl == ACTUNE_TW_KMAJOR_W4 || wl == ACTUNE_TW_KMAJOR_W4R4; }
constexpr int w_stride(int wl, int tn) {
  return kmajor(wl) ? tn + 16 : (wl == ACTUNE_TW_ROWS_S4 ? 40 : 20);
}
// activation bytes per staged row and K-step: int8 codes 64 per MFMA (the
// nibble-pair layout stages k = j.. and K/2 + j.. as two 32-byte pieces, the
// quarter layout four), packed A4 codes 32 bytes
constexpr int a_row_bytes(int wl, int al) { return al == ACTUNE_TW_ACT_A4 ? 32 : (wl == ACTUNE_TW_KMAJOR_W2 ? 128 : 64); }
constexpr int a_stride(int wl, int al) { return al == ACTUNE_TW_ACT_A4 ? 40 : a_row_bytes(wl, al) + 16; }

// Per-target operands of a launch over sibling projections (same activation
// rows, K, N and layouts); target 0 is also held in TwArgs' own fields.
struct TwTarget {
  const uint8_t* w;
  const uint8_t* r;
  const float* ws;
  const void* bias;
  void* out;
};

struct TwArgs {
  const uint8_t* a;     // int8 codes [M, K] or packed A4 [M, K/2]
  const void* x;        // activation rows [M, K] (fused quantization; a unused)
  const float* as;      // [M] (fused quantization: written by the launch)
  const uint8_t* w;     // weight buffer (layout WL)
  const float* ws;      // [N]
  const void* bias;     // [N] or nullptr
  void* out;            // [M, N]
  int32_t* partial;     // [T, S, M, N] int32 raw (shifted) partial sums (S > 1)
  const uint8_t* r;     // KMAJOR_W4R4: residual codes (nullptr: r4 = 0)
  float ws_mul;         // 1, or 1/16 for the nested 16 q4 + r4 codes (exact)
  int M, N, K, bias_dt, out_dt, splits, steps;
  int targets;          // T: grid z = S x T (GEMM), T (reduce)
  TwTarget t[ACTUNE_MAX_TARGETS];
};

// The launch's arguments as seen by the workgroups of target `i`: its
// weights, scales, bias and output, and its slice of the partial sums.
__device__ __forceinline__ TwArgs for_target(const TwArgs& in, int i) {
  TwArgs a = in;
  if (i > 0) {
    a.w = in.t[i].w;
    a.r = in.t[i].r;
    a.ws = in.t[i].ws;
    a.bias = in.t[i].bias;
    a.out = in.t[i].out;
    if (in.partial) a.partial = in.partial + (size_t)i * in.splits * in.M * in.N;
  }
  return a;
}

// y for output (m, n) from the true int32 accumulator, in the family's
// fixed fp32 sequence, stored in out_dt.
template <int EPI>
__device__ __forceinline__ void store_result(const TwArgs& a, int m, int n, int32_t acc) {
  const float x = (float)acc;
  const float as = a.as[m], ws = a.ws[n] * a.ws_mul;
  float y;
  if constexpr (EPI == ACTUNE_TW_EPI_A8) {
    const float t = x * as;
    y = a.bias ? __builtin_fmaf(t, ws, load_bias(a.bias, a.bias_dt, n)) : t * ws;
  } else {
    const float q = as * ws;
    y = a.bias ? __builtin_fmaf(x, q, load_bias(a.bias, a.bias_dt, n)) : x * q;
  }
  const size_t o = (size_t)m * a.N + n;
  if (a.out_dt == kBF16) store_out<kBF16>(a.out, o, y);
  else if (a.out_dt == kF16) store_out<kF16>(a.out, o, y);
  else store_out<kF32>(a.out, o, y);
}

// Writes a wave's MT x NT accumulator tiles (lane: rows row_base + 16 mt +
// 0..3, column col_base + 16 nt): with K splits, split z's raw int32 partial
// sums (tw_reduce adds the splits, in any order, and finishes); otherwise
// the finished outputs.
template <int WL, int AL, int EPI, int MT, int NT>
__device__ __forceinline__ void finish_tile(const TwArgs& args, const v4i (&acc)[MT][NT], int row_base,
                                            int col_base, int z) {
  constexpr int SHIFT = WTraits<WL>::TW + (AL == ACTUNE_TW_ACT_A4 ? 4 : 0);
  const int M = args.M, N = args.N;
  if (args.splits > 1) {
    int32_t* part = args.partial + (size_t)z * M * N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = row_base + mt * 16 + i, n = col_base + nt * 16;
          if (m < M && n < N) part[(size_t)m * N + n] = acc[mt][nt][i];
        }
    return;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = col_base + nt * 16;
    if (n >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = row_base + mt * 16 + i;
        if (m < M) store_result<EPI>(args, m, n, acc[mt][nt][i] >> SHIFT);
      }
  }
}

// Bytes of 16 q4 + r4 as int8, wrapped to 8 bits (decode_w4a8_triton.py:61-66
// forms the same value in int16 and casts it to int8), for the four nibble
// pairs in the low nibbles of q and r: the high nibble is q4 - [r4 < 0]
// (mod 16), the low nibble is r4's own. No carry crosses a byte (each sum is
// at most 30).
__device__ __forceinline__ uint32_t nested_r4(uint32_t q, uint32_t r) {
  const uint32_t qn = q & 0x0F0F0F0Fu, rn = r & 0x0F0F0F0Fu;
  const uint32_t neg = (rn >> 3) & 0x01010101u;
  return (((qn + neg * 15u) & 0x0F0F0F0Fu) << 4) | rn;
}

__device__ __forceinline__ v2u tr8(const uint8_t* p) {
  typedef int v2i_t __attribute__((ext_vector_type(2)));
  auto lp = (__attribute__((address_space(3))) v2i_t*)((__attribute__((address_space(3))) uint8_t*)p);
  const v2i_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(lp);
  return v2u{(uint32_t)r[0], (uint32_t)r[1]};
}

// 16-byte store to LDS at an address aligned to ALIGN bytes (16, 8 or 4)
template <int ALIGN>
__device__ __forceinline__ void lds_store16(uint8_t* p, const v4u& v) {
  if constexpr (ALIGN >= 16) {
    *reinterpret_cast<v4u*>(p) = v;
  } else if constexpr (ALIGN >= 8) {
    reinterpret_cast<v2u*>(p)[0] = v2u{v[0], v[1]};
    reinterpret_cast<v2u*>(p)[1] = v2u{v[2], v[3]};
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<uint32_t*>(p)[i] = v[i];
  }
}

constexpr int align_of_stride(int s) { return s % 16 == 0 ? 16 : (s % 8 == 0 ? 8 : 4); }

// Small-M tokenwise GEMM. WM waves along M (1 or 2), the rest along N; each
// wave owns MT x NT 16x16 output tiles. Workgroup tile: TM = 16 MT WM rows,
// TN = 16 NT (4/WM) columns. Grid: x = column tiles, y = row tiles, z = K
// splits (each split writes its int32 partial sums; tw_reduce adds them and
// finishes). A workgroup's whole K-range (at most NB K-steps: the host splits
// K until it is) is loaded at entry, every load in flight at once, staged into
// NB LDS buffers and computed after one barrier.
//
// XDT >= 0 (fused quantization, A8): the launch reads the rows x of dtype
// XDT instead of codes; XR = 1 takes one row, XR = 8 two to eight rows of
// 16-bit x. Every workgroup loads the whole rows for their amax (first, so
// that the in-order memory counter lets the amax finish before the weights
// land), then its K-range of x, then its weights; it computes each row's
// scale s = fl(max(amax, 1e-8) * fl(1/127)) and the codes rint(v / s)
// clamped to [-128, 127] exactly as tw_quantize_kernel does, and stages the
// codes as the activation tile. The first workgroup writes the scales to
// args.as (the integer reduce reads them).
template <int WL, int AL, int EPI, int WM, int MT, int NT, int NB, int XDT = -1, int XR = 1>
__global__ __launch_bounds__(kThreads) void tw_gemm(const TwArgs args_in) {
  const int target = (int)blockIdx.z / args_in.splits;
  const TwArgs args = for_target(args_in, target);
  using T = WTraits<WL>;
  constexpr int WN = 4 / WM;
  constexpr int TM = 16 * MT * WM, TN = 16 * NT * WN;
  constexpr int U = T::U;
  constexpr int WROWS = T::rows(TN), WRB = T::row_bytes(TN), WSTR = w_stride(WL, TN);
  constexpr int ARB = a_row_bytes(WL, AL), ASTR = a_stride(WL, AL);
  constexpr int WBUF = WROWS * WSTR, ABUF = TM * ASTR;
  constexpr int WCH = WROWS * WRB / 16, ACH = TM * ARB / 16;       // 16-byte chunks per step
  constexpr int NWC = (WCH + kThreads - 1) / kThreads, NAC = (ACH + kThreads - 1) / kThreads;
  constexpr int NBUF = NB;
  static_assert(NBUF * (WBUF + ABUF) <= 64 * 1024, "LDS tile buffers exceed 64 KiB");
  __shared__ __align__(16) uint8_t smem[NBUF * (WBUF + ABUF)];

  constexpr bool FX = XDT >= 0;
  static_assert(!FX || (AL == ACTUNE_TW_ACT_A8 && TM == 16 && T::KM), "fused quantization: A8, 16-row tiles");
  static_assert(XR == 1 || (XR == kTwFusedMaxRows && XDT != kF32), "fused rows: one, or up to 8 of 16-bit x");
  constexpr int XSZ = XDT == kF32 ? 4 : 2;  // bytes per x element
  constexpr int XRC = kTwFusedMaxK / (kThreads * 8);  // amax passes of 8 elements per thread

  const int M = args.M, N = args.N, K = args.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = (int)blockIdx.x * TN, m0 = (int)blockIdx.y * TM;
  const int S = args.splits, z = (int)blockIdx.z % S;
  const int g0 = (int)((long)z * args.steps / S), g1 = (int)((long)(z + 1) * args.steps / S);

  // buffer resources: reads past the end return zeros
  uint32_t wbytes;
  if constexpr (WL == ACTUNE_TW_KMAJOR_W8) wbytes = (uint32_t)K * N;
  else if constexpr (nibble_pairs(WL)) wbytes = (uint32_t)(K / 2) * N;
  else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) wbytes = (uint32_t)(K / 4) * N;
  else if constexpr (WL == ACTUNE_TW_ROWS_S4) wbytes = (uint32_t)N * (K / 2);
  else wbytes = (uint32_t)N * (K / 4);
  const uint32_t arow = AL == ACTUNE_TW_ACT_A4 ? (uint32_t)K / 2 : (uint32_t)K;
  const Rsrc wr = make_rsrc(args.w, wbytes);
  // the residual rows of W4R4 (a target without one reads zeros)
  const Rsrc rr = make_rsrc(args.r, args.r ? wbytes : 0u);
  constexpr bool R4 = WL == ACTUNE_TW_KMAJOR_W4R4;
  static_assert(!R4 || WCH == 2 * kThreads, "W4R4: load batch 0 holds the q4 rows, batch 1 the r4 rows");
  const Rsrc ar = FX ? make_rsrc(args.x, (uint32_t)M * K * XSZ) : make_rsrc(args.a, (uint32_t)M * arow);

  // Per-thread base offsets of its weight / activation chunks (step 0) and
  // the per-step byte strides, all 32-bit: a step's loads are then one add
  // each, in straight-line code. Chunks past the tile or the operand use
  // kOff (the load returns zeros and moves no data).
  uint32_t wbase[NWC], abase[NAC];
#pragma unroll
  for (int i = 0; i < NWC; ++i) {
    const int c = tid + i * kThreads, row = c / (WRB / 16), cb = c % (WRB / 16);
    bool live = c < WCH;
    if constexpr (T::KM) {
      live = live && n0 + 16 * cb < N;
      // W4R4: staged rows 32-63 are rows 0-31 of the residual buffer
      wbase[i] = live ? (uint32_t)(R4 ? row % 32 : row) * (uint32_t)N + (uint32_t)(n0 + 16 * cb) : kOff;
    } else {
      live = live && n0 + row < N;
      wbase[i] = live ? (uint32_t)(n0 + row) * (uint32_t)(WL == ACTUNE_TW_ROWS_S4 ? K / 2 : K / 4) + (uint32_t)(16 * cb)
                      : kOff;
    }
  }
  const uint32_t wstep = T::KM ? (uint32_t)(R4 ? WROWS / 2 : WROWS) * (uint32_t)N : (uint32_t)WRB;
#pragma unroll
  for (int i = 0; i < NAC; ++i) {
    const int c = tid + i * kThreads, row = c / (ARB / 16), cb = c % (ARB / 16);
    const bool live = c < ACH && m0 + row < M;
    uint32_t k;
    if constexpr (AL == ACTUNE_TW_ACT_A4) k = 16 * cb;                                   // packed row bytes
    else if constexpr (nibble_pairs(WL)) k = (uint32_t)(cb >> 1) * (K / 2) + 16 * (cb & 1);
    else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) k = (uint32_t)(cb >> 1) * (K / 4) + 16 * (cb & 1);
    else k = 16 * cb;
    // fused: byte offset of element k of the row (row 0 only)
    if constexpr (FX) abase[i] = live && row == 0 ? k * XSZ : kOff;
    else abase[i] = live ? (uint32_t)(m0 + row) * arow + k : kOff;
  }
  constexpr uint32_t astep = (AL == ACTUNE_TW_ACT_A4 || nibble_pairs(WL) || WL == ACTUNE_TW_KMAJOR_W2) ? 32 : 64;

  // loads of step g; a step outside [g0, g1) is switched off through the
  // scalar offset (reads zeros)
  auto issue = [&](int g, v4u (&wreg)[NWC], v4u (&areg)[NAC]) {
    const uint32_t soff = g < g1 ? 0u : kOff;
#pragma unroll
    for (int i = 0; i < NWC; ++i)
      wreg[i] = __builtin_amdgcn_raw_buffer_load_b128(R4 && i >= NWC / 2 ? rr : wr,
                                                      wbase[i] == kOff ? kOff : wbase[i] + (uint32_t)g * wstep, soff, 0);
#pragma unroll
    for (int i = 0; i < NAC; ++i)
      areg[i] = __builtin_amdgcn_raw_buffer_load_b128(ar, abase[i] == kOff ? kOff : abase[i] + (uint32_t)g * astep, soff, 0);
  };
  auto stage_w = [&](int buf, const v4u (&wreg)[NWC]) {
    uint8_t* wt = smem + buf * (WBUF + ABUF);
#pragma unroll
    for (int i = 0; i < NWC; ++i) {
      const int c = tid + i * kThreads;
      if (WCH % kThreads == 0 || c < WCH)
        lds_store16<align_of_stride(WSTR)>(wt + (c / (WRB / 16)) * WSTR + 16 * (c % (WRB / 16)), wreg[i]);
    }
  };
  auto stage = [&](int buf, const v4u (&wreg)[NWC], const v4u (&areg)[NAC]) {
    uint8_t* at = smem + buf * (WBUF + ABUF) + WBUF;
    stage_w(buf, wreg);
#pragma unroll
    for (int i = 0; i < NAC; ++i) {
      const int c = tid + i * kThreads;
      if (ACH % kThreads == 0 || c < ACH)
        lds_store16<align_of_stride(ASTR)>(at + (c / (ARB / 16)) * ASTR + 16 * (c % (ARB / 16)), areg[i]);
    }
  };

  v4i acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int r16 = lane & 15, kb = lane >> 4;
  // transposed-read lane address inside a 16-lane group: row i, half h
  const int tr_row = (lane & 15) >> 1, tr_half = lane & 1;

  auto compute = [&](int buf) {
    const uint8_t* wt = smem + buf * (WBUF + ABUF);
    const uint8_t* at = wt + WBUF;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t bf[NT][4];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int cn = wn * 16 * NT + nt * 16;
        if constexpr (WL == ACTUNE_TW_KMAJOR_W8) {
          const v2u lo = tr8(wt + (16 * kb + tr_row) * WSTR + cn + 8 * tr_half);
          const v2u hi = tr8(wt + (16 * kb + 8 + tr_row) * WSTR + cn + 8 * tr_half);
          bf[nt][0] = lo[0]; bf[nt][1] = lo[1]; bf[nt][2] = hi[0]; bf[nt][3] = hi[1];
        } else if constexpr (WL == ACTUNE_TW_KMAJOR_W4) {
          const v2u b = tr8(wt + (8 * kb + tr_row) * WSTR + cn + 8 * tr_half);
          bf[nt][0] = (b[0] << 4) & 0xF0F0F0F0u; bf[nt][1] = (b[1] << 4) & 0xF0F0F0F0u;
          bf[nt][2] = b[0] & 0xF0F0F0F0u;        bf[nt][3] = b[1] & 0xF0F0F0F0u;
        } else if constexpr (R4) {
          const v2u q = tr8(wt + (8 * kb + tr_row) * WSTR + cn + 8 * tr_half);
          const v2u r = tr8(wt + (32 + 8 * kb + tr_row) * WSTR + cn + 8 * tr_half);
          bf[nt][0] = nested_r4(q[0], r[0]); bf[nt][1] = nested_r4(q[1], r[1]);
          bf[nt][2] = nested_r4(q[0] >> 4, r[0] >> 4); bf[nt][3] = nested_r4(q[1] >> 4, r[1] >> 4);
        } else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) {
          const v2u b = tr8(wt + (8 * kb + tr_row) * WSTR + cn + 8 * tr_half);
          // fields 2u (k = j + 2u K/4) and 2u + 1 (k = j + (2u+1) K/4)
          const int s0 = 6 - 4 * u, s1 = 4 - 4 * u;  // u = 0: 6, 4; u = 1: 2, 0
          bf[nt][0] = (b[0] << s0) & 0xC0C0C0C0u;
          bf[nt][1] = (b[1] << s0) & 0xC0C0C0C0u;
          bf[nt][2] = (b[0] << s1) & 0xC0C0C0C0u;
          bf[nt][3] = (b[1] << s1) & 0xC0C0C0C0u;
        } else if constexpr (WL == ACTUNE_TW_ROWS_S4) {
          const v2u p = *reinterpret_cast<const v2u*>(wt + (cn + r16) * WSTR + 8 * kb);
          const uint32_t pp[2] = {p[0], p[1]};
          unpack_slot<4>(pp, bf[nt]);
        } else {
          const uint32_t p = *reinterpret_cast<const uint32_t*>(wt + (cn + r16) * WSTR + 4 * kb);
          unpack_slot<2>(&p, bf[nt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint8_t* arow_l = at + (wm * 16 * MT + mt * 16 + r16) * ASTR;
        uint32_t af[4];
        if constexpr (AL == ACTUNE_TW_ACT_A4) {
          const v2u p = *reinterpret_cast<const v2u*>(arow_l + 8 * kb);
          const uint32_t pp[2] = {p[0], p[1]};
          unpack_slot<4>(pp, af);
          if constexpr (WL == ACTUNE_TW_ROWS_S2) reorder_slot<4, 2>(af);
          else if constexpr (T::KM) reorder_slot<4, 8>(af);
        } else if constexpr (nibble_pairs(WL) || WL == ACTUNE_TW_KMAJOR_W2) {
          const v2u lo = *reinterpret_cast<const v2u*>(arow_l + 64 * u + 8 * kb);
          const v2u hi = *reinterpret_cast<const v2u*>(arow_l + 64 * u + 32 + 8 * kb);
          af[0] = lo[0]; af[1] = lo[1]; af[2] = hi[0]; af[3] = hi[1];
        } else {
          const v4u q = *reinterpret_cast<const v4u*>(arow_l + 16 * kb);
          af[0] = q[0]; af[1] = q[1]; af[2] = q[2]; af[3] = q[3];
          if constexpr (WL == ACTUNE_TW_ROWS_S4) reorder_slot<8, 4>(af);
          else if constexpr (WL == ACTUNE_TW_ROWS_S2) reorder_slot<8, 2>(af);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma16x16x64(af, bf[nt], acc[mt][nt]);
      }
    }
  };

  // every step of the K-range at once (steps past g1 load zeros and add
  // nothing, so the batch is straight-line code with no bounds tests)
  v4u wreg[NB][NWC], areg[NB][NAC];
  TwArgs fin = args;
  if constexpr (FX && XR > 1) {
    // rows padded to P (2, 4 or 8): thread t reads row t / (256 / P), 16
    // passes of 8 consecutive elements (the host keeps K <= 32768 / P)
    __shared__ float rp[2 * (kThreads / 64)];  // per wave: rows at lanes 0 and 32
    __shared__ float xsc[XR];                  // row scales for the epilogue
    const int lgt = M <= 2 ? 7 : M <= 4 ? 6 : 5;  // log2 threads per row
    const int xrow = tid >> lgt, xsub = tid & ((1 << lgt) - 1);
    v4u xq[kTwFusedRowPasses];
#pragma unroll
    for (int p = 0; p < kTwFusedRowPasses; ++p) {
      const int e = (p << (lgt + 3)) + xsub * 8;
      xq[p] = __builtin_amdgcn_raw_buffer_load_b128(ar, xrow < M && e < K ? ((uint32_t)xrow * K + e) * XSZ : kOff,
                                                    0, 0);
    }
    // this thread's EPT elements of every row at byte fb of staged step fi
    constexpr int EPT = NB * ARB / kThreads;
    static_assert(EPT == 1 || EPT == 2 || EPT == 4, "fused slice: 1, 2 or 4 elements per thread");
    const int fi = tid * EPT / ARB, fb = tid * EPT % ARB, fc = fb / 16;
    uint32_t kx;
    if constexpr (nibble_pairs(WL)) kx = (uint32_t)(fc >> 1) * (K / 2) + 16 * (fc & 1);
    else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) kx = (uint32_t)(fc >> 1) * (K / 4) + 16 * (fc & 1);
    else kx = 16 * fc;
    kx += (uint32_t)(fb % 16) + (uint32_t)(g0 + fi) * astep;
    uint32_t xsl[XR][EPT == 4 ? 2 : 1];
#pragma unroll
    for (int m = 0; m < XR; ++m) {
      const uint32_t off = m < M && g0 + fi < g1 ? ((uint32_t)m * K + kx) * XSZ : kOff;
      if constexpr (EPT == 4) {
        const v2u t = __builtin_amdgcn_raw_buffer_load_b64(ar, off, 0, 0);
        xsl[m][0] = t[0];
        xsl[m][1] = t[1];
      } else if constexpr (EPT == 2) {
        xsl[m][0] = __builtin_amdgcn_raw_buffer_load_b32(ar, off, 0, 0);
      } else {
        xsl[m][0] = __builtin_amdgcn_raw_buffer_load_b16(ar, off, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const uint32_t soff = g0 + i < g1 ? 0u : kOff;
#pragma unroll
      for (int c = 0; c < NWC; ++c)
        wreg[i][c] = __builtin_amdgcn_raw_buffer_load_b128(
            R4 && c >= NWC / 2 ? rr : wr, wbase[c] == kOff ? kOff : wbase[c] + (uint32_t)(g0 + i) * wstep, soff, 0);
    }
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < kTwFusedRowPasses; ++p) {
      float v8[8];
      unpack8<XDT>(xq[p], xq[p], v8);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v8[e]));
    }
    // the lanes of one row: 32 (P = 8) or the whole wave (P = 2, 4)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
      if (off < (1 << lgt)) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((lane & 31) == 0) rp[2 * wave + (lane >> 5)] = amax;
    __syncthreads();
    auto row_scale = [&](int m) {
      const float a = lgt == 5 ? rp[m] : lgt == 6 ? rp[2 * m] : fmaxf(rp[4 * m], rp[4 * m + 2]);
      return fmaxf(a, 1e-8f) * (1.0f / 127.0f);
    };
    if (tid < M) {
      const float sc = row_scale(tid);
      xsc[tid] = sc;
      if (blockIdx.x == 0 && blockIdx.z == 0) const_cast<float*>(args.as)[tid] = sc;
    }
    // the codes of rows 0 .. M-1 (rows past M are never stored; their
    // products are not written out)
#pragma unroll
    for (int m = 0; m < XR; ++m) {
      if (m < M) {
        const float sc = row_scale(m);
        uint32_t cw = 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const uint16_t h = (uint16_t)(xsl[m][e / 2] >> (16 * (e % 2)));
          const float v = XDT == kBF16 ? bf16_to_f32(h) : f16_to_f32(h);
          cw |= ((uint32_t)(int)fminf(fmaxf(rintf(v / sc), -128.0f), 127.0f) & 0xffu) << (8 * e);
        }
        uint8_t* dst = smem + fi * (WBUF + ABUF) + WBUF + m * ASTR + fb;
        if constexpr (EPT == 4) *reinterpret_cast<uint32_t*>(dst) = cw;
        else if constexpr (EPT == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)cw;
        else *dst = (uint8_t)cw;
      }
    }
    fin.as = xsc;  // the epilogue of an unsplit launch reads the scales from LDS
#pragma unroll
    for (int i = 0; i < NB; ++i) stage_w(i, wreg[i]);
  } else if constexpr (FX) {
    __shared__ float xs[kThreads / 64 + 1];
    // 1. the row for its amax, 2. this workgroup's K-range of x (EPT
    // consecutive elements per thread), 3. the weights
    float xm[XRC][8];
#pragma unroll
    for (int p = 0; p < XRC; ++p) {
      const int e = p * kThreads * 8 + tid * 8;
      buffer_load8<XDT>(ar, e < K ? (uint32_t)e * XSZ : kOff, xm[p]);
    }
    // thread tid: bytes b .. b + EPT - 1 of staged row 0 of step i (inside
    // one 16-byte chunk, so at consecutive k)
    constexpr int EPT = NB * ARB / kThreads;
    static_assert(EPT == 1 || EPT == 2 || EPT == 4, "fused slice: 1, 2 or 4 elements per thread");
    const int fi = tid * EPT / ARB, fb = tid * EPT % ARB, fc = fb / 16;
    uint32_t kx;
    if constexpr (nibble_pairs(WL)) kx = (uint32_t)(fc >> 1) * (K / 2) + 16 * (fc & 1);
    else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) kx = (uint32_t)(fc >> 1) * (K / 4) + 16 * (fc & 1);
    else kx = 16 * fc;
    kx += (uint32_t)(fb % 16) + (uint32_t)(g0 + fi) * astep;
    const uint32_t xoff = g0 + fi < g1 ? kx * XSZ : kOff;
    float xv[EPT];
    if constexpr (EPT * XSZ == 16) {
      const v4u q = __builtin_amdgcn_raw_buffer_load_b128(ar, xoff, 0, 0);
      if constexpr (XSZ == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = __uint_as_float(q[e]);
      } else {
        float v8[8];
        unpack8<XDT>(q, q, v8);
#pragma unroll
        for (int e = 0; e < EPT; ++e) xv[e] = v8[e];
      }
    } else {
      uint32_t q[2] = {0u, 0u};
      if constexpr (EPT * XSZ == 8) {
        const v2u t = __builtin_amdgcn_raw_buffer_load_b64(ar, xoff, 0, 0);
        q[0] = t[0]; q[1] = t[1];
      } else if constexpr (EPT * XSZ == 4) {
        q[0] = __builtin_amdgcn_raw_buffer_load_b32(ar, xoff, 0, 0);
      } else {
        q[0] = __builtin_amdgcn_raw_buffer_load_b16(ar, xoff, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if constexpr (XSZ == 4) xv[e] = __uint_as_float(q[e]);
        else {
          const uint16_t h = (uint16_t)(q[e / 2] >> (16 * (e % 2)));
          xv[e] = XDT == kBF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const uint32_t soff = g0 + i < g1 ? 0u : kOff;
#pragma unroll
      for (int c = 0; c < NWC; ++c)
        wreg[i][c] = __builtin_amdgcn_raw_buffer_load_b128(
            R4 && c >= NWC / 2 ? rr : wr, wbase[c] == kOff ? kOff : wbase[c] + (uint32_t)(g0 + i) * wstep, soff, 0);
    }
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < XRC; ++p)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xm[p][e]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (lane == 0) xs[wave] = amax;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) amax = fmaxf(amax, xs[w]);
    const float sc = fmaxf(amax, 1e-8f) * (1.0f / 127.0f);
    if (tid == 0) {
      xs[kThreads / 64] = sc;
      if (blockIdx.x == 0 && blockIdx.z == 0) const_cast<float*>(args.as)[0] = sc;
    }
    // this thread's codes into row 0 of step fi's activation tile (out of
    // range steps hold x = 0: code 0; rows 1-15 are never stored)
    uint32_t cw = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      cw |= ((uint32_t)(int)fminf(fmaxf(rintf(xv[e] / sc), -128.0f), 127.0f) & 0xffu) << (8 * e);
    uint8_t* dst = smem + fi * (WBUF + ABUF) + WBUF + fb;
    if constexpr (EPT == 4) *reinterpret_cast<uint32_t*>(dst) = cw;
    else if constexpr (EPT == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)cw;
    else *dst = (uint8_t)cw;
    fin.as = &xs[kThreads / 64];  // the epilogue of an unsplit launch reads s from LDS
#pragma unroll
    for (int i = 0; i < NB; ++i) stage_w(i, wreg[i]);
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i) issue(g0 + i, wreg[i], areg[i]);
#pragma unroll
    for (int i = 0; i < NB; ++i) stage(i, wreg[i], areg[i]);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NB; ++i) compute(i);

  finish_tile<WL, AL, EPI, MT, NT>(fin, acc, m0 + wm * 16 * MT + 4 * kb, n0 + wn * 16 * NT + r16, z);
}

// ------------------------------------------------------------ LDS-DMA ring
// buffer_load_dwordx4 ... lds writes lane l's 16 bytes at M0 + 16 l, and a
// lane whose offset is out of range writes zeros (both checked on MI355X).
// It is issued from inline asm so that the compiler's wait-count tracking
// does not see it: the compiler treats every LDS read as possibly aliasing
// any DMA in flight and would wait for all of them (vmcnt(0)) before each
// read, which serialises the ring; the kernel instead waits for exactly the
// loads of the step it is about to read. The s_nop is the one wait state an
// SALU write of M0 needs before an LDS DMA.
__device__ __forceinline__ void dma16(Rsrc r, uint32_t m0, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(m0), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

// waits until at most N of this wave's vector memory operations are in flight
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Staged rows of RB bytes are not padded (a DMA block is 1 KiB of
// consecutive chunks); chunk c of row r sits at chunk c ^ swz(r), with
// swz(r) = (r / rows per 256 bytes) % chunks per row, so that the rows one
// 16-lane group reads (8 or 16 consecutive rows, 8- or 16-byte pieces) fall
// on distinct banks.
template <int RB>
__device__ __forceinline__ constexpr int swz(int r) {
  return (r / (RB >= 256 ? 1 : 256 / RB)) % (RB / 16);
}
template <int RB>
__device__ __forceinline__ constexpr int lds_pos(int r, int b) {
  return r * RB + 16 * ((b >> 4) ^ swz<RB>(r)) + (b & 15);
}

// Large-M tokenwise GEMM: the tile geometry of tw_gemm, with the K-steps
// staged through a ring of D LDS slots filled by DMA loads; a slot holds KS
// consecutive K-steps (one ring step). Every K-step of a workgroup is NI
// 1-KiB blocks (weights, then activations); wave w issues blocks w, w + 4,
// ... (IPW per wave, the surplus aimed at a per-wave junk KiB with offsets
// out of range). Ring step t + D - 1 is issued right after the barrier that
// opens the read of ring step t + 1, into the slot ring step t - 1 used, so
// up to D - 2 ring steps are in flight beyond the one being read, with no
// registers held for them. A lane's global offsets are fixed; the K-step
// advance is the scalar offset (out of range past the workgroup's K-range).
template <int WL, int AL, int EPI, int WM, int MT, int NT, int KS, int D>
__global__ __launch_bounds__(kThreads) void tw_gemm_ring(const TwArgs args_in) {
  const TwArgs args = for_target(args_in, (int)blockIdx.z / args_in.splits);
  using T = WTraits<WL>;
  constexpr int WN = 4 / WM;
  constexpr int TM = 16 * MT * WM, TN = 16 * NT * WN;
  constexpr int U = T::U;
  constexpr int WROWS = T::rows(TN), WRB = T::row_bytes(TN), ARB = a_row_bytes(WL, AL);
  constexpr int WB = WROWS * WRB, AB = TM * ARB, SUB = WB + AB, SLOT = KS * SUB;
  static_assert(WB % 1024 == 0 && AB % 1024 == 0, "tiles are whole 1-KiB DMA blocks");
  constexpr int NWI = WB / 1024, NI = NWI + AB / 1024, IPW = (NI + 3) / 4;
  static_assert(D >= 3 && (D - 2) * KS * IPW <= 63, "ring depth");
  extern __shared__ __align__(16) uint8_t tw_ring[];

  const int M = args.M, N = args.N, K = args.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = (int)blockIdx.x * TN, m0 = (int)blockIdx.y * TM;
  const int z = (int)blockIdx.z % args.splits;
  const int g0 = (int)((long)z * args.steps / args.splits), g1 = (int)((long)(z + 1) * args.steps / args.splits);

  uint32_t wbytes;
  if constexpr (WL == ACTUNE_TW_KMAJOR_W8) wbytes = (uint32_t)K * N;
  else if constexpr (WL == ACTUNE_TW_KMAJOR_W4) wbytes = (uint32_t)(K / 2) * N;
  else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) wbytes = (uint32_t)(K / 4) * N;
  else if constexpr (WL == ACTUNE_TW_ROWS_S4) wbytes = (uint32_t)N * (K / 2);
  else wbytes = (uint32_t)N * (K / 4);
  const uint32_t arow = AL == ACTUNE_TW_ACT_A4 ? (uint32_t)K / 2 : (uint32_t)K;
  const Rsrc wr = make_rsrc(args.w, wbytes);
  const Rsrc ar = make_rsrc(args.a, (uint32_t)M * arow);
  const uint32_t wstep = T::KM ? (uint32_t)WROWS * (uint32_t)N : (uint32_t)WRB;
  constexpr uint32_t astep = (AL == ACTUNE_TW_ACT_A4 || WL == ACTUNE_TW_KMAJOR_W4 || WL == ACTUNE_TW_KMAJOR_W2) ? 32 : 64;

  // block j of this wave: lane offset (step 0), scalar step stride, LDS
  // offset inside a slot (or of the junk KiB), weight or activation buffer
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)tw_ring;
  uint32_t voff[IPW], sstep[IPW], lofs[IPW];
  bool isw[IPW], junk[IPW];
#pragma unroll
  for (int j = 0; j < IPW; ++j) {
    const int b = 4 * j + wave;
    isw[j] = b < NWI;
    junk[j] = b >= NI;
    if (b < NWI) {
      constexpr int SW = WRB / 16;
      const int p = 64 * b + lane, r = p / SW, c = (p % SW) ^ swz<WRB>(r);
      bool live;
      uint32_t off;
      if constexpr (T::KM) {
        live = n0 + 16 * c < N;
        off = (uint32_t)r * (uint32_t)N + (uint32_t)(n0 + 16 * c);
      } else {
        live = n0 + r < N;
        off = (uint32_t)(n0 + r) * (uint32_t)(WL == ACTUNE_TW_ROWS_S4 ? K / 2 : K / 4) + (uint32_t)(16 * c);
      }
      voff[j] = live ? off : kOff;
      sstep[j] = wstep;
      lofs[j] = (uint32_t)(1024 * b);
    } else if (b < NI) {
      constexpr int SA = ARB / 16;
      const int p = 64 * (b - NWI) + lane, r = p / SA, c = (p % SA) ^ swz<ARB>(r);
      uint32_t k;
      if constexpr (AL == ACTUNE_TW_ACT_A4) k = 16 * c;
      else if constexpr (WL == ACTUNE_TW_KMAJOR_W4) k = (uint32_t)(c >> 1) * (K / 2) + 16 * (c & 1);
      else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) k = (uint32_t)(c >> 1) * (K / 4) + 16 * (c & 1);
      else k = 16 * c;
      voff[j] = m0 + r < M ? (uint32_t)(m0 + r) * arow + k : kOff;
      sstep[j] = astep;
      lofs[j] = (uint32_t)(WB + 1024 * (b - NWI));
    } else {
      voff[j] = kOff;
      sstep[j] = 0;
      lofs[j] = (uint32_t)(D * SLOT + 1024 * wave);
    }
    // uniform per wave; readfirstlane keeps it in a scalar register
    lofs[j] = __builtin_amdgcn_readfirstlane(lds0 + lofs[j]);
  }
  // ring step t: K-steps g0 + KS t + q (q < KS) into sub-slot q of `slot`
  auto issue = [&](int t, int slot) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      const int g = g0 + KS * t + q;
#pragma unroll
      for (int j = 0; j < IPW; ++j) {
        const uint32_t m0v = lofs[j] + (junk[j] ? 0u : (uint32_t)(slot * SLOT + q * SUB));
        const uint32_t soff = g < g1 && !junk[j] ? (uint32_t)g * sstep[j] : kOff;
        dma16(isw[j] ? wr : ar, __builtin_amdgcn_readfirstlane(m0v), voff[j], __builtin_amdgcn_readfirstlane(soff));
      }
    }
  };

  // per-lane LDS read offsets inside a slot (step-invariant)
  const int r16 = lane & 15, kb = lane >> 4;
  const int tr_row = (lane & 15) >> 1, tr_half = lane & 1;
  int wofs[NT][2], aofs[MT][U][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int cn = wn * 16 * NT + nt * 16;
    if constexpr (WL == ACTUNE_TW_KMAJOR_W8) {
      wofs[nt][0] = lds_pos<WRB>(16 * kb + tr_row, cn + 8 * tr_half);
      wofs[nt][1] = lds_pos<WRB>(16 * kb + 8 + tr_row, cn + 8 * tr_half);
    } else if constexpr (T::KM) {
      wofs[nt][0] = wofs[nt][1] = lds_pos<WRB>(8 * kb + tr_row, cn + 8 * tr_half);
    } else if constexpr (WL == ACTUNE_TW_ROWS_S4) {
      wofs[nt][0] = wofs[nt][1] = lds_pos<WRB>(cn + r16, 8 * kb);
    } else {
      wofs[nt][0] = wofs[nt][1] = lds_pos<WRB>(cn + r16, 4 * kb);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = wm * 16 * MT + mt * 16 + r16;
      if constexpr (AL == ACTUNE_TW_ACT_A4) {
        aofs[mt][u][0] = aofs[mt][u][1] = WB + lds_pos<ARB>(row, 8 * kb);
      } else if constexpr (WL == ACTUNE_TW_KMAJOR_W4 || WL == ACTUNE_TW_KMAJOR_W2) {
        // k = j.. and the paired range: bytes 64 u + 8 kb and 64 u + 32 + 8 kb
        aofs[mt][u][0] = WB + lds_pos<ARB>(row, 64 * u + 8 * kb);
        aofs[mt][u][1] = WB + lds_pos<ARB>(row, 64 * u + 32 + 8 * kb);
      } else {
        aofs[mt][u][0] = aofs[mt][u][1] = WB + lds_pos<ARB>(row, 16 * kb);
      }
    }

  v4i acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // one step's operand fragments as read from LDS (weights still packed)
  struct Frag {
    v2u w[KS][U][NT][2];
    v2u a[KS][U][MT][2];
  };
  auto read = [&](int slot, Frag& f) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      const uint8_t* base = tw_ring + slot * SLOT + q * SUB;
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (WL == ACTUNE_TW_KMAJOR_W8) {
            f.w[q][u][nt][0] = tr8(base + wofs[nt][0]);
            f.w[q][u][nt][1] = tr8(base + wofs[nt][1]);
          } else if constexpr (T::KM) {
            if (u == 0) f.w[q][u][nt][0] = tr8(base + wofs[nt][0]);
          } else if constexpr (WL == ACTUNE_TW_ROWS_S4) {
            f.w[q][u][nt][0] = *reinterpret_cast<const v2u*>(base + wofs[nt][0]);
          } else {
            f.w[q][u][nt][0] = v2u{*reinterpret_cast<const uint32_t*>(base + wofs[nt][0]), 0u};
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (AL == ACTUNE_TW_ACT_A4) {
            f.a[q][u][mt][0] = *reinterpret_cast<const v2u*>(base + aofs[mt][u][0]);
          } else if constexpr (WL == ACTUNE_TW_KMAJOR_W4 || WL == ACTUNE_TW_KMAJOR_W2) {
            f.a[q][u][mt][0] = *reinterpret_cast<const v2u*>(base + aofs[mt][u][0]);
            f.a[q][u][mt][1] = *reinterpret_cast<const v2u*>(base + aofs[mt][u][1]);
          } else {
            const v4u v = *reinterpret_cast<const v4u*>(base + aofs[mt][u][0]);
            f.a[q][u][mt][0] = v2u{v[0], v[1]};
            f.a[q][u][mt][1] = v2u{v[2], v[3]};
          }
        }
      }
    }
  };
  // MFMAs in column-tile order: the unpack of tile nt + 1 can issue while
  // the MFMAs of tile nt run
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t af[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (AL == ACTUNE_TW_ACT_A4) {
            const uint32_t pp[2] = {f.a[q][u][mt][0][0], f.a[q][u][mt][0][1]};
            unpack_slot<4>(pp, af[mt]);
            if constexpr (WL == ACTUNE_TW_ROWS_S2) reorder_slot<4, 2>(af[mt]);
            else if constexpr (T::KM) reorder_slot<4, 8>(af[mt]);
          } else {
            af[mt][0] = f.a[q][u][mt][0][0]; af[mt][1] = f.a[q][u][mt][0][1];
            af[mt][2] = f.a[q][u][mt][1][0]; af[mt][3] = f.a[q][u][mt][1][1];
          }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          uint32_t bf[4];
          if constexpr (WL == ACTUNE_TW_KMAJOR_W8) {
            bf[0] = f.w[q][u][nt][0][0]; bf[1] = f.w[q][u][nt][0][1];
            bf[2] = f.w[q][u][nt][1][0]; bf[3] = f.w[q][u][nt][1][1];
          } else if constexpr (WL == ACTUNE_TW_KMAJOR_W4) {
            const v2u b = f.w[q][u][nt][0];
            bf[0] = (b[0] << 4) & 0xF0F0F0F0u; bf[1] = (b[1] << 4) & 0xF0F0F0F0u;
            bf[2] = b[0] & 0xF0F0F0F0u;        bf[3] = b[1] & 0xF0F0F0F0u;
          } else if constexpr (WL == ACTUNE_TW_KMAJOR_W2) {
            // fields 2u (k = j + 2u K/4) and 2u + 1 of the bytes read at u = 0
            const v2u b = f.w[q][0][nt][0];
            const int s0 = 6 - 4 * u, s1 = 4 - 4 * u;
            bf[0] = (b[0] << s0) & 0xC0C0C0C0u;
            bf[1] = (b[1] << s0) & 0xC0C0C0C0u;
            bf[2] = (b[0] << s1) & 0xC0C0C0C0u;
            bf[3] = (b[1] << s1) & 0xC0C0C0C0u;
          } else if constexpr (WL == ACTUNE_TW_ROWS_S4) {
            const uint32_t pp[2] = {f.w[q][u][nt][0][0], f.w[q][u][nt][0][1]};
            unpack_slot<4>(pp, bf);
          } else {
            const uint32_t pw = f.w[q][u][nt][0][0];
            unpack_slot<2>(&pw, bf);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16x16x64(af[mt], bf, acc[mt][nt]);
        }
      }
    }
  };
  // Step t's fragments are read from LDS one iteration ahead, so their LDS
  // latency hides behind step t - 1's MFMAs. The barrier that opens the
  // read of step t + 1 also tells every wave that step t - 1's slot (read
  // two iterations ago) is free for the DMA of step t + D - 1.
  const int nsteps = (g1 - g0 + KS - 1) / KS;
#pragma unroll
  for (int i = 0; i < D - 1; ++i) issue(i, i);
  Frag f0, f1;
  int rs = 1, ls = D - 1;  // slot read next, slot loaded next
  auto advance = [&]() {
    rs = rs == D - 1 ? 0 : rs + 1;
    ls = ls == D - 1 ? 0 : ls + 1;
  };
  if (nsteps > 0) {
    wait_vmem<(D - 2) * KS * IPW>();
    __syncthreads();
    read(0, f0);
  }
  // Two steps per trip, each with a next step to read. The trip has no
  // branch between a read and the MFMAs after it, so the compiler's
  // wait-count merge at a join cannot make step t's MFMAs wait for the
  // reads of step t + 1.
  int t = 0;
  for (; t + 2 < nsteps; t += 2) {
    wait_vmem<(D - 3) * KS * IPW>();
    __syncthreads();
    issue(t + D - 1, ls);
    read(rs, f1);
    advance();
    mma(f0);
    wait_vmem<(D - 3) * KS * IPW>();
    __syncthreads();
    issue(t + D, ls);
    read(rs, f0);
    advance();
    mma(f1);
  }
  // the last one or two steps (every later step was issued as out of range)
  if (t + 1 < nsteps) {
    wait_vmem<(D - 3) * KS * IPW>();
    __syncthreads();
    read(rs, f1);
    mma(f0);
    mma(f1);
  } else if (t < nsteps) {
    mma(f0);
  }
  // no DMA may still be writing this workgroup's LDS when it ends
  wait_vmem<0>();
  finish_tile<WL, AL, EPI, MT, NT>(args, acc, m0 + wm * 16 * MT + 4 * kb, n0 + wn * 16 * NT + r16, z);
}

// Adds the K splits' partial sums and finishes the outputs of target
// blockIdx.z: a thread takes CPT consecutive columns (1 or 4) of row
// blockIdx.y (+ gridDim.y ...), with
// all of up to NS splits' loads in flight at once (one round trip; more
// splits loop by NS). The partials of split s sit at s * M * N + m * N + n.
// With four columns and N a multiple of 4 (16-byte aligned quads) each split
// is one 16-byte load, otherwise one 4-byte load per column; columns past N
// are loaded as zeros and not stored.
template <int EPI, int NS, int CPT>
__global__ __launch_bounds__(kThreads) void tw_reduce(const TwArgs args_in, int shift) {
  const TwArgs args = for_target(args_in, (int)blockIdx.z);
  static_assert(CPT == 1 || CPT == 4, "one or four columns per thread");
  const int M = args.M, N = args.N, S = args.splits;
  const int n0 = CPT * ((int)blockIdx.x * kThreads + (int)threadIdx.x);
  if (n0 >= N) return;
  const uint32_t total = (uint32_t)M * (uint32_t)N;
  const Rsrc pr = make_rsrc(args.partial, (uint32_t)S * total * 4u);
  const bool quads = CPT == 4 && (N & 3) == 0;
  for (int m = (int)blockIdx.y; m < M; m += (int)gridDim.y) {
    const uint32_t base = (uint32_t)m * (uint32_t)N + (uint32_t)n0;
    int32_t sum[CPT] = {};
    for (int s0 = 0; s0 < S; s0 += NS) {
      int32_t v[NS][CPT];
      if (quads) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const v4u q = __builtin_amdgcn_raw_buffer_load_b128(
              pr, s0 + j < S ? ((uint32_t)(s0 + j) * total + base) * 4u : kOff, 0, 0);
#pragma unroll
          for (int r = 0; r < CPT; ++r) v[j][r] = (int32_t)q[r];
        }
      } else {
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
          for (int r = 0; r < CPT; ++r)
            v[j][r] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(
                pr, s0 + j < S && n0 + r < N ? ((uint32_t)(s0 + j) * total + base + (uint32_t)r) * 4u : kOff, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < NS; ++j)
#pragma unroll
        for (int r = 0; r < CPT; ++r) sum[r] += v[j][r];
    }
#pragma unroll
    for (int r = 0; r < CPT; ++r)
      if (n0 + r < N) store_result<EPI>(args, m, n0 + r, sum[r] >> shift);
  }
}

// ---------------------------------------------------------------- quantizer
// One workgroup per row: amax over the row (wave shuffles, then LDS across
// the 4 waves), s = fl(max(amax, f32(1e-8)) * fl(1/p)), codes rint(v / s)
// (IEEE division) clamped to [-p-1, p]. A8 writes int8 codes, A4 packs two
// codes per byte (low nibble = even k). Each lane owns 8 consecutive
// elements per 2048-element pass and keeps up to RC passes in registers
// between the amax and the code pass (K <= 2048 RC); longer rows re-read
// the rest (L2-resident).
template <int A, int DT>
__global__ __launch_bounds__(kThreads) void tw_quantize_kernel(const void* __restrict__ x, int K,
                                                               uint8_t* __restrict__ codes,
                                                               float* __restrict__ scales) {
  constexpr int P = (1 << (A - 1)) - 1;
  constexpr float R = 1.0f / (float)P;
  constexpr int ESZ = DT == kF32 ? 4 : 2;
  constexpr int RC = 8, PASS = kThreads * 8;
  __shared__ float red[kThreads / 64];
  const int m = blockIdx.x, tid = threadIdx.x;
  const char* row = static_cast<const char*>(x) + (size_t)m * K * ESZ;
  const Rsrc xr = make_rsrc(row, (uint32_t)K * ESZ);
  float v[RC][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < RC; ++p) {
    const int e = p * PASS + tid * 8;
    buffer_load8<DT>(xr, e < K ? (uint32_t)e * ESZ : kOff, v[p]);
  }
#pragma unroll
  for (int p = 0; p < RC; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[p][i]));
  for (int e = RC * PASS + tid * 8; e < K; e += PASS) {
    float w[8];
    load8<DT>(row, e, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(w[i]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(amax, 1e-8f) * R;
  if (tid == 0) scales[m] = s;
  auto emit = [&](int e, const float (&vv)[8]) {
    int c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = (int)fminf(fmaxf(rintf(vv[i] / s), (float)(-P - 1)), (float)P);
    if constexpr (A == 8) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) { lo |= ((uint32_t)c[i] & 0xffu) << (8 * i); hi |= ((uint32_t)c[4 + i] & 0xffu) << (8 * i); }
      *reinterpret_cast<v2u*>(codes + (size_t)m * K + e) = v2u{lo, hi};
    } else {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) w |= ((uint32_t)c[i] & 0xfu) << (4 * i);
      *reinterpret_cast<uint32_t*>(codes + (size_t)m * (K / 2) + e / 2) = w;
    }
  };
#pragma unroll
  for (int p = 0; p < RC; ++p) {
    const int e = p * PASS + tid * 8;
    if (e < K) emit(e, v[p]);
  }
  for (int e = RC * PASS + tid * 8; e < K; e += PASS) {
    float w[8];
    load8<DT>(row, e, w);
    emit(e, w);
  }
}

// ---------------------------------------------------------------- host side
struct Geometry {
  int wm, mt, nt, ns;   // small M: ns K-steps loaded at entry
  int ks, d;            // large M: K-steps per ring slot, ring slots
  int tm() const { return 16 * mt * wm; }
  int tn() const { return 16 * nt * (4 / wm); }
};

int kps_of(int wl) { return wl == ACTUNE_TW_KMAJOR_W2 ? 128 : 64; }
int64_t steps_of(int64_t K, int wl) { return (K + kps_of(wl) - 1) / kps_of(wl); }
// K-steps a small-M workgroup loads at entry: the int8 K-major tile is twice
// the others, so it keeps half as many steps to stay inside the LDS
int small_ns(int wl) { return wl == ACTUNE_TW_KMAJOR_W8 || wl == ACTUNE_TW_KMAJOR_W4R4 ? 4 : 8; }
int64_t tiles_of(int64_t M, int64_t N, const Geometry& g) {
  return ((N + g.tn() - 1) / g.tn()) * ((M + g.tm() - 1) / g.tm());
}

// M <= 32: 16-row x 128-column tiles, every K-step of a workgroup loaded at
// entry (small_ns; tw_gemm). Larger M: the LDS-DMA ring (tw_gemm_ring),
// chosen from measurements on MI355X at M = 512 over the Llama-2-7B shapes
// (six layout pairs): where the 64 x 128 grid holds at least 512 tiles (two or
// more workgroups per CU), 64 x 128 tiles with 3 slots of one K-step (two for
// the row-major S4 / S2 layouts), small enough in LDS for three workgroups
// per CU (W4A8 11008x4096: 60.8 -> 45.9 us); with fewer tiles, 4 slots of two
// K-steps, on 64 x 128 tiles for the K-major layouts and 64 x 64 tiles for S4
// / S2 (W4A8 4096x11008: 57.7 -> 51.2 us, W4A4 4096x4096: 30.4 -> 20.3 us).
Geometry pick_geometry(int64_t M, int64_t N, int wl) {
  if (M <= 32) return Geometry{1, 1, 2, small_ns(wl), 0, 0};
  const bool km = kmajor(wl);
  const Geometry big{2, 2, 4, 0, km ? 1 : 2, 3};
  if (tiles_of(M, N, big) >= 512) return big;
  return km ? Geometry{2, 2, 4, 0, 2, 4} : Geometry{2, 2, 2, 0, 2, 4};
}

// K splits. Small M: the fewest splits whose ranges fit a workgroup's entry
// loads (each workgroup then has the most bytes in flight, and the reduce
// the fewest partials). Measured on MI355X (W4A8, M = 1 and 8) against
// splitting further until the grid held 512 workgroups: 4096x4096 8.1 ->
// 7.6 us, 1024x4096 8.7 -> 6.7 us, 256x2048 6.9 -> 6.1 us, and with the rows
// quantized in the launch at M = 8, 4096x4096 10.6 -> 8.2 us; grids of 1024
// or 2048 workgroups were slower still. Large M: the
// split doubles while the grid holds fewer workgroups than CUs and the
// partials (S x M x N int32) stay within 8 MiB; below half a workgroup per
// CU each split keeps at least 4 K-steps, from there to one per CU at least
// 16. Measured on MI355X over the K-major layouts at M = 64-448 on the
// Llama-2-7B shapes, the second rule (a 128-workgroup grid split in two)
// takes M = 256 at N = 4096 from 27.7 to 23.2 us (K = 4096) and from 52.9
// to 33.9 us (K = 11008, W4A8), and M = 96-128 at K = 11008 by 19-32%;
// splitting to fewer than 16 K-steps lost up to 13%.
int pick_splits(int64_t M, int64_t N, int64_t K, int wl, const Geometry& g) {
  const int64_t tiles = tiles_of(M, N, g), steps = steps_of(K, wl);
  if (g.ns > 0) return (int)((steps + g.ns - 1) / g.ns);
  int64_t s = 1;
  while (tiles * s < 256 && s * (tiles * s < 128 ? 8 : 32) <= steps && 2 * s * M * N * 4 <= ((int64_t)8 << 20))
    s *= 2;
  return (int)s;
}

// The reduce of a split launch: loads per round trip sized to the splits;
// rows on grid y (at most 65535, more rows loop); four columns per thread
// only where that still leaves at least 256 workgroups (one per CU). Measured
// on MI355X (W4A8): four columns took M = 256 at N = 4096 from 23.1 to 20.4
// us (2 splits, K = 4096), while at M = 1 and 8 the 4-16 workgroups it left
// made the linear 0.4-1.1 us slower than one column per thread.
template <int EPI, int CPT>
void launch_reduce_c(const TwArgs& a, int shift, hipStream_t st) {
  const dim3 grid((unsigned)((a.N + CPT * kThreads - 1) / (CPT * kThreads)), (unsigned)std::min(a.M, 65535),
                  (unsigned)a.targets);
  if (a.splits <= 2) tw_reduce<EPI, 2, CPT><<<grid, kThreads, 0, st>>>(a, shift);
  else if (a.splits <= 4) tw_reduce<EPI, 4, CPT><<<grid, kThreads, 0, st>>>(a, shift);
  else if (a.splits <= 8) tw_reduce<EPI, 8, CPT><<<grid, kThreads, 0, st>>>(a, shift);
  else if (a.splits <= 16) tw_reduce<EPI, 16, CPT><<<grid, kThreads, 0, st>>>(a, shift);
  else if (a.splits <= 24) tw_reduce<EPI, 24, CPT><<<grid, kThreads, 0, st>>>(a, shift);
  else tw_reduce<EPI, 32, CPT><<<grid, kThreads, 0, st>>>(a, shift);
}

template <int EPI>
void launch_reduce(const TwArgs& a, int shift, hipStream_t st) {
  if ((int64_t)a.M * a.N >= (int64_t)4 * kThreads * 256) launch_reduce_c<EPI, 4>(a, shift, st);
  else launch_reduce_c<EPI, 1>(a, shift, st);
}

template <int WL, int AL, int EPI, int WM, int MT, int NT, int NB, int XDT = -1, int XR = 1>
void launch_gemm_t(const TwArgs& a, hipStream_t st) {
  constexpr int TM = 16 * MT * WM, TN = 16 * NT * (4 / WM);
  const dim3 grid((unsigned)((a.N + TN - 1) / TN), (unsigned)((a.M + TM - 1) / TM),
                  (unsigned)(a.splits * a.targets));
  tw_gemm<WL, AL, EPI, WM, MT, NT, NB, XDT, XR><<<grid, kThreads, 0, st>>>(a);
  if (a.splits > 1) launch_reduce<EPI>(a, WTraits<WL>::TW + (AL == ACTUNE_TW_ACT_A4 ? 4 : 0), st);
}

// LDS bytes of a tw_gemm_ring launch: D slots, and the junk KiB per wave when
// a step's blocks do not divide evenly over the four waves
template <int WL, int AL, int WM, int MT, int NT, int KS, int D>
constexpr size_t ring_lds_bytes() {
  constexpr int TM = 16 * MT * WM, TN = 16 * NT * (4 / WM);
  constexpr int SUB = WTraits<WL>::rows(TN) * WTraits<WL>::row_bytes(TN) + TM * a_row_bytes(WL, AL);
  return (size_t)D * KS * SUB + ((SUB / 1024) % 4 ? 4096 : 0);
}

template <int WL, int AL, int EPI, int WM, int MT, int NT, int KS, int D>
void launch_ring_t(const TwArgs& a, hipStream_t st) {
  constexpr int TM = 16 * MT * WM, TN = 16 * NT * (4 / WM);
  constexpr size_t lds = ring_lds_bytes<WL, AL, WM, MT, NT, KS, D>();
  static_assert(lds <= kStreamLdsMax, "ring exceeds the LDS budget");
  if constexpr (lds > 64 * 1024) allow_dynamic_lds<tw_gemm_ring<WL, AL, EPI, WM, MT, NT, KS, D>>();
  const dim3 grid((unsigned)((a.N + TN - 1) / TN), (unsigned)((a.M + TM - 1) / TM),
                  (unsigned)(a.splits * a.targets));
  tw_gemm_ring<WL, AL, EPI, WM, MT, NT, KS, D><<<grid, kThreads, lds, st>>>(a);
  if (a.splits > 1) launch_reduce<EPI>(a, WTraits<WL>::TW + (AL == ACTUNE_TW_ACT_A4 ? 4 : 0), st);
}

template <int WL, int AL, int EPI>
void launch_gemm_g(const TwArgs& a, const Geometry& g, hipStream_t st) {
  constexpr bool KM = WTraits<WL>::KM;
  if constexpr (WL == ACTUNE_TW_KMAJOR_W4R4) {  // small M only (the entry point checks M <= 32)
    launch_gemm_t<WL, AL, EPI, 1, 1, 2, 4>(a, st);
  } else {
    if (g.wm == 1) launch_gemm_t<WL, AL, EPI, 1, 1, 2, (WL == ACTUNE_TW_KMAJOR_W8 ? 4 : 8)>(a, st);
    else if (g.d == 3) launch_ring_t<WL, AL, EPI, 2, 2, 4, KM ? 1 : 2, 3>(a, st);
    else if constexpr (KM) launch_ring_t<WL, AL, EPI, 2, 2, 4, 2, 4>(a, st);
    else launch_ring_t<WL, AL, EPI, 2, 2, 2, 2, 4>(a, st);
  }
}

// A8 rows quantized inside the GEMM launch (small-M geometry, 16 x 128 tiles):
// one row, or two to eight rows of 16-bit x
template <int WL, int EPI, int XDT>
void launch_fused_t(const TwArgs& a, hipStream_t st) {
  constexpr int NB = WL == ACTUNE_TW_KMAJOR_W8 || WL == ACTUNE_TW_KMAJOR_W4R4 ? 4 : 8;
  if constexpr (XDT == kF32) {
    launch_gemm_t<WL, ACTUNE_TW_ACT_A8, EPI, 1, 1, 2, NB, XDT>(a, st);
  } else {
    if (a.M == 1) launch_gemm_t<WL, ACTUNE_TW_ACT_A8, EPI, 1, 1, 2, NB, XDT>(a, st);
    else launch_gemm_t<WL, ACTUNE_TW_ACT_A8, EPI, 1, 1, 2, NB, XDT, kTwFusedMaxRows>(a, st);
  }
}

void launch_fused(int wl, int epi, int xdt, const TwArgs& a, hipStream_t st) {
#define TWF(W_, E_)                                                      \
  if (wl == W_ && epi == E_) {                                           \
    if (xdt == kBF16) launch_fused_t<W_, E_, kBF16>(a, st);              \
    else if (xdt == kF16) launch_fused_t<W_, E_, kF16>(a, st);           \
    else launch_fused_t<W_, E_, kF32>(a, st);                            \
    return;                                                              \
  }
  TWF(ACTUNE_TW_KMAJOR_W8, ACTUNE_TW_EPI_A8) TWF(ACTUNE_TW_KMAJOR_W8, ACTUNE_TW_EPI_A4)
  TWF(ACTUNE_TW_KMAJOR_W4, ACTUNE_TW_EPI_A8) TWF(ACTUNE_TW_KMAJOR_W4, ACTUNE_TW_EPI_A4)
  TWF(ACTUNE_TW_KMAJOR_W2, ACTUNE_TW_EPI_A8) TWF(ACTUNE_TW_KMAJOR_W2, ACTUNE_TW_EPI_A4)
  TWF(ACTUNE_TW_KMAJOR_W4R4, ACTUNE_TW_EPI_A8) TWF(ACTUNE_TW_KMAJOR_W4R4, ACTUNE_TW_EPI_A4)
#undef TWF
}

// the six (weight layout, activation layout) pairs of the reference family
bool pair_ok(int wl, int al) {
  if (al == ACTUNE_TW_ACT_A8) return kmajor(wl);
  if (al == ACTUNE_TW_ACT_A4) return wl == ACTUNE_TW_KMAJOR_W8 || wl == ACTUNE_TW_ROWS_S4 || wl == ACTUNE_TW_ROWS_S2;
  return false;
}

void launch_gemm(int wl, int al, int epi, const TwArgs& a, const Geometry& g, hipStream_t st) {
#define TW_CASE(W_, A_)                                                            \
  if (wl == W_ && al == A_) {                                                      \
    if (epi == ACTUNE_TW_EPI_A8) launch_gemm_g<W_, A_, ACTUNE_TW_EPI_A8>(a, g, st); \
    else launch_gemm_g<W_, A_, ACTUNE_TW_EPI_A4>(a, g, st);                        \
    return;                                                                        \
  }
  TW_CASE(ACTUNE_TW_KMAJOR_W8, ACTUNE_TW_ACT_A8)
  TW_CASE(ACTUNE_TW_KMAJOR_W4, ACTUNE_TW_ACT_A8)
  TW_CASE(ACTUNE_TW_KMAJOR_W2, ACTUNE_TW_ACT_A8)
  TW_CASE(ACTUNE_TW_KMAJOR_W4R4, ACTUNE_TW_ACT_A8)
  TW_CASE(ACTUNE_TW_KMAJOR_W8, ACTUNE_TW_ACT_A4)
  TW_CASE(ACTUNE_TW_ROWS_S4, ACTUNE_TW_ACT_A4)
  TW_CASE(ACTUNE_TW_ROWS_S2, ACTUNE_TW_ACT_A4)
#undef TW_CASE
}

int fail(const char* msg) {
  set_last_error(msg);
  return ACTUNE_ERR_INVALID;
}

thread_local char g_tw_msg[128];

// Shape checks shared by the workspace query and the linear.
int check_tw_shape(int64_t M, int64_t N, int64_t K, int wl, int al) {
  if (!pair_ok(wl, al)) return fail("unsupported tokenwise weight/activation layout pair");
  if (M < 0 || N <= 0 || K <= 0) return fail("invalid dimensions");
  if (wl == ACTUNE_TW_KMAJOR_W4R4 && M > 32) return fail("the W4R4 layout takes up to 32 rows");
  if (K >= (1 << 17)) return fail("K must stay below 131072 (exact int32 accumulation)");
  const int kq = nibble_pairs(wl) ? 32 : (wl == ACTUNE_TW_KMAJOR_W2 ? 128 : 64);
  if (K % kq) {
    snprintf(g_tw_msg, sizeof g_tw_msg, "in_features must be divisible by %d for this layout", kq);
    return fail(g_tw_msg);
  }
  if (kmajor(wl) && N % 16) return fail("K-major weight layouts need out_features divisible by 16");
  if (N > INT_MAX / 2 || M > INT_MAX / 2 || M * K >= ((int64_t)1 << 31) || N * K >= ((int64_t)1 << 31) ||
      M * N * 4 >= ((int64_t)1 << 31))
    return fail("operand too large (each buffer must stay below 2 GiB)");
  return ACTUNE_OK;
}

}  // namespace
}  // namespace actune

using namespace actune;

extern "C" {

int actune_tokenwise_quantize(const void* x, int x_dtype, int64_t M, int64_t K, int A, void* codes,
                              float* scales, void* stream) {
  set_last_error("");
  if (A != 8 && A != 4) return fail("tokenwise activations are A8 or A4");
  if (x_dtype != kBF16 && x_dtype != kF16 && x_dtype != kF32) return fail("unsupported activation dtype");
  if (M < 0 || K <= 0 || K % 8) return fail("in_features must be a positive multiple of 8");
  if (M > INT_MAX || M * K >= ((int64_t)1 << 31)) return fail("activation too large");
  if (M == 0) return ACTUNE_OK;
  if (!x || !codes || !scales) return fail("null pointer");
  if (((uintptr_t)x % 16) || ((uintptr_t)codes % 8) || ((uintptr_t)scales % 4))
    return fail("misaligned operand (x needs 16 B, codes 8 B)");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)M);
  uint8_t* c = static_cast<uint8_t*>(codes);
#define TWQ(A_, DT_) tw_quantize_kernel<A_, DT_><<<grid, kThreads, 0, st>>>(x, (int)K, c, scales)
  if (A == 8) {
    if (x_dtype == kBF16) TWQ(8, kBF16); else if (x_dtype == kF16) TWQ(8, kF16); else TWQ(8, kF32);
  } else {
    if (x_dtype == kBF16) TWQ(4, kBF16); else if (x_dtype == kF16) TWQ(4, kF16); else TWQ(4, kF32);
  }
#undef TWQ
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error(hipGetErrorString(e));
    return ACTUNE_ERR_DEVICE;
  }
  return ACTUNE_OK;
}

int64_t actune_tokenwise_workspace_bytes(int64_t M, int64_t N, int64_t K, int w_layout, int a_layout) {
  if (check_tw_shape(M, N, K, w_layout, a_layout)) return -1;
  const Geometry g = pick_geometry(M, N, w_layout);
  const int S = pick_splits(M, N, K, w_layout, g);
  return S == 1 ? 0 : (int64_t)S * M * N * 4;
}

}  // extern "C"

namespace actune {
namespace {

// Checks shared by the two linear entry points and the launch arguments;
// act is the codes (a) or the row (x) pointer, checked for 16-byte alignment.
int prepare_linear(TwArgs& args, const void* act, int a_layout, const float* a_scales, const void* w, int w_layout,
                   const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype, int64_t M,
                   int64_t N, int64_t K, int epilogue, void* workspace, int64_t workspace_bytes) {
  int rc = check_tw_shape(M, N, K, w_layout, a_layout);
  if (rc) return rc;
  if (epilogue != ACTUNE_TW_EPI_A8 && epilogue != ACTUNE_TW_EPI_A4) return fail("unknown epilogue");
  if ((bias && bias_dtype != kBF16 && bias_dtype != kF16 && bias_dtype != kF32) ||
      (out_dtype != kBF16 && out_dtype != kF16 && out_dtype != kF32))
    return fail("unsupported output/bias dtype");
  if (M == 0) return ACTUNE_OK;
  if (!act || !a_scales || !w || !w_scale || !out) return fail("null pointer");
  if (((uintptr_t)act % 16) || ((uintptr_t)w % 16) || ((uintptr_t)a_scales % 4) || ((uintptr_t)w_scale % 4))
    return fail("misaligned operand (packed data needs 16 B)");
  const Geometry g = pick_geometry(M, N, w_layout);
  const int S = pick_splits(M, N, K, w_layout, g);
  args = TwArgs{};
  args.as = a_scales;
  args.w = static_cast<const uint8_t*>(w);
  args.ws = w_scale;
  args.bias = bias;
  args.out = out;
  args.M = (int)M;
  args.N = (int)N;
  args.K = (int)K;
  args.bias_dt = bias_dtype;
  args.out_dt = out_dtype;
  args.splits = S;
  args.steps = (int)steps_of(K, w_layout);
  args.targets = 1;
  args.r = nullptr;
  args.ws_mul = w_layout == ACTUNE_TW_KMAJOR_W4R4 ? 0.0625f : 1.0f;
  if (S > 1) {
    const int64_t need = (int64_t)S * M * N * 4;
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 16))
      return fail("workspace missing, misaligned or smaller than actune_tokenwise_workspace_bytes()");
    if (need >= ((int64_t)1 << 31)) return fail("split-K partials too large");
    args.partial = static_cast<int32_t*>(workspace);
  }
  return ACTUNE_OK;
}

// Checks of a launch that quantizes the rows x itself.
int check_fused(int x_dtype, int w_layout, int64_t M, int64_t K) {
  if (x_dtype != kBF16 && x_dtype != kF16 && x_dtype != kF32) return fail("unsupported activation dtype");
  if (!kmajor(w_layout)) return fail("fused quantization takes the K-major (A8) weight layouts");
  if (M < 1 || M > kTwFusedMaxRows) return fail("fused quantization takes 1 to 8 rows");
  if (M > 1 && x_dtype == kF32) return fail("fused quantization of more than one row takes bf16 or f16 x");
  if (K > tw_fused_max_k(M)) {
    snprintf(g_tw_msg, sizeof g_tw_msg, "fused quantization takes in_features <= %d at M = %d",
             (int)tw_fused_max_k(M), (int)M);
    return fail(g_tw_msg);
  }
  return ACTUNE_OK;
}

int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error(hipGetErrorString(e));
    return ACTUNE_ERR_DEVICE;
  }
  return ACTUNE_OK;
}

}  // namespace
}  // namespace actune

extern "C" {

int actune_tokenwise_linear(const void* a, int a_layout, const float* a_scales, const void* w, int w_layout,
                            const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                            int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  set_last_error("");
  if (w_layout == ACTUNE_TW_KMAJOR_W4R4) return fail("the W4R4 layout takes a residual: use actune_tokenwise_linear_multi");
  TwArgs args;
  const int rc = prepare_linear(args, a, a_layout, a_scales, w, w_layout, w_scale, bias, bias_dtype, out, out_dtype,
                                M, N, K, epilogue, workspace, workspace_bytes);
  if (rc || M == 0) return rc;
  args.a = static_cast<const uint8_t*>(a);
  launch_gemm(w_layout, a_layout, epilogue, args, pick_geometry(M, N, w_layout), (hipStream_t)stream);
  return launch_status();
}

int actune_tokenwise_linear_x(const void* x, int x_dtype, float* a_scales, const void* w, int w_layout,
                              const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                              int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  set_last_error("");
  if (w_layout == ACTUNE_TW_KMAJOR_W4R4) return fail("the W4R4 layout takes a residual: use actune_tokenwise_linear_multi");
  const int rc = check_fused(x_dtype, w_layout, M, K);
  if (rc) return rc;
  TwArgs args;
  const int rc2 = prepare_linear(args, x, ACTUNE_TW_ACT_A8, a_scales, w, w_layout, w_scale, bias, bias_dtype, out,
                                 out_dtype, M, N, K, epilogue, workspace, workspace_bytes);
  if (rc2) return rc2;
  args.x = x;
  launch_fused(w_layout, epilogue, x_dtype, args, (hipStream_t)stream);
  return launch_status();
}

int actune_tokenwise_linear_multi(const void* a, int a_layout, const void* x, int x_dtype, float* a_scales,
                                  int w_layout, const actune_tw_target* targets, int ntargets, int bias_dtype,
                                  int out_dtype, int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  set_last_error("");
  if ((a == nullptr) == (x == nullptr)) return fail("pass either activation codes or activation rows");
  if (ntargets < 1 || ntargets > ACTUNE_MAX_TARGETS) return fail("1 to ACTUNE_MAX_TARGETS targets");
  if (!targets) return fail("null pointer");
  if (w_layout == ACTUNE_TW_KMAJOR_W4R4)
    for (int i = 0; i < ntargets; ++i)
      if ((uintptr_t)targets[i].r % 16) return fail("misaligned residual (packed data needs 16 B)");
  if (x) {
    const int rc = check_fused(x_dtype, w_layout, M, K);
    if (rc) return rc;
    a_layout = ACTUNE_TW_ACT_A8;
  }
  // every target is checked as a single call would be; the splits and the
  // per-target partial size do not depend on the target
  const int64_t per = actune_tokenwise_workspace_bytes(M, N, K, w_layout, a_layout);
  if (per < 0) return ACTUNE_ERR_INVALID;
  TwArgs args;
  for (int i = ntargets - 1; i >= 0; --i) {
    const actune_tw_target& t = targets[i];
    const int rc = prepare_linear(args, x ? x : a, a_layout, a_scales, t.w, w_layout, t.w_scale, t.bias, bias_dtype,
                                  t.out, out_dtype, M, N, K, epilogue, per ? workspace : nullptr, per);
    if (rc) return rc;
  }
  if (M == 0) return ACTUNE_OK;
  if (per && (int64_t)ntargets * per > workspace_bytes)
    return fail("workspace missing, misaligned or smaller than ntargets x actune_tokenwise_workspace_bytes()");
  args.targets = ntargets;
  const bool r4 = w_layout == ACTUNE_TW_KMAJOR_W4R4;
  for (int i = 0; i < ntargets; ++i)
    args.t[i] = TwTarget{static_cast<const uint8_t*>(targets[i].w),
                         r4 ? static_cast<const uint8_t*>(targets[i].r) : nullptr, targets[i].w_scale,
                         targets[i].bias, targets[i].out};
  args.r = args.t[0].r;
  hipStream_t st = (hipStream_t)stream;
  if (x) {
    args.x = x;
    launch_fused(w_layout, epilogue, x_dtype, args, st);
  } else {
    args.a = static_cast<const uint8_t*>(a);
    launch_gemm(w_layout, a_layout, epilogue, args, pick_geometry(M, N, w_layout), st);
  }
  return launch_status();
}

}  // extern "C"
