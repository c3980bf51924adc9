// fp8-MFMA prefill GEMM for gfx950, W and A of at most 4 bits: the same
// group-64 arithmetic as gemm_prefill (actune/kernels/grouped_native.cu:42-88
// and grouped_big_m.cu:42-90 for W, A <= 4; canonical chunked fp32 order of
// common.hpp), bit for bit, on v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Why fp8. The int8 MFMA returns int32 dots, so each (token, channel, group)
// costs v_cvt_f32_i32 + fma; an fp8 MFMA over exactly represented codes
// returns the dot already in fp32, so the rescale is one fma. Measured
// register-resident ceilings on MI355X: 38-40% of the int8 peak against
// 28-29% for the int8 loop (bench `ceilings`).
//
// Exact fp8 operands. e4m3 bytes 0..15 encode p * 2^-9 (the subnormal and
// first normal binade are one linear range), bit 7 the sign; with the
// instruction's E8M0 block scale 2^9 on both operands every product is an
// exact integer and every partial sum an integer below 2^24:
//  * weights are offset binary: byte c + 8 for a code c (3 VALU per packed
//    dword for W4: (x ^ 0x88888888) & 0x0F0F0F0F and the same for x >> 4);
//  * activations are sign-magnitude bytes written by the quantizer's fp8
//    mode (launch_quantize_f8), in the element order the weights unpack to;
//  * the offset o (8 for W4, 2 for W2) adds o * sum_k a_k per (token,
//    group); a second MFMA of the constant -o against the same activation
//    fragment yields -o * sum_k a_k at every output position of that token,
//    and feeds the main MFMA's C: D = sum_k (c_w + o) a_k - o sum_k a_k = the
//    exact dot.
//
// Structure. A workgroup is 4 waves over a 64-channel x 64-token tile, wave w
// taking the 32 x 32 sub-tile (channels w & 1, tokens w >> 1). The MFMA's A
// operand is 32 weight rows (lane l: row l % 32, K-half l / 32, 16 packed
// bytes per group for W4, 8 for W2), its B operand 32 tokens from LDS; lane l
// ends with token l % 32 and channels 8 (r / 4) + 4 (l / 32) + r % 4 of
// registers r = 0..15, so the per-group rescale uses one scale per lane.
// Activations are staged per stage of 4 groups (one quad) into
// double-buffered LDS rows of 256 bytes (16-byte chunks XOR-swizzled by
// row), one barrier per stage; weights run 2 stages ahead in registers. The
// MFMAs of group g are issued before the rescale of group g - 1. Tiles are
// dealt to the 8 XCDs as in gemm_prefill.
#include "common.hpp"
#include "launch.hpp"
#include "operands.hpp"

namespace actune {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kF8Xcds = 8;
constexpr int kF8BN = 64, kF8BM = 64, kF8KG = 4;      // workgroup tile, groups per stage
constexpr int kF8Row = kF8KG * kGroup;                 // LDS bytes per token row of a stage
constexpr int kF8ABytes = kF8BM * kF8Row;              // activation bytes per stage
constexpr int kF8SBytes = kF8KG * kF8BM * 4;           // scales per stage
constexpr int kF8Scale = 127 + 9;                      // E8M0 block scale 2^9

// LDS offset of 16-byte chunk c (0..15) of token row `row` of a stage
__device__ __forceinline__ int f8_chunk_addr(int row, int c) { return row * kF8Row + ((c ^ (row & 15)) << 4); }

// Offset-binary e4m3 bytes (c + 8, or c + 2 for W2) of one group's weight
// codes held by this lane (W4: 4 dwords = 32 codes; W2: 2 dwords), in the
// width's native element order (common.hpp): byte t of dword r holds code
// 8 (r / 2) + 2t + r % 2 (W4) or 16 (r / 4) + 4t + r % 4 (W2).
template <int W>
__device__ __forceinline__ v8i f8_weights(const uint32_t (&x)[W == 4 ? 4 : 2]) {
  v8i w;
  if constexpr (W == 4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      w[2 * d] = (int)((x[d] ^ 0x88888888u) & 0x0F0F0F0Fu);
      w[2 * d + 1] = (int)(((x[d] >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu);
    }
  } else {
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * d + j] = (int)(((x[d] >> (2 * j)) ^ 0x02020202u) & 0x03030303u);
  }
  return w;
}

// CPS (one chunk per stage): with Q = ceil(G/4) <= kChunks every nonempty
// canonical chunk is one quad, i.e. one stage; its partial starts with
// p = d * s (== fmaf(d, s, +0)) and is added to acc when the stage ends.
template <int W, bool CPS>
__global__ __launch_bounds__(256) void gemm_prefill_f8(const LinearArgs args, int tiles_m) {
  constexpr int WD = W == 4 ? 4 : 2;  // packed weight dwords per lane per group
  constexpr int DW = 2;               // weight stages in flight
  __shared__ __align__(16) uint8_t alds[2][kF8ABytes + kF8SBytes];
  __shared__ float wsl[kF8BN], bsl[kF8BN];

  const int M = args.M, K = args.K, N = args.prob[0].N, G = K / kGroup;
  const int Qn = (G + kF8KG - 1) / kF8KG;  // stages (quads)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ct = wave & 1, tt = wave >> 1, half = lane >> 5, l32 = lane & 31;

  const int ntiles = (int)gridDim.x, id = (int)blockIdx.x;
  const int xcd = id % kF8Xcds, per = ntiles / kF8Xcds, rem = ntiles % kF8Xcds;
  const int tile = xcd * per + (xcd < rem ? xcd : rem) + id / kF8Xcds;
  const int n_blk = (tile / tiles_m) * kF8BN, m_blk = (tile % tiles_m) * kF8BM;

  for (int t = tid; t < kF8BN; t += 256) {
    const ChannelConst cc = fetch_channel(args.prob[0].ws, args.prob[0].bias, args.bias_dt, N, n_blk + t, true);
    wsl[t] = cc.ws;
    bsl[t] = bias_from_bits(cc.bias_bits, args.bias_dt);
  }

  // ---------------------------------------------------------------- loads
  const uint32_t wrow_bytes = (uint32_t)K * W / 8;
  const Rsrc wres = make_rsrc(args.prob[0].w, (uint32_t)N * wrow_bytes);
  const Rsrc ares = make_rsrc(args.a, (uint32_t)M * (uint32_t)K);
  const Rsrc sres = make_rsrc(args.as, (uint32_t)M * G * 4u);
  const int n_row = n_blk + ct * 32 + l32;
  // bytes past the row (tail stage) read the next row or zeros: their
  // activations are zero, so they add nothing
  const uint32_t wbase = n_row < N ? (uint32_t)n_row * wrow_bytes + (uint32_t)half * (W * 4) : kOff;
  uint32_t wring[DW][kF8KG][WD];
  auto load_weights = [&](int q, int gl, uint32_t (&dst)[WD]) {
    const uint32_t off = (uint32_t)(q * kF8KG + gl) * (uint32_t)(8 * W);
    if constexpr (W == 4) {
      const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wres, wbase + off, 0, 0);
      dst[0] = v[0]; dst[1] = v[1]; dst[2] = v[2]; dst[3] = v[3];
    } else {
      const v2u v = __builtin_amdgcn_raw_buffer_load_b64(wres, wbase + off, 0, 0);
      dst[0] = v[0]; dst[1] = v[1];
    }
  };
  // activation chunk j of this thread: token row (tid + 256 j) / 16, chunk
  // (tid + 256 j) % 16 of the stage's 256 bytes
  uint32_t abase[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ch = tid + 256 * j, row = ch >> 4, m = m_blk + row;
    abase[j] = m < M ? (uint32_t)m * (uint32_t)K + (uint32_t)(ch & 15) * 16u : kOff;
  }
  const int s_row = tid & 63, s_gl = tid >> 6;  // the scale this thread stages
  const uint32_t sbase = m_blk + s_row < M ? (uint32_t)(m_blk + s_row) * (uint32_t)G * 4u : kOff;
  v4u araw[4];
  float sraw;
  auto load_acts = [&](int q) {
    const uint32_t qoff = (uint32_t)q * kF8Row;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // chunks past K (tail stage) read zeros: their bytes would be the next
      // row's codes (or any byte, NaN included, past the last row)
      const bool inside = abase[j] != kOff && qoff + (uint32_t)((tid + 256 * j) & 15) * 16u < (uint32_t)K;
      araw[j] = __builtin_amdgcn_raw_buffer_load_b128(ares, inside ? abase[j] + qoff : kOff, 0, 0);
    }
    const int g = q * kF8KG + s_gl;
    const bool s_in = sbase != kOff && g < G;
    sraw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sres, s_in ? sbase + (uint32_t)g * 4u : kOff, 0, 0));
  };
  auto store_acts = [&](uint8_t* buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = tid + 256 * j;
      *reinterpret_cast<v4u*>(buf + f8_chunk_addr(ch >> 4, ch & 15)) = araw[j];
    }
    reinterpret_cast<float*>(buf + kF8ABytes)[s_gl * kF8BM + s_row] = sraw;
  };

  // ---------------------------------------------------------------- accumulators
  float acc[16], p[16];
  v16f D[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) { acc[r] = p[r] = 0.f; D[0][r] = D[1][r] = 0.f; }
  float s_prev = 0.f;  // scale of the group whose dots wait in D
  int c = 0, cend = chunk_begin(1, G);
  const v16f zero16 = {};
  // minus the weight code offset everywhere: -8 for W4 (byte 0x88 = -8 * 2^-9),
  // -2 for W2 (0x82)
  constexpr uint32_t kNegOffset = W == 4 ? 0x88888888u : 0x82828282u;
  v8i aconst;
#pragma unroll
  for (int j = 0; j < 8; ++j) aconst[j] = (int)kNegOffset;
  auto rescale = [&](int par, float s, bool first) {
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = first ? D[par][r] * s : __builtin_fmaf(D[par][r], s, p[r]);
  };
  auto close_chunk = [&]() {
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[r] = acc[r] + p[r]; p[r] = 0.f; }
    ++c;
    cend = chunk_begin(c + 1, G);
  };

  // ---------------------------------------------------------------- prologue
  load_acts(0);
#pragma unroll
  for (int v = 0; v < DW; ++v)
#pragma unroll
    for (int gl = 0; gl < kF8KG; ++gl) load_weights(v, gl, wring[v][gl]);
  store_acts(alds[0]);
  load_acts(1);
  __syncthreads();

  const int brow = tt * 32 + l32;  // this lane's token row in the tile
  for (int v0 = 0; v0 < Qn; v0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int q = v0 + u;
      if (q < Qn) {  // uniform
        const uint8_t* buf = alds[u];
        const float* sl = reinterpret_cast<const float*>(buf + kF8ABytes);
#pragma unroll
        for (int gl = 0; gl < kF8KG; ++gl) {
          const int g = q * kF8KG + gl;
          const v4u b0 = *reinterpret_cast<const v4u*>(buf + f8_chunk_addr(brow, gl * 4 + half * 2));
          const v4u b1 = *reinterpret_cast<const v4u*>(buf + f8_chunk_addr(brow, gl * 4 + half * 2 + 1));
          const float s = sl[gl * kF8BM + brow];
          const v8i bf = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
          const v8i wf = f8_weights<W>(wring[u][gl]);
          load_weights(q + DW, gl, wring[u][gl]);
          const v16f corr = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aconst, bf, zero16, 0, 0, 0, kF8Scale, 0,
                                                                           kF8Scale);
          D[gl & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, bf, corr, 0, 0, 0, kF8Scale, 0, kF8Scale);
          // the previous group's dots; at a stage start, then close the
          // chunk of the previous stage where it ended there
          rescale((gl + 1) & 1, s_prev, CPS && gl == 1);
          if (gl == 0) {
            if constexpr (CPS) {
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[r] = acc[r] + p[r];
            } else {
              while (g >= cend && c < kChunks - 1) close_chunk();
            }
          }
          s_prev = s;
        }
        store_acts(alds[u ^ 1]);
        load_acts(q + 2);
      }
      __syncthreads();
    }
  }
  rescale(((Qn * kF8KG) - 1) & 1, s_prev, false);  // the last group
  if constexpr (CPS) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = acc[r] + p[r];
  } else {
    while (c < kChunks) close_chunk();
  }

  // ---------------------------------------------------------------- epilogue
  const int m = m_blk + brow;
  if (m >= M) return;
  const bool has_bias = args.prob[0].bias != nullptr;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int nl = ct * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
    const int n = n_blk + nl;
    if (n >= N) continue;
    const float y = has_bias ? __builtin_fmaf(acc[r], wsl[nl], bsl[nl]) : acc[r] * wsl[nl];
    const long o = (long)m * N + n;
    if (args.out_dt == kBF16) store_out<kBF16>(args.prob[0].out, o, y);
    else if (args.out_dt == kF16) store_out<kF16>(args.prob[0].out, o, y);
    else store_out<kF32>(args.prob[0].out, o, y);
  }
}

}  // namespace

void launch_prefill_f8(int W, int A, const LinearArgs& g, hipStream_t st) {
  (void)A;  // the activation width only changes the quantizer's codes
  const int tn = (g.prob[0].N + kF8BN - 1) / kF8BN, tm = (g.M + kF8BM - 1) / kF8BM;
  const bool cps = (g.K / kGroup + 3) / 4 <= kChunks;
  const dim3 grid((unsigned)(tn * tm));
  if (W == 4) {
    if (cps) gemm_prefill_f8<4, true><<<grid, 256, 0, st>>>(g, tm);
    else gemm_prefill_f8<4, false><<<grid, 256, 0, st>>>(g, tm);
  } else {
    if (cps) gemm_prefill_f8<2, true><<<grid, 256, 0, st>>>(g, tm);
    else gemm_prefill_f8<2, false><<<grid, 256, 0, st>>>(g, tm);
  }
}

}  // namespace actune
