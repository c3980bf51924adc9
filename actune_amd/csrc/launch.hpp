// Host-side launch descriptors shared by the kernel translation units and the
// C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace actune {

constexpr int kMaxProblems = 4;
// Group-row indices (group of a wave's K-range x token of a 16-token block)
// of the decode kernel stay below this; LinearArgs::m_div is exact there.
constexpr int kDecodeMaxGroupRows = 256;
// LDS budget of the streaming kernel (gfx950 has 160 KiB per CU)
constexpr size_t kStreamLdsMax = 144 * 1024;

// One linear of a launch: all problems of a launch share the activation
// (x or its packed codes), K and A, and all but the mixed-width decode
// launch (launch_decode_mixed) share W.
struct Problem {
  const uint8_t* w;     // packed weights [N, K*W/8]
  const float* ws;      // weight scale [N]
  const void* bias;     // [N] in bias_dt, or nullptr
  void* out;            // [M, N] in out_dt
  int N;
  int tile0;            // first 16-row tile of this problem in the launch grid
  int W;                // weight width of this problem
};

enum { kModePacked = 0, kModeFused = 1, kModeDots = 2 };

struct LinearArgs {
  Problem prob[kMaxProblems];
  int nprob;
  int tiles;            // 16-row tiles over all problems
  const uint8_t* a;     // packed activations [M, K*A/8] (packed / dots modes)
  const float* as;      // activation scales [M, K/64]
  const void* x;        // activation source [M, K] (fused mode)
  const void* xscale;   // channel scale [K] or nullptr (fused mode)
  int x_dt;
  int32_t* dots;        // [M, N, K/64] (dots mode, single problem)
  int M, K, bias_dt, out_dt;
  // ceil(2^16 / M). With e = m_div * M - 2^16 (0 <= e < M), idx / M ==
  // (idx * m_div) >> 16 whenever idx * e < 2^16, so for every idx < 2^16 / 16
  // = 4096 when M <= 16 (it fails first at idx 4694 for M = 15). The decode
  // kernel, its only user, divides group-row indices below
  // kDecodeMaxGroupRows = 16 groups x 16 tokens (decode_fits enforces it).
  uint32_t m_div;
  uint32_t m_div_tail;  // the same for the last 16-token block, M - 16 * ((M - 1) / 16) tokens
};

// The problem owning row tile `tile`. Every slot is read unconditionally and
// the owner is picked with scalar selects, so the by-value kernel arguments
// arrive in one batch of scalar loads (a branch per slot would put a load
// round trip on the path to the first weight load for each slot).
__device__ __forceinline__ Problem select_problem(const LinearArgs& args, int tile) {
  Problem pp[kMaxProblems];
#pragma unroll
  for (int q = 0; q < kMaxProblems; ++q) pp[q] = args.prob[q];
  int sel = 0;
#pragma unroll
  for (int q = 1; q < kMaxProblems; ++q) sel += (q < args.nprob && tile >= pp[q].tile0) ? 1 : 0;
  Problem pr = pp[0];
#pragma unroll
  for (int q = 1; q < kMaxProblems; ++q) {
    const bool s = sel == q;
    pr.w = s ? pp[q].w : pr.w;
    pr.ws = s ? pp[q].ws : pr.ws;
    pr.bias = s ? pp[q].bias : pr.bias;
    pr.out = s ? pp[q].out : pr.out;
    pr.N = s ? pp[q].N : pr.N;
    pr.tile0 = s ? pp[q].tile0 : pr.tile0;
    pr.W = s ? pp[q].W : pr.W;
  }
  return pr;
}

// Lets kernel KERN take up to kStreamLdsMax bytes of dynamic LDS on the
// current device (above the default per-launch limit). Done once per
// (kernel, device); safe to call from several host threads.
template <auto KERN>
inline void allow_dynamic_lds() {
  static std::atomic<uint64_t> done{0};  // bit d: raised on device d
  int dev = 0;
  (void)hipGetDevice(&dev);
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kStreamLdsMax);
  done.fetch_or(bit, std::memory_order_release);
}

// Sets the calling thread's actune_last_error() message.
void set_last_error(const char* msg);

void launch_quantize(const void* x, int dt, const void* sc, long M, long K, int A, uint8_t* packed,
                     float* scales, hipStream_t stream);
void launch_quantize_gated(const void* gate, const void* up, int dt, int act, const void* sc, long M, long K, int A,
                           uint8_t* packed, float* scales, hipStream_t stream);
void launch_smallm(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st);
void launch_tiled(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st);
void launch_stream(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st);
void launch_prefill(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st);
// packed: the activations are codes + scales from the quantizer launch
// (g.a, g.as); otherwise bf16 x is quantized inside the launch (g.x)
void launch_decode(int W, int A, int nw, bool packed, const LinearArgs& g, hipStream_t st);
// The decode kernel over problems of different widths (Problem::W, each in
// {2, 4, 8}), one launch; every width must pass decode_fits
void launch_decode_mixed(int A, int nw, bool packed, const LinearArgs& g, hipStream_t st);
// cmp: with compact chunk partials (one slot per nonempty chunk)
size_t decode_lds_bytes(int K, int M, int nw, int tr, bool cmp = false);
// true when the decode kernel with nw waves takes an M x K problem of width W
// in the given activation mode (every wave's loads fit its register ring and
// activation passes; the fused mode takes bf16 x only)
bool decode_fits(int K, int M, int W, int nw, bool packed, int x_dt);
// 16-row tiles per workgroup of a decode launch (1, 2 or 4) for nprob
// problems of `tiles` row tiles each; results do not depend on it
// compact: the launch can take compact chunk partials (the single-width
// kernel; the mixed-width kernel cannot)
int decode_row_tiles(int K, int M, int W, int nw, int tiles, int nprob, bool compact = true);
size_t stream_lds_bytes(int K, int M, int nw);

}  // namespace actune
