// Host-side launch descriptors shared by the kernel translation units and the
// C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace actune {

constexpr int kMaxProblems = 4;
// LDS budget of the streaming kernel (gfx950 has 160 KiB per CU)
constexpr size_t kStreamLdsMax = 144 * 1024;

// One linear of a launch: all problems of a launch share the activation
// (x or its packed codes), K, W and A.
struct Problem {
  const uint8_t* w;     // packed weights [N, K*W/8]
  const float* ws;      // weight scale [N]
  const void* bias;     // [N] in bias_dt, or nullptr
  void* out;            // [M, N] in out_dt
  int N;
  int tile0;            // first 16-row tile of this problem in the launch grid
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
};

// The problem owning row tile `tile`, selected field by field with constant
// indices so the by-value kernel arguments stay in scalar kernarg loads.
__device__ __forceinline__ Problem select_problem(const LinearArgs& args, int tile) {
  Problem pr;
  pr.w = args.prob[0].w; pr.ws = args.prob[0].ws; pr.bias = args.prob[0].bias;
  pr.out = args.prob[0].out; pr.N = args.prob[0].N; pr.tile0 = args.prob[0].tile0;
#pragma unroll
  for (int q = 1; q < kMaxProblems; ++q) {
    if (q < args.nprob && tile >= args.prob[q].tile0) {
      pr.w = args.prob[q].w; pr.ws = args.prob[q].ws; pr.bias = args.prob[q].bias;
      pr.out = args.prob[q].out; pr.N = args.prob[q].N; pr.tile0 = args.prob[q].tile0;
    }
  }
  return pr;
}

void launch_quantize(const void* x, int dt, const void* sc, long M, long K, int A, uint8_t* packed,
                     float* scales, hipStream_t stream);
void launch_smallm(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st);
void launch_tiled(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st);
void launch_stream(int W, int A, int nw, int mode, const LinearArgs& g, hipStream_t st);
void launch_prefill(int W, int A, int shape, bool dots, const LinearArgs& g, hipStream_t st);
void launch_decode(int W, int A, int nw, const LinearArgs& g, hipStream_t st);
size_t decode_lds_bytes(int K, int M, int nw);
// true when the decode kernel with nw waves takes an M x K problem of width W
// (every wave's loads fit its register ring and x passes)
bool decode_fits(int K, int M, int W, int nw);
size_t stream_lds_bytes(int K, int M, int nw);

}  // namespace actune
