// Host-side launchers shared by the kernel translation units and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace actune {

struct GemmArgs {
  const uint8_t* a;     // packed activations [M, K*A/8]
  const float* as;      // activation scales [M, K/64]
  const uint8_t* w;     // packed weights [N, K*W/8]
  const float* ws;      // weight scale [N]
  const void* bias;     // [N] in bias_dt, or nullptr
  int bias_dt;
  void* out;            // [M, N] in out_dt
  int out_dt;
  int32_t* dots;        // [M, N, K/64] (dots mode only)
  int M, N, K;
};

void launch_quantize(const void* x, int dt, const void* sc, long M, long K, int A, uint8_t* packed,
                     float* scales, hipStream_t stream);
void launch_gemm(int W, int A, int config, const GemmArgs& g, hipStream_t st);
void launch_dots(int W, int A, int config, const GemmArgs& g, hipStream_t st);

}  // namespace actune
