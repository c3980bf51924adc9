// Allocation-free quantize + linear: actune_grouped_forward with its
// packed-activation scratch in a library-owned static device array.
//
// For callers that cannot allocate device memory (code under stream capture,
// tight serving loops, harnesses that forbid hipMalloc): the caller passes x,
// the weights and the output; the packed activation codes and group scales
// that actune_grouped_forward takes as caller-owned scratch live in
// `scratch` below instead. Each GPU holds its own copy of the array (8 MiB)
// until the process ends.
//
// `scratch` is a device symbol: in host code its name is not a device
// address. Its address on each device is looked up once, with that device
// current, through hipGetSymbolAddress, and only that pointer is handed to
// kernels. Every call on one device shares that device's array: calls that
// overlap on one GPU (two streams, or two host threads) race on it. Nothing
// in it has to start at zero: the quantizer writes every code and scale the
// GEMM then reads.
#include <stdio.h>

#include <mutex>

#include "../../include/actune_hip.h"
#include "launch.hpp"

namespace {

constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr size_t kScratchAlign = 256;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

uint8_t* g_scratch_ptr[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_status[kMaxDevices];

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// The current device's copy of `scratch` (null and a message on failure).
uint8_t* device_scratch(int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    char msg[256];
    snprintf(msg, sizeof msg, "no usable current device (%s)", hipGetErrorString(e));
    actune::set_last_error(msg);
    *rc = ACTUNE_ERR_DEVICE;
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  });
  if (g_scratch_status[dev] != hipSuccess || !g_scratch_ptr[dev]) {
    char msg[256];
    snprintf(msg, sizeof msg, "scratch array address lookup failed on device %d: %s", dev,
             hipGetErrorString(g_scratch_status[dev]));
    actune::set_last_error(msg);
    *rc = ACTUNE_ERR_DEVICE;
    return nullptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int actune_grouped_forward_noalloc(const void* x, int x_dtype, const void* input_scale, const uint8_t* w,
                                   const float* w_scale, const void* bias, int bias_dtype, void* out, int64_t M,
                                   int64_t N, int64_t K, int W, int A, int config, void* stream) {
  if (M < 0 || K <= 0 || K % 64 || (A != 2 && A != 4 && A != 8)) {
    // argument errors are reported by the regular entry point
    return actune_grouped_forward(x, x_dtype, input_scale, nullptr, nullptr, w, w_scale, bias, bias_dtype, out,
                                  M, N, K, W, A, config, stream);
  }
  const size_t codes = round_up((size_t)M * (size_t)K * (size_t)A / 8, kScratchAlign);
  const size_t scales = (size_t)M * (size_t)(K / 64) * sizeof(float);
  if (M > (int64_t)kScratchBytes || K > (int64_t)kScratchBytes || codes + scales > kScratchBytes) {
    actune::set_last_error("activation too large for the static scratch: M*K*A/8 (rounded up to 256) + "
                           "M*K/16 bytes must be at most 8 MiB (8388608)");
    return ACTUNE_ERR_INVALID;
  }
  if (M == 0)
    return actune_grouped_forward(x, x_dtype, input_scale, nullptr, nullptr, w, w_scale, bias, bias_dtype, out,
                                  M, N, K, W, A, config, stream);
  int rc = ACTUNE_OK;
  uint8_t* base = device_scratch(&rc);
  if (!base) return rc;
  return actune_grouped_forward(x, x_dtype, input_scale, base, reinterpret_cast<float*>(base + codes), w, w_scale,
                                bias, bias_dtype, out, M, N, K, W, A, config, stream);
}

}  // extern "C"
