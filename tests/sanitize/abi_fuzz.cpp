// Host-sanitizer driver of the C ABI (built and run by tests/sanitize/Makefile
// against objects whose host code carries AddressSanitizer and
// UndefinedBehaviorSanitizer; the device code is the shipped one).
//
// Every entry point is called over edge-case and invalid dimensions, widths,
// dtypes, layouts and configs: in the first half of the rounds with NULL
// buffers (each call must return ACTUNE_ERR_INVALID, or ACTUNE_OK for an
// empty call), in the second half with a 4 KiB host block standing in for
// every buffer, so that calls that pass validation also run their host-side
// config selection and launch geometry, then fail at the launch on a machine
// without a GPU (ACTUNE_ERR_DEVICE). Run it only where no GPU is visible:
// with a GPU, the second half would launch kernels on host memory.
#include <cstdio>
#include <cstdint>
#include <random>
#include "../../include/actune_hip.h"
struct AnyPtr {
  void* p;
  template <class T> operator T*() const { return (T*)p; }
};
int main(int argc, char** argv) {
  const int rounds = argc > 1 ? atoi(argv[1]) : 2000;
  const int64_t MS[] = {-1, 0, 1, 2, 8, 17, 64, 65, 512, 1024, 1025, 1LL << 31, 1LL << 40};
  const int64_t NS[] = {-1, 0, 1, 16, 42, 4096, 1LL << 31, 1LL << 40};
  const int64_t KS[] = {-64, 0, 1, 64, 100, 128, 4096, 11008, 65536, 1LL << 31, 1LL << 40};
  const int WS[] = {-1, 0, 1, 2, 3, 4, 8, 16};
  const int CODES[] = {-2, -1, 0, 1, 2, 3, 5, 6, 99};
  const int CFG[] = {-2, -1, 0, 3, 9, 10, 14, 16, 17};
  std::mt19937 rng(0);
  // a 4 KiB aligned host block stands in for every buffer in the second half
  // of the rounds: valid calls then run their host-side selection and launch
  // geometry and fail at the launch (no GPU here)
  void* blk = aligned_alloc(4096, 4096);
  auto pick = [&](auto& arr) { return arr[rng() % (sizeof(arr) / sizeof(arr[0]))]; };
  int bad = 0, launched = 0;
  AnyPtr B{nullptr};
  auto st = [&](const char* name, int rc, int64_t m) {
    if (rc == 2) ++launched;
    if (rc < 0 || rc > 2 || (rc == 0 && m != 0 && B.p == nullptr)) { ++bad; printf("bad %s rc %d m %lld\n", name, rc, (long long)m); }
  };
  for (int r = 0; r < rounds; ++r) {
    B.p = r >= rounds / 2 ? blk : nullptr;
    const int64_t m = pick(MS), n = pick(NS), k = pick(KS);
    const int w = pick(WS), a = pick(WS), dt = pick(CODES), dt2 = pick(CODES), cfg = pick(CFG);
    const int lay = pick(CODES), lay2 = pick(CODES);
    const int nt = (int)(rng() % 7) - 1;
    const int64_t wsb = (int64_t[]){0, -1, 1 << 20}[rng() % 3];
    actune_linear_target t[5];
    for (auto& x : t) x = actune_linear_target{(const uint8_t*)blk, (const float*)blk, nullptr, blk, pick(NS), pick(WS)};
    actune_tw_target tw[5];
    for (auto& x : tw) x = actune_tw_target{blk, nullptr, (const float*)blk, nullptr, blk};
    st("quantize_groups", actune_quantize_groups(B, dt, B, m, k, a, B, B, nullptr), m);
    st("quantize_gated", actune_quantize_gated(B, B, dt, lay, B, m, k, a, B, B, nullptr), m);
    st("grouped_linear", actune_grouped_linear(B, B, B, B, B, dt, B, dt2, m, n, k, w, a, cfg, nullptr), m);
    st("grouped_forward", actune_grouped_forward(B, dt, B, B, B, B, B, B, dt2, B, m, n, k, w, a, cfg, nullptr), m);
    st("grouped_forward_multi", actune_grouped_forward_multi(B, dt, B, B, B, nt >= 0 ? t : B, nt, dt2, m, k, w, a, cfg, nullptr), m);
    st("forward_noalloc", actune_grouped_forward_noalloc(B, dt, B, B, B, B, dt2, B, m, n, k, w, a, cfg, nullptr), m);
    st("dots_i32", actune_grouped_dots_i32(B, B, m, n, k, w, a, cfg, B, nullptr), m);
    actune_forward_fuses_quantizer(m, n, k, w, a, dt, cfg);
    actune_default_config(m, n, k, w, a);
    actune_config_valid(cfg, m);
    st("tw_quantize", actune_tokenwise_quantize(B, dt, m, k, a, B, B, nullptr), m);
    actune_tokenwise_workspace_bytes(m, n, k, lay, lay2);
    st("tw_linear", actune_tokenwise_linear(B, lay2, B, B, lay, B, B, dt, B, dt2, m, n, k, cfg, B, wsb, nullptr), m);
    st("tw_linear_x", actune_tokenwise_linear_x(B, dt, B, B, lay, B, B, dt, B, dt2, m, n, k, cfg, B, wsb, nullptr), m);
    st("tw_linear_multi", actune_tokenwise_linear_multi(B, lay2, B, dt, B, lay, nt >= 0 ? tw : B, nt, dt, dt2, m, n, k, cfg, B, wsb, nullptr), m);
  }
  if (actune_layout_selftest()) { printf("selftest failed\n"); ++bad; }
  printf("%d rounds, %d bad, %d calls reached a launch\n", rounds, bad, launched);
  return bad ? 1 : 0;
}
