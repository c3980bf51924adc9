/*
 * Exhaustive proof that the quantizer's fast division yields the same codes
 * as the IEEE quotient, for every 16-bit (bf16 or f16) input.
 *
 * The group-64 quantizer needs c = clamp(rint(fl(x / s)), -p-1, p) with the
 * IEEE quotient (actune/calibration.py:14). The kernels compute
 *   y  = fl(1 / s)            (IEEE division, once per group)
 *   q0 = fl(x * y)
 *   r  = fma(-q0, s, x)       (exact residual)
 *   q1 = fma(r, y, q0)        (Markstein's correction)
 * For p > 1 the kernels form s itself without a division, as
 *   s = fma(fma(-q, p, amax), yp, q),  q = fl(amax * yp),  yp = fl(1 / p),
 * and this program checks that it equals fl(amax / p) bit for bit.
 * It checks rint(q1) == rint(x / s) after clamping for every
 * p in {1, 7, 127}, every positive finite amax of the format (plus the f32
 * 1e-8 floor), s = fl(max(amax, 1e-8) / p), and every x of the format with
 * 0 <= x <= amax (negative x is symmetric under round-to-nearest-even).
 *
 * usage: exhaustive_division <bf16|f16> [stride]   (stride > 1 samples amax)
 * exit status 0 iff no mismatch.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bf16(uint32_t b) { uint32_t u = b << 16; float f; memcpy(&f, &u, 4); return f; }

static float from_f16(uint32_t h) {
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return (float)m * 5.9604644775390625e-8f;
  if (e == 31) return INFINITY;
  uint32_t u = ((e + 112u) << 23) | (m << 13);
  float f; memcpy(&f, &u, 4); return f;
}

static int code(float q, int p) {
  float c = rintf(q);
  if (c < (float)(-p - 1)) c = (float)(-p - 1);
  if (c > (float)p) c = (float)p;
  return (int)c;
}

int main(int argc, char** argv) {
  int f16 = argc > 1 && strcmp(argv[1], "f16") == 0;
  long stride = argc > 2 ? atol(argv[2]) : 1;
  uint32_t top = f16 ? 0x7C00u : 0x7F80u;  /* first non-finite pattern */
  float (*conv)(uint32_t) = f16 ? from_f16 : from_bf16;
  const int ps[3] = {1, 7, 127};
  long bad = 0, checked = 0, bad_scale = 0;
  for (int pi = 0; pi < 3; ++pi) {
    const int p = ps[pi];
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, checked, bad_scale)
    for (long ab = 1; ab <= (long)top; ab += stride) {
      float amax = ab == (long)top ? 1e-8f : conv((uint32_t)ab);  /* top stands for the floor */
      if (amax < 1e-8f) amax = 1e-8f;
      const float s = amax / (float)p;
      if (p > 1) {  /* the kernels' constant-divisor form of s for 16-bit inputs */
        const float yp = 1.0f / (float)p;
        const float sq0 = amax * yp;
        const float sr = fmaf(-sq0, (float)p, amax);
        const float sf = fmaf(sr, yp, sq0);
        if (memcmp(&sf, &s, 4) != 0) ++bad_scale;
      }
      const float y = 1.0f / s;
      for (uint32_t xb = 0; xb < top; ++xb) {
        const float x = conv(xb);
        if (x > amax) break;
        const float q0 = x * y;
        const float r = fmaf(-q0, s, x);
        const float q1 = fmaf(r, y, q0);
        ++checked;
        if (code(q1, p) != code(x / s, p)) ++bad;
      }
    }
  }
  printf("%s: checked %ld (x, s) pairs, mismatches %ld, scale mismatches %ld\n", f16 ? "f16" : "bf16", checked, bad,
         bad_scale);
  return bad != 0 || bad_scale != 0;
}
