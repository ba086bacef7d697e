/* Exhaustive check of the INT8 quantiser's division-free law (test
 * infrastructure; compiled and run by tests/test_quant_law.py).
 *
 * The reference quantises q = round_half_away(fl(x / s)) with
 * s = fl(fl(amax / 127) + 1e-12) per 64x64 tile (kernel_sparse_qat.py:136-141).
 * The gfx950 kernel computes, with r = fl(1 / s):
 *   q0 = fl(x r),  qf = fma(fma(-q0, s, x), r, q0),
 *   q  = (int) fl(qf + copysign(0.5 - 2^-25, x))
 * This program compares the two for every 16-bit x (both signs) against every
 * 16-bit tile maximum amax >= |x|, for bf16 and fp16 values.
 *
 * usage: quant_law_check STRIDE   -- amax bit patterns 1, 1 + STRIDE, ...
 *        (STRIDE 1 = the full sweep, 2.07e9 pairs)
 * prints "pairs N mismatches M"; exit status 1 when M > 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static float f16_to_f32(uint16_t h) {
  int e = (h >> 10) & 31, m = h & 1023;
  return e == 0 ? ldexpf((float)m, -24) : ldexpf((float)(m + 1024), e - 25);
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 10) : 1u;
  long long pairs = 0, bad = 0;
  for (int kind = 0; kind < 2; ++kind) {
    const uint32_t lim = kind == 0 ? 0x7f80u : 0x7c00u; /* positive finite values */
    for (uint32_t ab = 1; ab < lim; ab += stride) {
      const float amax = kind == 0 ? bf16_to_f32((uint16_t)ab) : f16_to_f32((uint16_t)ab);
      volatile float t = amax / 127.0f;
      const float s = t + 1e-12f;
      volatile float one = 1.0f;
      const float r = one / s;
      for (uint32_t xb = 0; xb < lim; ++xb) {
        const float xp = kind == 0 ? bf16_to_f32((uint16_t)xb) : f16_to_f32((uint16_t)xb);
        if (xp > amax) break;
        for (int sg = 0; sg < 2; ++sg) {
          const float x = sg ? -xp : xp;
          volatile float exact = x / s;
          const int want = (int)roundf(exact);
          const float q0 = x * r;
          const float qf = fmaf(fmaf(-q0, s, x), r, q0);
          volatile float sum = qf + copysignf(0x1.fffffep-2f, x);
          const int got = (int)sum;
          ++pairs;
          if (got != want) {
            if (bad < 5)
              printf("mismatch: kind %d amax %.9g x %.9g want %d got %d\n", kind, amax, x, want, got);
            ++bad;
          }
        }
      }
    }
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}
