/*
 * Exhaustive check of the store_int8 kernel's quotient arithmetic on the CPU.
 *
 * The kernel (csrc/store_int8.hip) replaces the IEEE division x / s of the
 * reference quantiser (kernels/titan_kv.py:17) by
 *     y  = fl(1 / s)             once per row
 *     q0 = fl(x * y)
 *     r  = fma(-q0, s, x)
 *     q1 = fma(r, y, q0)
 *     t  = fl(q1 + 1.5 * 2^23)   int8 code = low byte of t's bit pattern
 * This program walks the whole input domain: every finite non-negative bf16
 * amax (the row maximum, from which s = max(amax / 127, 1e-12)) and every
 * bf16 x with |x| <= amax, and counts
 *   div_mismatch      : q1 != fl(x / s)        (Markstein identity)
 *   div_mismatch_big  : the same with |x / s| >= 1e-20
 *   code_mismatch     : low byte of t != int8(clamp(nearbyint(x / s), +-127))
 * The identity can fail only where intermediates underflow (|x / s| tiny);
 * those quotients round to code 0 on both paths.
 * Build with -O2 -ffp-contract=off (no fast-math) so each line rounds once.
 * -DPLANT_NO_CORRECTION drops the correction step (q1 = q0), a plausible
 * slip the check must detect.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf(uint32_t h) { uint32_t u = h << 16; float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(void) {
  long long div_mismatch = 0, div_mismatch_big = 0, code_mismatch = 0, pairs = 0;
#pragma omp parallel for schedule(dynamic, 64) \
    reduction(+ : div_mismatch, div_mismatch_big, code_mismatch, pairs)
  for (int a = 0; a <= 0x7F7F; a++) {            /* finite non-negative bf16 */
    const float amax = bf((uint32_t)a);
    float s = amax / 127.0f;
    if (!(s > 1.0e-12f)) s = 1.0e-12f;
    const float y = 1.0f / s;
    for (int sign = 0; sign < 2; sign++) {
      for (int m = 0; m <= a; m++) {
        if (sign && m == 0) continue;
        const float x = bf((uint32_t)(m | (sign << 15)));
        const float exact = x / s;
        float ref = nearbyintf(exact);
        ref = fminf(fmaxf(ref, -127.0f), 127.0f);
        const uint8_t want = (uint8_t)(int8_t)(int)ref;
        const float q0 = x * y;
        const float r = fmaf(-q0, s, x);
#ifdef PLANT_NO_CORRECTION
        const float q1 = q0 + 0.0f * r;   /* planted mistake: skip the correction */
#else
        const float q1 = fmaf(r, y, q0);
#endif
        const float t = q1 + 12582912.0f;
        const uint8_t got = (uint8_t)(bits(t) & 0xffu);
        const int dm = (bits(q1) != bits(exact)) && !(q1 == 0.0f && exact == 0.0f);
        div_mismatch += dm;
        div_mismatch_big += dm && fabsf(exact) >= 1.0e-20f;
        code_mismatch += got != want;
        pairs++;
      }
    }
  }
  printf("{\"pairs\": %lld, \"div_mismatch\": %lld, \"div_mismatch_big\": %lld, "
         "\"code_mismatch\": %lld}\n", pairs, div_mismatch, div_mismatch_big, code_mismatch);
  return 0;
}
