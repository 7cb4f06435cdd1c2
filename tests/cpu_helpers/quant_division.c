/* CPU check of the division in the activation quantisation (quant_value<0> of
 * freetoken_amd/csrc/quant.h): with s = max(amax, 1e-10f) / 448 and
 * r = RN(1 / s), the value q = RN(x r), e = fma(-q, s, x), y = RN(fma(e, r, q))
 * with x's sign must equal the IEEE quotient x / s for every pair of bf16
 * values with 0 <= amax finite and |x| <= amax, except where x is so small
 * that the residual e underflows (all such quotients are below 2^-71, far
 * below e4m3's smallest subnormal 2^-9): those convert to the zero code of x's
 * sign either way.  Prints "pairs P mismatches M large L" and exits
 * non-zero when L > 0 or a mismatch has a different sign or is not tiny. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(void) {
  unsigned long long pairs = 0, mism = 0, large = 0, odd = 0;
#pragma omp parallel for reduction(+ : pairs, mism, large, odd) schedule(dynamic, 64)
  for (uint32_t ab = 0; ab < 0x7f80u; ++ab) {
    const float amax = f_of(ab << 16);
    const float s = fmaxf(amax, 1e-10f) / 448.0f;
    const float r = 1.0f / s;
    for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
      const float x = f_of(xb << 16);
      if (!(fabsf(x) <= amax)) continue;
      ++pairs;
      const float ref = fminf(fmaxf(x / s, -448.0f), 448.0f);
      const float q = x * r;
      const float e = fmaf(-q, s, x);
      float y = fmaf(e, r, q);
      y = f_of((u_of(y) & 0x7fffffffu) | (u_of(x) & 0x80000000u));
      y = fminf(fmaxf(y, -448.0f), 448.0f);
      if (u_of(y) != u_of(ref)) {
        ++mism;
        if (fabsf(ref) >= 0x1p-64f) ++large;
        if ((u_of(y) ^ u_of(ref)) >> 31 || fabsf(y) >= 0x1p-64f) ++odd;
      }
    }
  }
  printf("pairs %llu mismatches %llu large %llu odd %llu\n", pairs, mism, large, odd);
  return (large || odd) ? 1 : 0;
}
