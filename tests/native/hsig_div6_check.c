/* Exhaustive check of the division by 6 in the gating kernels' hardsigmoid
 * (pom_amd/csrc/common.h, hsig): for every fp32 x in [2^-122, 6] and x = 0,
 * fma(fma(-q, 6, x), r, q) with q = x * r, r = RN(1/6) equals RN(x / 6).
 * Exit status 0 when every value agrees. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
  const float r = 1.0f / 6.0f;
  const float lo = 0x1p-122f, hi = 6.0f;
  uint32_t b0, b1;
  memcpy(&b0, &lo, 4);
  memcpy(&b1, &hi, 4);
  uint64_t bad = 0, n = 0;
  for (uint64_t b = b0; b <= b1; ++b) {
    uint32_t u = (uint32_t)b;
    float x;
    memcpy(&x, &u, 4);
    volatile float ref = x / 6.0f;
    const float q = x * r;
    const float got = fmaf(fmaf(-q, 6.0f, x), r, q);
    if (got != ref) {
      if (bad < 5) printf("mismatch x=%a ref=%a got=%a\n", x, ref, got);
      ++bad;
    }
    ++n;
  }
  {
    const float x = 0.0f, q = x * r;
    if (fmaf(fmaf(-q, 6.0f, x), r, q) != 0.0f) ++bad;
  }
  printf("checked %llu values, %llu mismatches\n", (unsigned long long)n + 1, (unsigned long long)bad);
  return bad != 0;
}
