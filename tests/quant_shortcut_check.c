/* Exhaustive CPU check of the division shortcut used by the int8 archive
 * kernel (flashcodec_amd/csrc/fc_codec.hip, div127): for every finite
 * float a >= 0, fma(fma(-y0, 127, a), R, y0) with y0 = fl(a R) and
 * R = fl(1/127) equals the IEEE quotient fl(a / 127).  Prints the number of
 * values checked and of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
  const float R = 1.0f / 127.0f;
  unsigned long long bad = 0, n = 0;
  /* dynamic: the subnormal range at the start is far slower on most CPUs */
#pragma omp parallel for reduction(+ : bad, n) schedule(dynamic, 8)
  for (long long hi = 0; hi < 0x7f80; ++hi) {
    for (uint32_t lo = 0; lo < 0x10000u; ++lo) {
      const uint32_t u = ((uint32_t)hi << 16) | lo;
      float a;
      memcpy(&a, &u, 4);
      const float y0 = a * R;
      const float e = fmaf(-y0, 127.0f, a);
      const float y1 = fmaf(e, R, y0);
      const float ref = a / 127.0f;
      bad += memcmp(&y1, &ref, 4) != 0;
      ++n;
    }
  }
  printf("%llu %llu\n", n, bad);
  return 0;
}
