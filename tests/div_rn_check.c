// Exhaustive check of the quotient the QDQ kernels use (rx-met_amd/csrc/div_rn.h): Markstein's
// q1 = fma(fma(-q, b, a), y, q) with q = RN(a y), y = RN(1 / b), against the IEEE division a / b
// for every fp32 a (both signs; every `stride`-th bit pattern) and a set of scales b (simple,
// all-ones and minimal significands, tiny, huge, random), wherever the kernels take that path
// (a and q in [2^-100, 2^100]).  usage: div_rn_check [stride [first_b last_b]]; exit 0 when
// no quotient differs.  Run with stride 1 over all 24 scales: no difference in 1.8e11.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>
static float fb(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
int main(int argc, char **argv) {
  float bs[64]; int nb = 0;
  const float fixed[] = {1.0f, 1.5f, 3.0f, 0.1f, 0.0173f, 7.0f, 1e-3f, 0.05f, 65535.0f, 1e-30f, 1e30f,
                         fb(0x3fffffff), fb(0x3f7fffff), fb(0x3f800001), fb(0x3fc00001), fb(0x407fffff)};
  for (unsigned i = 0; i < sizeof(fixed) / sizeof(fixed[0]); ++i) bs[nb++] = fixed[i];
  srand(7);
  while (nb < 24) { uint32_t u = (0x3c000000u + ((uint32_t)rand() % 0x07000000u)) | ((uint32_t)rand() & 0x7fffff); bs[nb++] = fb(u); }
  long long bad = 0, fast = 0;
  const int i0 = argc > 2 ? atoi(argv[2]) : 0, i1 = argc > 3 ? atoi(argv[3]) : nb;
  for (int i = i0; i < i1 && i < nb; ++i) {
    const float b = bs[i];
    volatile float one = 1.0f;
    const float y = one / b;
    for (uint64_t u = 0; u < (1ull << 32); u += (argc > 1 ? atoi(argv[1]) : 1)) {
      const float a = fb((uint32_t)u);
      if (!isfinite(a)) continue;
      const float q = a * y;
      const float aq = fabsf(q);
      const float aa = fabsf(a);
      if (!(aq >= 0x1p-100f && aq <= 0x1p100f && aa >= 0x1p-100f && aa <= 0x1p100f)) continue;
      ++fast;
      const float r = fmaf(-q, b, a);
      const float q1 = fmaf(r, y, q);
      const float ref = a / b;
      if (bf(q1) != bf(ref)) { if (bad < 12) { printf("b=%a y=%a a=%a q=%a fast=%a ref=%a\n", b, y, a, q, q1, ref); fflush(stdout); } ++bad; }
    }
    printf("b=%a done, bad so far %lld of %lld\n", b, bad, fast); fflush(stdout);
  }
  printf("TOTAL bad=%lld fast=%lld\n", bad, fast);
  return bad != 0;
}
