/* Exhaustive check of the MX encoder's fast block-exponent path (csrc/mx_state.hip,
 * block_exponent_fast) against the IEEE-correct quotient t = RN(absmax / 2M).
 *
 * The exact rule (mamba_state_8b_kernel.py:172, 560) is e = ceil(log2(max(t, 1e-30))) + 127
 * clamped to [1, 254], log2 rounded to fp32; for t = 2^E (1 + j 2^-23) it equals E + 1 + 127
 * whenever j > 44 (the band bound pinned by the oracle's ceil_log2_f32 tests). The fast path
 * claims eb = biased(q) + 1 with q = RN(absmax * RN(1/2M)) for absmax in [AMAX_LO, AMAX_HI) and
 * q's mantissa in [MANT_LO, MANT_HI]. It is correct exactly when, for every such absmax,
 * biased(t) == biased(q), mant(t) > 44, t >= 1e-30 and eb <= 254. This program checks that
 * for every fp32 bit pattern in the range and both formats (2M = 14 and 126), and prints the
 * number of values on the fast path and of failures. Constants come in on the command line.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  if (argc != 5) { fprintf(stderr, "usage: amax_lo amax_hi mant_lo mant_hi\n"); return 2; }
  const uint32_t amax_lo = (uint32_t)strtoul(argv[1], 0, 0), amax_hi = (uint32_t)strtoul(argv[2], 0, 0);
  const uint32_t mant_lo = (uint32_t)strtoul(argv[3], 0, 0), mant_hi = (uint32_t)strtoul(argv[4], 0, 0);
  const float floor_t = 1.0e-30f;
  int status = 0;
  for (int f = 0; f < 2; ++f) {
    const float two_m = f == 0 ? 14.0f : 126.0f;
    const float c = 1.0f / two_m;  /* RN(1/2M), as the device constant */
    long long fast = 0, bad = 0;
    uint32_t first_bad = 0;
#pragma omp parallel for reduction(+ : fast, bad) schedule(static)
    for (long long i = amax_lo; i < (long long)amax_hi; ++i) {
      const float amax = f_of((uint32_t)i);
      const uint32_t qb = u_of(amax * c);
      if ((qb & 0x7fffffu) - mant_lo > mant_hi - mant_lo) continue;
      ++fast;
      const uint32_t tb = u_of(amax / two_m);
      const uint32_t eb = (qb >> 23) + 1;
      if ((tb >> 23) != (qb >> 23) || (tb & 0x7fffffu) <= 44u || f_of(tb) < floor_t || eb > 254u) {
        ++bad;
#pragma omp critical
        if (first_bad == 0) first_bad = (uint32_t)i;
      }
    }
    printf("2M=%g fast=%lld bad=%lld first_bad=0x%08x\n", (double)two_m, fast, bad, first_bad);
    if (bad != 0 || fast == 0) status = 1;
  }
  return status;
}
