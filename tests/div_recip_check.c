/* CPU check of the reciprocal division the Int8Absmax GEMM epilogue uses (div_by_recip in
 * matmulfreellmcpu_amd/csrc/mmf_device.hpp, restated here): for every integer numerator a
 * with |a| <= 2^21 and each of ND divisors d, y = RN(1/d), q = RN(a*y), then twice
 * r = fma(-d, q, a), q = fma(r, y, q), must equal the correctly rounded a / d bit for bit.
 * Divisors: half scale_w * scale_a over the scales' range, half random normals with
 * exponents -60 .. 60. Prints the mismatch count; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return rng;
}

static float div_by_recip(float a, float d, float y) {
  float q = a * y;
  float r = fmaf(-d, q, a);
  q = fmaf(r, y, q);
  r = fmaf(-d, q, a);
  return fmaf(r, y, q);
}

int main(int argc, char** argv) {
  const int nd = argc > 1 ? atoi(argv[1]) : 16;
  long bad = 0, total = 0;
  for (int k = 0; k < nd; ++k) {
    float d;
    if (k % 2 == 0) {
      const float sw = 1.0f / (0.005f + 0.05f * (float)(next() % 1000000) / 1e6f);
      const float amax = powf(10.0f, -5.0f + 8.0f * (float)(next() % 1000000) / 1e6f);
      d = sw * (127.0f / amax);
    } else {
      const uint32_t bits = (uint32_t)(next() & 0x7FFFFF) | ((uint32_t)(127 - 60 + next() % 121) << 23);
      memcpy(&d, &bits, 4);
    }
    const float y = 1.0f / d;
    for (int32_t ai = -(1 << 21); ai <= (1 << 21); ++ai) {
      const float a = (float)ai, q = div_by_recip(a, d, y), ref = a / d;
      uint32_t b1, b2;
      memcpy(&b1, &q, 4);
      memcpy(&b2, &ref, 4);
      bad += b1 != b2;
      ++total;
    }
  }
  printf("divisors %d checks %ld mismatches %ld\n", nd, total, bad);
  return bad != 0;
}
