/* Host check of the bulk encoder's division (block-gqt-webgpu_amd/csrc/encode_bulk.hip):
 * for x every finite nonzero FP16 value (as float, both signs) and d over sampled positive
 * floats and group norms sqrt(sum of 32 FP16 squares + 1e-30), r = RN(1/d), q0 = RN(x r),
 * q1 = RN(fma(RN(fma(-q0, d, x)), r, q0)) must equal RN(x / d) bit for bit.
 * Usage: host_division_check <divisors>; prints "checked N mismatches M", exit status 1 on M > 0. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float h2f(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u, b;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;
    return (h & 0x8000u) ? -v : v;
  }
  b = sign | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint64_t state = 88172645463325252ull;
static uint64_t next(void) {
  state ^= state << 13;
  state ^= state >> 7;
  state ^= state << 17;
  return state;
}

static float group_norm(uint32_t max_half) {
  float acc = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float v = h2f((uint16_t)(next() % max_half));
    acc += v * v;
  }
  return sqrtf(acc + 1e-30f);
}

int main(int argc, char **argv) {
  const int nd = argc > 1 ? atoi(argv[1]) : 2000;
  static float xs[2 * 0x7c00];
  int nx = 0;
  for (uint32_t h = 1; h < 0x7c00; ++h) {
    xs[nx++] = h2f((uint16_t)h);
    xs[nx++] = -h2f((uint16_t)h);
  }
  long long bad = 0, total = 0;
  for (int k = 0; k < nd; ++k) {
    float d;
    if (k % 3 == 0) { /* any float in [2^-34, 2^20) */
      const uint32_t b = (uint32_t)(next() % (54u << 23)) + ((127u - 34u) << 23);
      memcpy(&d, &b, 4);
    } else {
      d = group_norm(k % 3 == 1 ? 0x7c00u : 0x3c00u);
    }
    const float r = 1.0f / d;
    for (int i = 0; i < nx; ++i) {
      const float x = xs[i], q = x / d, q0 = x * r;
      const float q1 = fmaf(fmaf(-q0, d, x), r, q0);
      uint32_t a, b;
      memcpy(&a, &q, 4);
      memcpy(&b, &q1, 4);
      if (a != b) {
        if (bad < 5) printf("mismatch x=%a d=%a %a %a\n", x, d, q, q1);
        ++bad;
      }
      ++total;
    }
  }
  printf("checked %lld mismatches %lld\n", total, bad);
  return bad != 0;
}
