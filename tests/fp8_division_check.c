/* The FP8 row quantiser divides by the row scale sc as q = RN(x * r), r = RN(1 / sc), then RN(q + fma(-q, sc, x) * r)
 * with the sign of x (csrc/fp8_quant.hip: div_sc). This checks that the result equals IEEE RN(x / sc) wherever the
 * quotient can reach an e4m3 value (|x / sc| >= 2^-12; smaller quotients are +-0 in e4m3 either way):
 *   - every finite bf16 x against NB scales (the first 1024 with significands next to all ones),
 *   - NR random finite fp32 x against random scales, x spanning [sc * 2^-12, sc * 448].
 * Scales range over [1e-12, 2^119], the values max(amax / 448, 1e-12) takes for finite inputs.
 * Usage: fp8_division_check NB NR; prints the counts and exits 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }

static float div_sc(float x, float sc, float r) {
  const float q = x * r;
  return copysignf(fmaf(fmaf(-q, sc, x), r, q), x);
}

static float scale(long i) {
  const uint64_t s = next();
  uint32_t m = (uint32_t)(s >> 20) & 0x7FFFFF;
  if (i < 1024) m = 0x7FFFFF - (uint32_t)i;
  float b = f_of(((87 + (uint32_t)(s % 160)) << 23) | m);
  if (!(b >= 1e-12f)) b = 1e-12f;
  return b;
}

int main(int argc, char** argv) {
  const long nb = argc > 1 ? atol(argv[1]) : 2048, nr = argc > 2 ? atol(argv[2]) : 20000000;
  long checked = 0, bad = 0;
  for (long i = 0; i < nb; ++i) {
    const float b = scale(i), r = 1.0f / b;
    for (uint32_t h = 0; h < 65536; ++h) {
      const float x = f_of(h << 16);
      if (!isfinite(x) || !isfinite(b * 448.f)) continue;
      const float ref = x / b;
      if (fabsf(ref) < 0x1p-12f || fabsf(ref) > 448.f * 1.001f) continue;
      ++checked;
      if (u_of(div_sc(x, b, r)) != u_of(ref)) ++bad;
    }
  }
  for (long i = 0; i < nr; ++i) {
    const float b = scale(1024 + i), r = 1.0f / b;
    const float lo = b * 0x1p-12f, hi = b * 448.f;
    const uint64_t s = next();
    float x = lo + (hi - lo) * (float)((s >> 11) * 0x1p-53);
    if (s & 1) x = -x;
    if (!isfinite(x) || !isfinite(hi)) continue;
    const float ref = x / b;
    ++checked;
    if (u_of(div_sc(x, b, r)) != u_of(ref)) ++bad;
  }
  printf("checked %ld mismatches %ld\n", checked, bad);
  return bad != 0;
}
