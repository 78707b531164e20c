/* Check of the append stream kernel's code rounding (kvbridge_amd/csrc/append.hip,
 * quantize_lane, fp32 sources).  The kernel wants c = rint(RN(x / s)) (IEEE single division,
 * round half to even) for a source element x and its row's scale s.  With r a
 * reciprocal of s within one ulp (the documented accuracy of v_rcp_f32),
 *   r_lo = RN(r * (1 - 2^-K)),  r_hi = RN(r * (1 + 2^-K)),  M = 1.5 * 2^23,
 *   lo = RN(x * r_lo + M),      hi = RN(x * r_hi + M)      (single-rounding fma),
 * x * r_lo and x * r_hi bracket RN(x / s); rounding to the nearest integer is
 * monotone, so when lo == hi that integer is c, and lo - M is it.  Where they
 * differ the kernel divides.  This program checks the claim:
 *   - every stride-th fp16 row maximum a (s = RN(a / 127)), every fp32 r within
 *     one ulp of 1/s, every fp16 x with |x| <= a, both signs;
 *   - random fp32 rows (a spread over 2^-100 .. 2^100) with x uniform in
 *     [-a, a] and x = a * j / 254 (the exact ties).
 * Usage: quant_bracket_check [stride] [fp32 samples] [K]
 *   (defaults 5, 20000000, 21; K = 0 takes r_lo = r_hi = r, no bracket, which
 *   must fail).  Prints the counts; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const float kMagic = 12582912.0f; /* 1.5 * 2^23 */
static unsigned long long n_checked, n_bad, n_fallback;
static float g_lo_mul = 1.0f, g_hi_mul = 1.0f;

static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float half_to_float(uint32_t h) { /* h: 15-bit magnitude pattern */
  return (h >> 10) ? ldexpf(1.0f + (float)(h & 0x3ffu) / 1024.0f, (int)(h >> 10) - 15) : ldexpf((float)h, -24);
}

static void check_x(float x, float s, float r_lo, float r_hi) {
  volatile float q = x / s; /* IEEE single division */
  const float want = fminf(fmaxf(rintf(q), -127.0f), 127.0f);
  const float lo = fmaf(x, r_lo, kMagic), hi = fmaf(x, r_hi, kMagic);
  ++n_checked;
  if (bits(lo) != bits(hi)) {
    ++n_fallback;
    return;
  }
  if (lo - kMagic != want) {
    if (n_bad < 5) printf("x=%a s=%a r_lo=%a r_hi=%a got=%g want=%g\n", x, s, r_lo, r_hi, lo - kMagic, want);
    ++n_bad;
  }
}

/* Every fp32 r with |r - 1/s| <= one ulp of 1/s's binade. */
static int reciprocals(float s, float* out) {
  const double inv = 1.0 / (double)s;
  const double ulp = ldexp(1.0, ilogb(inv) - 23);
  float f = (float)inv;
  int n = 0;
  f = nextafterf(nextafterf(f, 0.0f), 0.0f);
  for (int i = 0; i < 5; ++i, f = nextafterf(f, INFINITY))
    if (fabs((double)f - inv) <= ulp) out[n++] = f;
  return n;
}

static void check_row(float s, void (*xs)(float, float, float, float, uint32_t), uint32_t arg) {
  float rs[5];
  const int nr = reciprocals(s, rs);
  for (int i = 0; i < nr; ++i) {
    const float r_lo = rs[i] * g_lo_mul, r_hi = rs[i] * g_hi_mul;
    if (!(r_hi <= 3.4028234663852886e38f)) continue; /* the kernel divides such rows */
    xs(s, rs[i], r_lo, r_hi, arg);
  }
}

static void fp16_xs(float s, float r, float r_lo, float r_hi, uint32_t ha) {
  (void)r;
  for (uint32_t h = 0; h <= ha; ++h) {
    const float x = half_to_float(h);
    check_x(x, s, r_lo, r_hi);
    check_x(-x, s, r_lo, r_hi);
  }
}

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint64_t next_u64(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}
static float uniform01(void) { return (float)(next_u64() >> 40) * 0x1p-24f; }

static float g_a;
static void fp32_xs(float s, float r, float r_lo, float r_hi, uint32_t n) {
  (void)r;
  for (uint32_t i = 0; i < n; ++i) {
    const float x = (2.0f * uniform01() - 1.0f) * g_a;
    check_x(x, s, r_lo, r_hi);
  }
  for (uint32_t j = 0; j <= 254; j += 1 + (uint32_t)(next_u64() % 17)) {
    const float x = g_a * (float)j / 254.0f;
    check_x(x, s, r_lo, r_hi);
    check_x(-x, s, r_lo, r_hi);
  }
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 0) : 5u;
  const unsigned long long samples = argc > 2 ? strtoull(argv[2], 0, 0) : 20000000ull;
  const int k = argc > 3 ? atoi(argv[3]) : 21;
  if (k > 0) {
    g_lo_mul = 1.0f - ldexpf(1.0f, -k);
    g_hi_mul = 1.0f + ldexpf(1.0f, -k);
  }
  for (uint32_t ha = 1; ha < 0x7c00u; ha += stride) {
    const float a = half_to_float(ha);
    volatile float s = a / 127.0f;
    check_row(s, fp16_xs, ha);
  }
  const unsigned long long fp16_checked = n_checked;
  const uint32_t per_row = 64;
  for (unsigned long long done = 0; done < samples; done += per_row) {
    g_a = ldexpf(1.0f + uniform01(), (int)(next_u64() % 201) - 100);
    volatile float s = g_a / 127.0f;
    check_row(s, fp32_xs, per_row);
  }
  printf("code rounding (bracket 2^-%d): %llu fp16 + %llu fp32 elements, %llu divided, %llu mismatches\n", k,
         fp16_checked, n_checked - fp16_checked, n_fallback, n_bad);
  return n_bad != 0;
}
