/* Check of the append stream kernel's quotient for fp16 and bf16 sources
 * (kvbridge_amd/csrc/append.hip, quantize_lane): with s = RN(a / 127) the
 * scale of a row whose absmax is a, r any fp32 value within one ulp of 1/s
 * (the documented accuracy of v_rcp_f32) and x a source value with |x| <= a,
 *   q0 = RN(x * r),  q = RN(RN(x - q0 * s) * r + q0)   (fma: one rounding each)
 * equals the IEEE quotient RN(x / s) for every such (a, r, x) with
 * s >= 2^-100 -- so rint(q) is the code.  Exhaustive over the 16-bit source
 * formats: every stride-th row maximum a (stride 1: all of them), every r,
 * every x of the format with |x| <= a, both signs.
 * Usage: quant_fmadiv_check fp16|bf16 [stride] [mode]
 *   mode 0: the kernel's formula (default); 1: q0 alone, no residual step;
 *   2: no 2^-100 cutoff.  Modes 1 and 2 are planted mistakes that must fail
 *   (mode 2 on bf16, whose range reaches scales near 2^-126).
 * Prints the counts; exit status 1 on any mismatch.  Threads with OpenMP
 * where the compiler has it. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_fp16(uint32_t h) { /* 15-bit magnitude pattern */
  return (h >> 10) ? ldexpf(1.0f + (float)(h & 0x3ffu) / 1024.0f, (int)(h >> 10) - 15) : ldexpf((float)h, -24);
}

static float from_bf16(uint32_t h) {
  const uint32_t u = h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Every fp32 r with |r - 1/s| <= one ulp of 1/s's binade. */
static int reciprocals(float s, float* out) {
  const double inv = 1.0 / (double)s;
  const double ulp = ldexp(1.0, ilogb(inv) - 23);
  float f = nextafterf(nextafterf((float)inv, 0.0f), 0.0f);
  int n = 0;
  for (int i = 0; i < 5; ++i, f = nextafterf(f, INFINITY))
    if (fabs((double)f - inv) <= ulp) out[n++] = f;
  return n;
}

int main(int argc, char** argv) {
  const int bf = argc > 1 && strcmp(argv[1], "bf16") == 0;
  const uint32_t stride = argc > 2 ? (uint32_t)strtoul(argv[2], 0, 0) : 1u;
  const int mode = argc > 3 ? atoi(argv[3]) : 0;
  const uint32_t inf = bf ? 0x7f80u : 0x7c00u;
  const float cutoff = mode == 2 ? 0.0f : 0x1p-100f;
  unsigned long long n = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : n, bad)
  for (uint32_t ha = 1; ha < inf; ha += stride) {
    const float a = bf ? from_bf16(ha) : from_fp16(ha);
    volatile float sv = a / 127.0f; /* IEEE single division */
    const float s = sv;
    if (!(s >= cutoff) || s == 0.0f) continue; /* the kernel divides these rows */
    float rs[5];
    const int nr = reciprocals(s, rs);
    for (int k = 0; k < nr; ++k) {
      const float r = rs[k];
      if (!(r <= 3.4028234663852886e38f)) continue;
      for (uint32_t hx = 0; hx <= ha; ++hx) {
        const float m = bf ? from_bf16(hx) : from_fp16(hx);
        for (int sg = 0; sg < 2; ++sg) {
          const float x = sg ? -m : m;
          volatile float qv = x / s;
          const float q0 = x * r;
          const float q = mode == 1 ? q0 : fmaf(fmaf(-q0, s, x), r, q0);
          ++n;
          if (rintf(q) != rintf(qv)) {
            if (bad < 5) printf("a=%a x=%a s=%a r=%a q=%a ieee=%a\n", a, x, s, r, q, (float)qv);
            ++bad;
          }
        }
      }
    }
  }
  printf("%s quotient (mode %d, stride %u): %llu checked, %llu mismatches\n", bf ? "bf16" : "fp16", mode, stride, n,
         bad);
  return bad != 0;
}
