/* Check of the append kernels' scale division (kvbridge_amd/csrc/append.hip,
 * scale_of): for finite a >= 0, with C = RN(1/127), q0 = RN(a * C),
 *   fma(fma(-q0, 127, a), C, q0) == RN(a / 127)   bitwise.
 * Usage: scale_div_check [stride]  -- every stride-th bit pattern of the
 * non-negative finite fp32 range (stride 1: all of them), plus every value an
 * fp16 row maximum can take.  Prints the mismatch count; exit status 1 on any. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int check(uint32_t u, unsigned long long* bad) {
  float a;
  memcpy(&a, &u, 4);
  volatile float ref = a / 127.0f; /* IEEE single division */
  const float c = 1.0f / 127.0f;
  volatile float q0 = a * c;
  const float s = fmaf(fmaf(-q0, 127.0f, a), c, q0);
  const float r = ref;
  if (memcmp(&r, &s, 4) != 0) {
    if (*bad < 5) printf("a=%a ref=%a fast=%a\n", a, r, s);
    ++*bad;
    return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 0) : 61u;
  unsigned long long bad = 0, n = 0;
  for (uint64_t u = 0; u < 0x7f800000u; u += stride, ++n) check((uint32_t)u, &bad);
  check(0x7f7fffffu, &bad); /* largest finite */
  for (uint32_t h = 0; h < 0x7c00u; ++h, ++n) { /* fp16 magnitudes as fp32 */
    const float f = (h >> 10) ? ldexpf(1.0f + (h & 0x3ffu) / 1024.0f, (int)(h >> 10) - 15) : ldexpf((float)h, -24);
    uint32_t u;
    memcpy(&u, &f, 4);
    check(u, &bad);
  }
  printf("scale division: %llu values, %llu mismatches\n", n, bad);
  return bad != 0;
}
