/* Compares the restated expf (bebelm_amd/csrc/bb_expf.h, built here as plain C) with the
 * platform expf bit for bit over a strided sweep of all 2^32 float bit patterns plus listed
 * inputs. Prints "<checked> <mismatches> <first mismatch bits>". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bb_expf.h"

static int same(float a, float b) {
  if (isnan(a) && isnan(b)) return 1;
  return memcmp(&a, &b, 4) == 0;
}

int main(int argc, char** argv) {
  uint64_t stride = argc > 1 ? strtoull(argv[1], 0, 0) : 61;
  uint64_t checked = 0, bad = 0;
  uint32_t first = 0;
  for (uint64_t u = 0; u < (1ull << 32); u += stride) {
    float x;
    uint32_t v = (uint32_t)u;
    memcpy(&x, &v, 4);
    checked++;
    if (!same(expf(x), bb_expf(x))) { if (!bad) first = v; bad++; }
  }
  for (int i = 2; i < argc; ++i) {
    uint32_t v = (uint32_t)strtoul(argv[i], 0, 0);
    float x;
    memcpy(&x, &v, 4);
    checked++;
    if (!same(expf(x), bb_expf(x))) { if (!bad) first = v; bad++; }
  }
  printf("%llu %llu 0x%08x\n", (unsigned long long)checked, (unsigned long long)bad, first);
  return 0;
}
