// Host check of the stale-max refresh predicate (csrc/h3a_stale.h) on finite,
// infinite and NaN stage sums.  Built by tests/test_stale_sum.py with the
// library's -fno-honor-nans (clang) and with -ffinite-math-only (gcc), under
// which a float compare could drop the NaN case.  Prints "OK" or the first
// wrong answer.
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "h3a_stale.h"

static float from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, sizeof f);
  return f;
}

// Inputs are read from argv so that no case is a compile-time constant.
int main(int argc, char **argv) {
  struct Case {
    uint32_t bits;
    bool want;
    const char *what;
  } cases[] = {
      {0x00000000u, false, "+0"},
      {0x00000001u, false, "smallest denormal"},
      {0x3f800000u, false, "1"},
      {0x477fff00u, false, "just below 2^16"},
      {0x47800000u, false, "2^16 (the limit)"},
      {0x47800001u, true, "next float above 2^16"},
      {0x4b000000u, true, "2^23"},
      {0x7f7fffffu, true, "largest finite"},
      {0x7f800000u, true, "+inf"},
      {0x7fc00000u, true, "quiet NaN"},
      {0x7f800001u, true, "signalling NaN"},
      {0xffc00000u, true, "negative quiet NaN"},
  };
  const uint32_t salt = argc > 1 ? (uint32_t)argv[1][0] - '0' : 0;  // 0 when run as intended
  for (const Case &c : cases) {
    const float ps = from_bits(c.bits ^ salt);
    if (h3a::stage_sum_needs_refresh(ps) != c.want) {
      printf("stage_sum_needs_refresh(%s, bits 0x%08x) = %d, want %d\n", c.what, c.bits, !c.want, c.want);
      return 1;
    }
  }
  printf("OK\n");
  return 0;
}
