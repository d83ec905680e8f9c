// Host check: grid_round (floating point) against grid_round_int (integer
// operations) for every f32 bit pattern of the binades that matter on grid j
// (x / 2^(j-23) in [2^-3, 2^26)), plus special values, for the j listed on
// the command line.  Prints "ok <count>" or the first mismatch.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include "../llama.zig_amd/csrc/llz_exact.h"

static float bitsf(uint32_t b) { float f; std::memcpy(&f, &b, 4); return f; }

static bool check(uint32_t bits, int j, unsigned long long& n) {
  const float x = bitsf(bits);
  bool t0 = false, t1 = false;
  const uint32_t r0 = llz::grid_round_int(x, j, t0);
  const uint32_t r1 = llz::grid_round(x, j, t1);
  ++n;
  if (r0 != r1 || t0 != t1) {
    std::printf("mismatch j=%d x=%08x: int %u tie %d, fp %u tie %d\n", j, bits, r0, (int)t0, r1, (int)t1);
    return false;
  }
  return true;
}

int main(int argc, char** argv) {
  unsigned long long n = 0;
  const uint32_t specials[] = {0u, 1u, 2u, 0x7fffffu, 0x800000u, 0x7f7fffffu, 0x7f800000u, 0x7fc00000u, 0x7f800001u};
  for (int a = 1; a < argc; ++a) {
    const int j = std::atoi(argv[a]);
    for (uint32_t b : specials)
      if (!check(b, j, n) || !check(b | 0x80000000u, j, n)) return 1;
    // binades of x: exponents E with 2^(E-127) / 2^(j-23) in [2^-3, 2^26)
    for (int E = j + 127 - 26; E <= j + 127 + 2; ++E) {
      if (E < 0 || E > 254) continue;
      const uint32_t base = (uint32_t)E << 23;
      for (uint32_t m = 0; m < (1u << 23); ++m)
        if (!check(base | m, j, n)) return 1;
    }
  }
  std::printf("ok %llu\n", n);
  return 0;
}
