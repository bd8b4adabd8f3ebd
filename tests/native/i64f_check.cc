// Host check of the shift-free 64-bit integer -> float32 conversions of tallymap_amd/csrc/tm_device.h (test
// infrastructure): tm_u64f / tm_i64f over edge values, ties and near-ties, and pseudo-random operands at every
// magnitude, against the host compiler's native conversions (rounded to nearest even); prints the mismatch count.
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include "../../tallymap_amd/csrc/tm_device.h"

static unsigned fbits(float f) { unsigned u; memcpy(&u, &f, 4); return u; }

int main() {
  long bad = 0, n = 0;
  auto check = [&](u64 u) {
    ++n;
    if (fbits(tm_u64f(u)) != fbits((float)u)) ++bad;
    const i64 s = (i64)u;
    if (fbits(tm_i64f(s)) != fbits((float)s)) ++bad;
  };
  const u64 edge[] = {0ull, 1ull, ~0ull, 0x8000000000000000ull, 0x7fffffffffffffffull, 0xffffffffull,
                      0x100000000ull, 0x100000001ull, (1ull << 40) + (1ull << 16), (1ull << 40) + (1ull << 16) + 1,
                      (1ull << 40) + 3 * (1ull << 16), (1ull << 63) - (1ull << 38), (1ull << 56) + (1ull << 32) + 1,
                      0xffffff8000000000ull, 0xffffff7fffffffffull, 0x0000008000000001ull};
  for (u64 e : edge) {
    check(e);
    check(0ull - e);
  }
  // ties and their neighbours at every exponent: 24 significant bits, then a half ulp, +-1
  for (int e = 24; e < 64; ++e)
    for (u64 m : {0x800000ull, 0x800001ull, 0xffffffull, 0xabcdefull})
      for (int d = -1; d <= 1; ++d) {
        const u64 t = (m << (e - 23)) + (1ull << (e - 24)) + (u64)(i64)d;
        check(t);
        check(0ull - t);
      }
  u64 r = 0x9e3779b97f4a7c15ull;
  for (int i = 0; i < 2000000; ++i) {      // xorshift64, shifted down to every magnitude
    r ^= r << 13; r ^= r >> 7; r ^= r << 17;
    check(r >> (i % 64));
  }
  printf("%ld %ld\n", bad, n);
  return 0;
}
