// Host check of the 32-bit-half 64-bit shifts of tallymap_amd/csrc/tm_device.h (test infrastructure): every amount
// 0..63 over edge and pseudo-random operands against the host's native 64-bit shifts; prints the mismatch count.
#include <cstdio>
#include "../../tallymap_amd/csrc/tm_device.h"

int main() {
  u64 xs[4096];
  const u64 edge[] = {0ull, 1ull, ~0ull, 0x8000000000000000ull, 0x7fffffffffffffffull, 0xffffffffull,
                      0x100000000ull, 0x80000000ull, 0xffffffff00000000ull, 0x0123456789abcdefull};
  int n = 0;
  for (u64 e : edge) xs[n++] = e;
  u64 r = 0x9e3779b97f4a7c15ull;
  while (n < 4096) {                       // xorshift64
    r ^= r << 13; r ^= r >> 7; r ^= r << 17;
    xs[n++] = r;
  }
  long bad = 0;
  for (int i = 0; i < n; ++i)
    for (u32 s = 0; s < 64u; ++s) {
      const u64 x = xs[i];
      bad += tm_shl64(x, s) != (x << s);
      bad += tm_shr64(x, s) != (x >> s);
      bad += tm_sar64((i64)x, s) != ((i64)x >> s);
    }
  printf("%ld mismatches\n", bad);
  return bad != 0;
}
