// Host check of tm_fmodf / tm_fmod (tallymap_amd/csrc/tm_device.h) against glibc's fmodf / fmod (exact), test
// infrastructure: special values x special values, then pseudo-random pairs over the whole exponent range
// (including subnormals).  Prints the number of mismatches (NaN == NaN) and the first few.
#include <cmath>
#include <cstdio>
#include <cstring>
#include "../../tallymap_amd/csrc/tm_device.h"

static u64 st = 0x9E3779B97F4A7C15ull;
static u64 rnd() { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }

int main(int argc, char** argv) {
  const long n = argc > 1 ? atol(argv[1]) : 20000000;
  long bad = 0, tot = 0;
  const float fs[] = {0.0f, -0.0f, INFINITY, -INFINITY, NAN, 1e-45f, -1e-45f, 1.17549435e-38f, 3e-39f, 1.0f, -1.0f,
                      0.5f, 3.0f, 7.0f, -7.0f, 1e10f, 3.4028235e38f, 2.5f, 0.1f, 16777217.0f};
  auto chkf = [&](float x, float y) {
    const float g = tm_fmodf(x, y), w = fmodf(x, y);
    ++tot;
    if (!((g != g && w != w) || tm_f2u(g) == tm_f2u(w))) {
      if (bad++ < 5) printf("f32 fmod(%a, %a) = %a, glibc %a\n", x, y, g, w);
    }
  };
  auto chkd = [&](double x, double y) {
    const double g = tm_fmod(x, y), w = fmod(x, y);
    ++tot;
    if (!((g != g && w != w) || tm_d2u(g) == tm_d2u(w))) {
      if (bad++ < 5) printf("f64 fmod(%a, %a) = %a, glibc %a\n", x, y, g, w);
    }
  };
  for (float x : fs)
    for (float y : fs) { chkf(x, y); chkd(x, y); chkd(x * 1e-300, y); chkd(x, y * 1e-300); }
  for (long i = 0; i < n; ++i) {
    const u64 r = rnd();
    chkf(tm_u2f((u32)r), tm_u2f((u32)(r >> 32)));
    const u32 a = (u32)r, b = (a & 0x807fffffu) | ((u32)(rnd() % 24u + ((a >> 23) & 255u) - (rnd() % 24u)) & 255u) << 23;
    chkf(tm_u2f(a), tm_u2f(b));                 // (close exponents: long quotients are rare, short ones common)
    if (i % 16 == 0) chkd(tm_u2d(rnd()), tm_u2d(rnd()));
    if (i % 16 == 1) { const u64 q = rnd(); chkd(tm_u2d(q), tm_u2d((q & 0x800fffffffffffffull) | ((((q >> 52) & 2047u) + rnd() % 64u - 32u) & 2047u) << 52)); }
  }
  printf("%ld %ld\n", bad, tot);
  return bad != 0;
}
