// Host check of the exact accumulator of tallymap_amd/csrc/tm_device.h (test infrastructure): reads f32 values
// (one "%a"-free hex word per line on stdin), emits them into one bin with tm_xemit_with (a plain add standing in
// for the device's int64 atomic), and prints the readout's bits and the flag.
#include <cstdio>
#include <cstdint>
#include "../../tallymap_amd/csrc/tm_device.h"

struct PlainAdd {
  i64 operator()(u64* a, int j, i64 q) const { const i64 o = (i64)a[j]; a[j] = (u64)((u64)o + (u64)q); return o; }
};

int main() {
  u64 w[5] = {0, 0, 0, 0, 0};
  bool flag = false;
  unsigned b;
  while (scanf("%x", &b) == 1) flag = tm_xemit_with(w, tm_u2f(b), PlainAdd()) || flag;
  bool bad = false;
  const float r = tm_xread(w, &bad);
  printf("%08x %d\n", tm_f2u(r), (int)(flag || bad));
  return 0;
}
