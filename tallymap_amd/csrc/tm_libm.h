// tm_libm.h -- the transcendental functions of generated kernels, host + device.
//
// The parity target is the reference's CPU kernel backend, whose transcendentals are glibc's libm (reference
// tallymap/backends/kernel/host.py:43-48, op_table.py:199-223).  glibc's f32 functions are not correctly rounded,
// so the device cannot use its own math library and agree bitwise.  Each function here is written from a published
// method and checked on the host against glibc over the argument sets the tests name (exhaustively where the set
// is enumerable); tests/test_libm.py holds the checks and their results.
//
//   tm_log     double natural log: the classic fdlibm argument reduction and odd-series in s = f / (2 + f)
//              (Sun fdlibm e_log.c, freely redistributable), < 1 ulp.
//   tm_erfinvf f32 erf_inv as the reference's CPU target computes it: Giles (2010)'s single-precision polynomial
//              evaluated in double (log, sqrt), rounded once to f32 (host.py:102-132).  Checked bitwise against
//              the reference formula with glibc's log over every argument jax.random.normal can produce (all 2^23
//              uniform values).
#pragma once

TM_FN double tm_log(double x) {
  const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
  const double two54 = 1.80143985094819840000e+16;
  const double Lg1 = 6.666666666666735130e-01, Lg2 = 3.999999999940941908e-01, Lg3 = 2.857142874366239149e-01,
               Lg4 = 2.222219843214978396e-01, Lg5 = 1.818357216161805012e-01, Lg6 = 1.531383769920937332e-01,
               Lg7 = 1.479819860511658591e-01;
  u64 bits = tm_d2u(x);
  i32 hx = (i32)(bits >> 32);
  u32 lx = (u32)bits;
  i32 k = 0;
  if (hx < 0x00100000) {                         // x < 2^-1022
    if (((hx & 0x7fffffff) | (i32)lx) == 0) return -two54 / 0.0;   // log(+-0) = -inf
    if (hx < 0) return (x - x) / 0.0;                               // log(-#) = NaN
    k -= 54;
    x *= two54;                                  // subnormal: scale up
    bits = tm_d2u(x);
    hx = (i32)(bits >> 32);
  }
  if (hx >= 0x7ff00000) return x + x;
  k += (hx >> 20) - 1023;
  hx &= 0x000fffff;
  const i32 i = (hx + 0x95f64) & 0x100000;
  bits = ((u64)(u32)(hx | (i ^ 0x3ff00000)) << 32) | (u64)(u32)tm_d2u(x);   // normalise x or x/2
  x = tm_u2d(bits);
  k += (i >> 20);
  const double f = x - 1.0;
  if ((0x000fffff & (2 + hx)) < 3) {             // -2^-20 <= f < 2^-20
    if (f == 0.0) {
      if (k == 0) return 0.0;
      const double dk = (double)k;
      return dk * ln2_hi + dk * ln2_lo;
    }
    const double R = f * f * (0.5 - 0.33333333333333333 * f);
    if (k == 0) return f - R;
    const double dk = (double)k;
    return dk * ln2_hi - ((R - dk * ln2_lo) - f);
  }
  const double s = f / (2.0 + f);
  const double dk = (double)k;
  const double z = s * s;
  i32 ii = hx - 0x6147a;
  const double w = z * z;
  const i32 j = 0x6b851 - hx;
  const double t1 = w * (Lg2 + w * (Lg4 + w * Lg6));
  const double t2 = z * (Lg1 + w * (Lg3 + w * (Lg5 + w * Lg7)));
  ii |= j;
  const double R = t2 + t1;
  if (ii > 0) {
    const double hfsq = 0.5 * f * f;
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return dk * ln2_hi - ((hfsq - (s * (hfsq + R) + dk * ln2_lo)) - f);
  }
  if (k == 0) return f - s * (f - R);
  return dk * ln2_hi - ((s * (f - R) - dk * ln2_lo) - f);
}

TM_FN double tm_giles(double y) {
  const double a = y < 0.0 ? -y : y;
  double w = -tm_log((1.0 - a) * (1.0 + a)), p;
  if (w < 5.0) {
    w -= 2.5;
    p = 2.81022636e-08;
    p = 3.43273939e-07 + p * w;
    p = -3.5233877e-06 + p * w;
    p = -4.39150654e-06 + p * w;
    p = 0.00021858087 + p * w;
    p = -0.00125372503 + p * w;
    p = -0.00417768164 + p * w;
    p = 0.246640727 + p * w;
    p = 1.50140941 + p * w;
  } else {
    w = __builtin_sqrt(w) - 3.0;
    p = -0.000200214257;
    p = 0.000100950558 + p * w;
    p = 0.00134934322 + p * w;
    p = -0.00367342844 + p * w;
    p = 0.00573950773 + p * w;
    p = -0.0076224613 + p * w;
    p = 0.00943887047 + p * w;
    p = 1.00167406 + p * w;
    p = 2.83297682 + p * w;
  }
  return p * a;
}

TM_FN float tm_erfinvf(float y) {
  if (!(y > -1.0f && y < 1.0f)) {
    return y == 1.0f ? __builtin_inff() : (y == -1.0f ? -__builtin_inff() : __builtin_nanf(""));
  }
  if (y == 0.0f) return y;
  const double r = tm_giles((double)y);
  return (float)(y < 0.0f ? -r : r);
}
