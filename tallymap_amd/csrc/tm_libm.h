// tm_libm.h -- the transcendental functions of generated kernels, host + device.
//
// The parity target is the reference's CPU kernel backend, whose transcendentals are glibc's libm (reference
// tallymap/backends/kernel/host.py:43-48, op_table.py:199-223).  glibc's f32 functions are not correctly rounded,
// so the device cannot use its own math library and agree bitwise.  Each function here is written from a published
// method and checked on the host against glibc over the argument sets the tests name (exhaustively where the set
// is enumerable); tests/native/libm_check.cc and tests/test_native_cpu.py hold the checks.
//
//   tm_erfinvf f32 erf_inv as the reference's CPU target computes it: Giles (2010)'s single-precision polynomial
//              evaluated in double, rounded once to f32 (host.py:102-132).  Here the double part is a division-free
//              table log (tm_log_erfinv) and fused multiply-adds; the results are checked bitwise against the
//              reference formula (glibc's log, separate multiplies and adds) on EVERY f32 argument in (-1, 1):
//              2,130,706,430 arguments, 0 mismatches (so on all 2^23 that jax.random.normal produces).
//   tm_logf, tm_expf, tm_sinf, tm_cosf
//              glibc 2.35's f32 functions are the ARM optimized-routines algorithms (MIT / Apache-2.0; Szabolcs
//              Nagy), built on x86-64 in an FMA variant selected at run time on FMA/AVX2 hosts.  Restated here:
//              the same reductions, tables and polynomials, with an explicit fma wherever that build contracts a
//              multiply-add.  Checked bitwise against glibc on ALL 2^32 inputs: logf, sinf, cosf agree
//              everywhere; expf everywhere except two inputs whose glibc result lies on a rounding knife-edge of
//              the same evaluation, listed in tm_expf.  The exp2 table is 2^(i/32) rounded to double, minus i << 47
//              (computed from that definition); the 2/pi bit table is the binary expansion of 2/pi.
//   tm_exp2f, tm_log2f, tm_powf
//              the same library's exp2f / log2f / powf on the expf / logf tables.  exp2f and log2f agree with
//              glibc on all 2^32 inputs; powf on 1.0e9 random pairs (bit patterns, x near 1 with large |y|,
//              integer and non-integer y of both signs) and a grid of special pairs, 0 mismatches.
//   tm_atanf, tm_atan2f
//              fdlibm's float atanf / atan2f (Sun, freely redistributable) in float arithmetic, in glibc's form
//              (atanf returns +-pi/2 from |x| >= 2^25).  Checked bitwise against glibc on all 2^32 atanf arguments
//              and on random atan2f pairs over the full exponent range.
//   tm_expm1f, tm_log1pf, tm_tanhf
//              fdlibm's float expm1f / log1pf / tanhf, float arithmetic without contraction, as glibc 2.35's
//              generic build compiles them: bitwise equal to glibc on all 2^32 inputs.
//   tm_logisticf
//              1 / (1 + tm_expf(-x)), the reference CPU target's expression: all 2^32 inputs bitwise.
//
// Upstream notices of the restated code (the logf / expf / exp2f / log2f / powf / sinf / cosf reductions, tables
// and polynomial coefficients, and the atanf / atan2f / expm1f / log1pf / tanhf code and coefficients):
//
//   ARM optimized-routines (math/logf.c, math/expf.c, math/exp2f.c, math/log2f.c, math/powf.c, math/sinf.c,
//   math/cosf.c and their data files):
//     Copyright (c) 2017-2022, Arm Limited.
//     SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception.  Used here under the MIT license:
//     Permission is hereby granted, free of charge, to any person obtaining a copy of this software and
//     associated documentation files (the "Software"), to deal in the Software without restriction, including
//     without limitation the rights to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
//     copies of the Software, and to permit persons to whom the Software is furnished to do so, subject to the
//     following conditions: The above copyright notice and this permission notice shall be included in all copies
//     or substantial portions of the Software.  THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
//     EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY, FITNESS FOR A PARTICULAR
//     PURPOSE AND NONINFRINGEMENT.  IN NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
//     DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM, OUT OF OR IN
//     CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE SOFTWARE.
//
//   fdlibm (s_atanf.c, e_atan2f.c, s_expm1f.c, s_log1pf.c, s_tanhf.c; float versions by Ian Lance Taylor,
//   Cygnus Support):
//     Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//     Developed at SunPro, a Sun Microsystems, Inc. business.
//     Permission to use, copy, modify, and distribute this software is freely granted, provided that this notice
//     is preserved.
#pragma once

// w = -log(t) for erf_inv, t = (1 - a)(1 + a) in [2^-24, 1]: t = 2^k z, z in [0x1.6ap-1, 0x1.6ap0) split into 64
// equal pieces by the top six mantissa bits; log t = k ln2 + log c + log1p(z / c - 1) with 1/c the piece's
// midpoint reciprocal rounded to double, log c = -log(1/c) rounded to double (both from their definitions at 60
// digits), and log1p(r), |r| < 2^-7, by its Taylor series to r^8 (remainder < 2^-63).  No division.  The absolute
// error is below 4e-16 on this domain; erf_inv reads w through w - 2.5 or sqrt(w), so absolute accuracy is what
// matters (the function is not a general-purpose log: its relative error near t = 1 is large).
TM_FN double tm_log_erfinv(double x) {
  const double T[64][2] = {
      {0x1.6816816816817p+0, -0x1.5d5bddf595f31p-2},
      {0x1.642c8590b2164p+0, -0x1.522ae0738a3d7p-2},
      {0x1.6058160581606p+0, -0x1.4718dc271c41cp-2},
      {0x1.5c9882b931057p+0, -0x1.3c25277333183p-2},
      {0x1.58ed2308158edp+0, -0x1.314f1e1d35ce3p-2},
      {0x1.5555555555555p+0, -0x1.269621134db91p-2},
      {0x1.51d07eae2f815p+0, -0x1.1bf99635a6b95p-2},
      {0x1.4e5e0a72f0539p+0, -0x1.1178e8227e47ap-2},
      {0x1.4afd6a052bf5bp+0, -0x1.07138604d5864p-2},
      {0x1.47ae147ae147bp+0, -0x1.f991c6cb3b37ap-3},
      {0x1.446f86562d9fbp+0, -0x1.e530effe71013p-3},
      {0x1.4141414141414p+0, -0x1.d1037f2655e7bp-3},
      {0x1.3e22cbce4a902p+0, -0x1.bd087383bd8aap-3},
      {0x1.3b13b13b13b14p+0, -0x1.a93ed3c8ad9e5p-3},
      {0x1.3813813813814p+0, -0x1.95a5adcf70182p-3},
      {0x1.3521cfb2b78c1p+0, -0x1.823c16551a3c0p-3},
      {0x1.323e34a2b10bfp+0, -0x1.6f0128b756ab9p-3},
      {0x1.2f684bda12f68p+0, -0x1.5bf406b543db0p-3},
      {0x1.2c9fb4d812ca0p+0, -0x1.4913d8333b563p-3},
      {0x1.29e4129e4129ep+0, -0x1.365fcb0159014p-3},
      {0x1.27350b8812735p+0, -0x1.23d712a49c201p-3},
      {0x1.2492492492492p+0, -0x1.1178e8227e47ap-3},
      {0x1.21fb78121fb78p+0, -0x1.fe89139dbd565p-4},
      {0x1.1f7047dc11f70p+0, -0x1.da7276384469ep-4},
      {0x1.1cf06ada2811dp+0, -0x1.b6ac88dad5b1dp-4},
      {0x1.1a7b9611a7b96p+0, -0x1.9335e5d594988p-4},
      {0x1.1811811811812p+0, -0x1.700d30aeac0e8p-4},
      {0x1.15b1e5f75270dp+0, -0x1.4d3115d207eacp-4},
      {0x1.135c81135c811p+0, -0x1.2aa04a44717a1p-4},
      {0x1.1111111111111p+0, -0x1.08598b59e3a06p-4},
      {0x1.0ecf56be69c90p+0, -0x1.ccb73cdddb2d0p-5},
      {0x1.0c9714fbcda3bp+0, -0x1.894aa149fb34bp-5},
      {0x1.0a6810a6810a7p+0, -0x1.466aed42de3f9p-5},
      {0x1.0842108421084p+0, -0x1.0415d89e74440p-5},
      {0x1.0624dd2f1a9fcp+0, -0x1.8492528c8cac5p-6},
      {0x1.0410410410410p+0, -0x1.0205658935837p-6},
      {0x1.0204081020408p+0, -0x1.010157588de69p-7},
      {0x1.ff007fc01ff00p-1, 0x1.ff802a9ab11e6p-10},
      {0x1.f81f81f81f820p-1, 0x1.fc0a8b0fc03c4p-7},
      {0x1.f07c1f07c1f08p-1, 0x1.f829b0e7832f8p-6},
      {0x1.e9131abf0b767p-1, 0x1.77458f632dcffp-5},
      {0x1.e1e1e1e1e1e1ep-1, 0x1.f0a30c01162a8p-5},
      {0x1.dae6076b981dbp-1, 0x1.341d7961bd1d0p-4},
      {0x1.d41d41d41d41dp-1, 0x1.6f0d28ae56b4ep-4},
      {0x1.cd85689039b0bp-1, 0x1.a926d3a4ad562p-4},
      {0x1.c71c71c71c71cp-1, 0x1.e27076e2af2eap-4},
      {0x1.c0e070381c0e0p-1, 0x1.0d77e7cd08e5bp-3},
      {0x1.bacf914c1bad0p-1, 0x1.29552f81ff521p-3},
      {0x1.b4e81b4e81b4fp-1, 0x1.44d2b6ccb7d1cp-3},
      {0x1.af286bca1af28p-1, 0x1.5ff3070a793d6p-3},
      {0x1.a98ef606a63bep-1, 0x1.7ab890210d907p-3},
      {0x1.a41a41a41a41ap-1, 0x1.9525a9cf456b6p-3},
      {0x1.9ec8e951033d9p-1, 0x1.af3c94e80bff3p-3},
      {0x1.999999999999ap-1, 0x1.c8ff7c79a9a20p-3},
      {0x1.948b0fcd6e9e0p-1, 0x1.e27076e2af2e8p-3},
      {0x1.8f9c18f9c18fap-1, 0x1.fb9186d5e3e29p-3},
      {0x1.8acb90f6bf3aap-1, 0x1.0a324e27390e2p-2},
      {0x1.8618618618618p-1, 0x1.1675cababa60fp-2},
      {0x1.8181818181818p-1, 0x1.22941fbcf7966p-2},
      {0x1.7d05f417d05f4p-1, 0x1.2e8e2bae11d31p-2},
      {0x1.78a4c8178a4c8p-1, 0x1.3a64c556945eap-2},
      {0x1.745d1745d1746p-1, 0x1.4618bc21c5ec2p-2},
      {0x1.702e05c0b8170p-1, 0x1.51aad872df82ep-2},
      {0x1.6c16c16c16c17p-1, 0x1.5d1bdbf5809cap-2}};
  const u64 OFF = 0x3fe6a00000000000ull;
  const double Ln2hi = 0x1.62e42fefa3800p-1, Ln2lo = 0x1.ef35793c76730p-45;
  const u64 ix = tm_d2u(x);
  const u64 tmp = ix - OFF;
  const int i = (int)((tmp >> 46) & 63u);
  const i64 k = (i64)tmp >> 52;
  const double z = tm_u2d(ix - (tmp & (0xfffull << 52)));
  const double r = __builtin_fma(z, T[i][0], -1.0);
  const double kd = (double)k;
  const double r2 = r * r;
  double q = __builtin_fma(r, -0.125, 0x1.2492492492492p-3);
  q = __builtin_fma(r, q, -0x1.5555555555555p-3);
  q = __builtin_fma(r, q, 0x1.999999999999ap-3);
  q = __builtin_fma(r, q, -0.25);
  q = __builtin_fma(r, q, 0x1.5555555555555p-2);
  q = __builtin_fma(r, q, -0.5);
  const double hi = __builtin_fma(kd, Ln2hi, T[i][1]);
  return (hi + r) + __builtin_fma(r2, q, kd * Ln2lo);
}

// Giles (2010), "Approximating the erfinv function", the single-precision coefficients, evaluated in double with
// fused multiply-adds (host.py:107-118 evaluates the same polynomial with separate multiplies and adds and glibc's
// log; the f32 results agree bitwise on every f32 argument in (-1, 1): see tm_erfinvf).
TM_FN double tm_giles(double y) {
  const double a = y < 0.0 ? -y : y;
  double w = -tm_log_erfinv((1.0 - a) * (1.0 + a)), p;
  if (w < 5.0) {
    w -= 2.5;
    p = 2.81022636e-08;
    p = __builtin_fma(p, w, 3.43273939e-07);
    p = __builtin_fma(p, w, -3.5233877e-06);
    p = __builtin_fma(p, w, -4.39150654e-06);
    p = __builtin_fma(p, w, 0.00021858087);
    p = __builtin_fma(p, w, -0.00125372503);
    p = __builtin_fma(p, w, -0.00417768164);
    p = __builtin_fma(p, w, 0.246640727);
    p = __builtin_fma(p, w, 1.50140941);
  } else {
    w = __builtin_sqrt(w) - 3.0;
    p = -0.000200214257;
    p = __builtin_fma(p, w, 0.000100950558);
    p = __builtin_fma(p, w, 0.00134934322);
    p = __builtin_fma(p, w, -0.00367342844);
    p = __builtin_fma(p, w, 0.00573950773);
    p = __builtin_fma(p, w, -0.0076224613);
    p = __builtin_fma(p, w, 0.00943887047);
    p = __builtin_fma(p, w, 1.00167406);
    p = __builtin_fma(p, w, 2.83297682);
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

// ------------------------------------------------------------------------------------------------ logf
// x = 2^k z, z in [0x3f330000, 2 * 0x3f330000); c near the center of z's sixteenth; log x = k ln2 + log c +
// log1p(z / c - 1), the last by a degree-4 polynomial in r = z * (1/c) - 1 evaluated in double.
TM_FN float tm_logf(float x) {
  const double T[16][2] = {
      {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
      {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
      {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
      {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
      {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
      {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
      {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
      {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2},  {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}};
  const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2;
  const double Ln2 = 0x1.62e42fefa39efp-1;
  u32 ix = tm_f2u(x);
  if (ix == 0x3f800000u) return 0.0f;
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2u == 0u) return -__builtin_inff();
    if (ix == 0x7f800000u) return x;
    if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return __builtin_nanf("");
    ix = tm_f2u(x * 0x1p23f);                     // a subnormal: normalise
    ix -= 23u << 23;
  }
  const u32 tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> 19) % 16u);
  const int k = (i32)tmp >> 23;
  const u32 iz = ix - (tmp & 0xff800000u);
  const double z = (double)tm_u2f(iz);
  const double r = __builtin_fma(z, T[i][0], -1.0);
  const double y0 = __builtin_fma((double)k, Ln2, T[i][1]);
  const double r2 = r * r;
  double y = __builtin_fma(A1, r, A2);
  y = __builtin_fma(A0, r2, y);
  y = __builtin_fma(y, r2, y0 + r);
  return (float)y;
}

// ------------------------------------------------------------------------------------------------ expf
// x * 32 / ln2 = k + r, |r| <= 1/2; exp x = 2^(k/32) 2^(r/32), 2^(k/32) from the table (exponent added to the
// bits), 2^(r/32) by a cubic in r.
TM_FN float tm_expf(float x) {
  const u64 T[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  const double InvLn2N = 0x1.71547652b82fep+0 * 32, SHIFT = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const u32 ux = tm_f2u(x);
  if (ux == 0x4202422fu) return 0x1.f93e38p+46f;         // the two knife-edge inputs (see the header)
  if (ux == 0xc27c65d9u) return 0x1.f45326p-92f;
  const u32 abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= (tm_f2u(88.0f) >> 20)) {
    if (ux == tm_f2u(-__builtin_inff())) return 0.0f;
    if (abstop >= (tm_f2u(__builtin_inff()) >> 20)) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  double z = InvLn2N * (double)x;
  double kd = z + SHIFT;
  const u64 ki = tm_d2u(kd);
  kd -= SHIFT;
  const double r = z - kd;
  u64 t = T[ki % 32u];
  t += ki << 47;
  const double s = tm_u2d(t);
  z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// ------------------------------------------------------------------------------------------ sinf / cosf
// ARM's __sincosf_table[0] as constants.  Its second table is the same with the cosine coefficients c0..c4 negated,
// and a polynomial with every coefficient negated gives exactly the negated result (each fma and the final rounding
// are symmetric under negation), so the device keeps one constant set and flips the sign of the cosine result
// instead of selecting a table per lane: a per-lane table address turns every coefficient into a global load.
constexpr double TM_SC_HPI_INV = 0x1.45F306DC9C883p+23, TM_SC_HPI = 0x1.921FB54442D18p0;
constexpr double TM_SC_C0 = 0x1p0, TM_SC_C1 = -0x1.ffffffd0c621cp-2, TM_SC_C2 = 0x1.55553e1068f19p-5,
                 TM_SC_C3 = -0x1.6c087e89a359dp-10, TM_SC_C4 = 0x1.99343027bf8c3p-16;
constexpr double TM_SC_S1 = -0x1.555545995a603p-3, TM_SC_S2 = 0x1.1107605230bc4p-7, TM_SC_S3 = -0x1.994eb3774cf24p-13;
// the table's sign[n & 3] = {1, -1, -1, 1}: -1 when bits 0 and 1 of n differ
TM_FN double tm_sc_sign(int n) { return ((n ^ (n >> 1)) & 1) ? -1.0 : 1.0; }
// n even: the sine polynomial; n odd: the cosine polynomial, negated when `flip` (the second table).  Both are
// evaluated and one is selected: the lanes of a wave reduce to quadrants of both parities, and a branch would run
// both sides anyway, each with part of the lanes (each polynomial's operations are glibc's, so the bits are too).
TM_FN float tm_sc_poly(double x, double x2, int n, bool flip) {
  const double x3 = x * x2;
  const double s1 = __builtin_fma(x2, TM_SC_S3, TM_SC_S2);
  const double x7 = x3 * x2;
  const double s = __builtin_fma(x3, TM_SC_S1, x);
  const float rs = (float)__builtin_fma(x7, s1, s);
  const double x4 = x2 * x2;
  const double c2 = __builtin_fma(x2, TM_SC_C4, TM_SC_C3);
  const double c1 = __builtin_fma(x2, TM_SC_C1, TM_SC_C0);
  const double x6 = x4 * x2;
  const double c = __builtin_fma(x4, TM_SC_C2, c1);
  const float rc = (float)__builtin_fma(x6, c2, c);
  return (n & 1) == 0 ? rs : (flip ? -rc : rc);
}
// |x| < 120: n = round(x 2/pi) (through 2^24-scaled integer arithmetic), x - n pi/2 with one fma
TM_FN double tm_sc_reduce_fast(double x, int* np) {
  const double r = x * TM_SC_HPI_INV;
  const int n = ((i32)r + 0x800000) >> 24;
  *np = n;
  return __builtin_fma(-(double)n, TM_SC_HPI, x);
}
// |x| >= 120: x (4/pi) mod 4 in 64-bit fixed point from a 2/pi bit table
TM_FN double tm_sc_reduce_large(u32 xi, int* np) {
  const u32 P[24] = {0xa2u, 0xa2f9u, 0xa2f983u, 0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u, 0x6e4e4415u, 0x4e441529u,
                     0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u, 0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu,
                     0xf534ddc0u, 0x34ddc0dbu, 0xddc0db62u, 0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u,
                     0x993c4390u, 0x3c439041u};
  const u32* arr = &P[(xi >> 26) & 15u];
  const int shift = (int)((xi >> 23) & 7u);
  xi = (xi & 0xffffffu) | 0x800000u;
  xi <<= shift;
  u64 res0 = (u64)(u32)(xi * arr[0]);
  const u64 res1 = (u64)xi * arr[4];
  const u64 res2 = (u64)xi * arr[8];
  res0 = (res2 >> 32) | (res0 << 32);
  res0 += res1;
  const u64 n = (res0 + (1ull << 61)) >> 62;
  res0 -= n << 62;
  *np = (int)n;
  return (double)(i64)res0 * 0x1.921FB54442D18p-62;
}
TM_FN u32 tm_abstop12(float x) { return (tm_f2u(x) >> 20) & 0x7ffu; }
// glibc evaluates |y| < pi/4 without the reduction and returns y itself below 2^-12; there the fast reduction gives
// n = 0 and r = y exactly, and the same polynomial: one path for every |y| < 120, so the lanes of a wave do not
// split on |y| < pi/4, with y itself selected below 2^-12 (the polynomial turns -0 into +0).  Bitwise glibc's on
// all 2^32 inputs.
TM_FN float tm_sinf(float y) {
  double x = y;
  int n;
  if (tm_abstop12(y) < tm_abstop12(120.0f)) {
    x = tm_sc_reduce_fast(x, &n);
    const double s = tm_sc_sign(n);
    const float r = tm_sc_poly(x * s, x * x, n, (n & 2) != 0);
    return tm_abstop12(y) < tm_abstop12(0x1p-12f) ? y : r;
  }
  if (tm_abstop12(y) < tm_abstop12(__builtin_inff())) {
    const u32 xi = tm_f2u(y);
    const int sign = (int)(xi >> 31);
    x = tm_sc_reduce_large(xi, &n);
    const double s = tm_sc_sign(n + sign);
    return tm_sc_poly(x * s, x * x, n, ((n + sign) & 2) != 0);
  }
  return y - y;
}
TM_FN float tm_cosf(float y) {             // (one path for |y| < 120, as tm_sinf; glibc returns 1 below 2^-12)
  double x = y;
  int n;
  if (tm_abstop12(y) < tm_abstop12(120.0f)) {
    x = tm_sc_reduce_fast(x, &n);
    const double s = tm_sc_sign(n);
    const float r = tm_sc_poly(x * s, x * x, n ^ 1, (n & 2) != 0);
    return tm_abstop12(y) < tm_abstop12(0x1p-12f) ? 1.0f : r;
  }
  if (tm_abstop12(y) < tm_abstop12(__builtin_inff())) {
    const u32 xi = tm_f2u(y);
    const int sign = (int)(xi >> 31);
    x = tm_sc_reduce_large(xi, &n);
    const double s = tm_sc_sign(n + sign);
    return tm_sc_poly(x * s, x * x, n ^ 1, ((n + sign) & 2) != 0);
  }
  return y - y;
}

// -------------------------------------------------------------------------------------- atanf / atan2f
TM_FN float tm_atanf(float x) {
  const float atanhi[4] = {4.6364760399e-01f, 7.8539812565e-01f, 9.8279368877e-01f, 1.5707962513e+00f};
  const float atanlo[4] = {5.0121582440e-09f, 3.7748947079e-08f, 3.4473217170e-08f, 7.5497894159e-08f};
  const float aT[11] = {3.3333334327e-01f, -2.0000000298e-01f, 1.4285714924e-01f, -1.1111110449e-01f,
                        9.0908870101e-02f, -7.6918758452e-02f, 6.6610731184e-02f, -5.8335702866e-02f,
                        4.9768779427e-02f, -3.6531571299e-02f, 1.6285819933e-02f};
  const i32 hx = (i32)tm_f2u(x), ix = hx & 0x7fffffff;
  int id;
  if (ix >= 0x4c000000) {                          // |x| >= 2^25
    if (ix > 0x7f800000) return x + x;
    return hx > 0 ? atanhi[3] + atanlo[3] : -atanhi[3] - atanlo[3];
  }
  if (ix < 0x3ee00000) {
    if (ix < 0x31000000) return x;
    id = -1;
  } else {
    x = __builtin_fabsf(x);
    if (ix < 0x3f980000) {
      if (ix < 0x3f300000) { id = 0; x = (2.0f * x - 1.0f) / (2.0f + x); }
      else { id = 1; x = (x - 1.0f) / (x + 1.0f); }
    } else {
      if (ix < 0x401c0000) { id = 2; x = (x - 1.5f) / (1.0f + 1.5f * x); }
      else { id = 3; x = -1.0f / x; }
    }
  }
  const float z = x * x, w = z * z;
  const float s1 = z * (aT[0] + w * (aT[2] + w * (aT[4] + w * (aT[6] + w * (aT[8] + w * aT[10])))));
  const float s2 = w * (aT[1] + w * (aT[3] + w * (aT[5] + w * (aT[7] + w * aT[9]))));
  if (id < 0) return x - x * (s1 + s2);
  const float r = atanhi[id] - ((x * (s1 + s2) - atanlo[id]) - x);
  return hx < 0 ? -r : r;
}
TM_FN float tm_atan2f(float y, float x) {
  const float tiny = 1.0e-30f, pi_o_4 = 7.8539818525e-01f, pi_o_2 = 1.5707963705e+00f, pi = 3.1415927410e+00f,
              pi_lo = -8.7422776573e-08f;
  const i32 hx = (i32)tm_f2u(x), ix = hx & 0x7fffffff, hy = (i32)tm_f2u(y), iy = hy & 0x7fffffff;
  if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;
  if (hx == 0x3f800000) return tm_atanf(y);
  const int m = ((hy >> 31) & 1) | ((hx >> 30) & 2);
  if (iy == 0) return m == 0 || m == 1 ? y : (m == 2 ? pi + tiny : -pi - tiny);
  if (ix == 0) return hy < 0 ? -pi_o_2 - tiny : pi_o_2 + tiny;
  if (ix == 0x7f800000) {
    if (iy == 0x7f800000) {
      return m == 0 ? pi_o_4 + tiny : (m == 1 ? -pi_o_4 - tiny : (m == 2 ? 3.0f * pi_o_4 + tiny : -3.0f * pi_o_4 - tiny));
    }
    return m == 0 ? 0.0f : (m == 1 ? -0.0f : (m == 2 ? pi + tiny : -pi - tiny));
  }
  if (iy == 0x7f800000) return hy < 0 ? -pi_o_2 - tiny : pi_o_2 + tiny;
  const i32 k = (iy - ix) >> 23;
  float z;
  if (k > 60) z = pi_o_2 + 0.5f * pi_lo;
  else if (hx < 0 && k < -60) z = 0.0f;
  else z = tm_atanf(__builtin_fabsf(y / x));
  switch (m) {
    case 0: return z;
    case 1: return tm_u2f(tm_f2u(z) ^ 0x80000000u);
    case 2: return pi - (z - pi_lo);
    default: return (z - pi_lo) - pi;
  }
}
// ----------------------------------------------------------------------------------------------- exp2f
// the exp2f of glibc 2.35 (ARM optimized-routines): x = k/32 + r, |r| <= 1/64; 2^(k/32) from tm_expf's table, 2^r by
// a cubic (the unscaled coefficients of tm_expf's polynomial: C_i here = C_i there x 32^(3-i)).
TM_FN double tm_exp2_table(u64 ki) {
  const u64 T[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  u64 t = T[ki % 32u];
  t += ki << 47;
  return tm_u2d(t);
}
TM_FN float tm_exp2f(float x) {
  const double SHIFT = 0x1.8p+52 / 32, C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3,
               C2 = 0x1.62e42ff0c52d6p-1;
  const u32 ux = tm_f2u(x);
  const u32 abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= (tm_f2u(128.0f) >> 20)) {
    if (ux == tm_f2u(-__builtin_inff())) return 0.0f;
    if (abstop >= (tm_f2u(__builtin_inff()) >> 20)) return x + x;
    if (x > 0.0f) return __builtin_inff();
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = xd + SHIFT;
  const u64 ki = tm_d2u(kd);
  kd -= SHIFT;
  const double r = xd - kd;
  const double s = tm_exp2_table(ki);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// ----------------------------------------------------------------------------------------------- log2f
// the log2f of glibc 2.35 (ARM optimized-routines): tm_logf's reduction and invc values; log2 c = -log2(invc)
// rounded to double (computed from that definition, as tm_logf's log c = -log(invc) is); log1p(r) / ln2 by a
// quartic in double.
TM_FN float tm_log2f(float x) {
  const double T[16][2] = {
      {0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2}, {0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2},
      {0x1.49539f0f010b0p+0, -0x1.7418b0a1fb77bp-2}, {0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7bp-2},
      {0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2}, {0x1.25e227b0b8ea0p+0, -0x1.97c1d1b3b7af0p-3},
      {0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3}, {0x1.12358f08ae5bap+0, -0x1.960cbbf788d5cp-4},
      {0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5}, {0x1.0000000000000p+0, 0x0.0p+0},
      {0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53dp-4}, {0x1.ca4b31f026aa0p-1, 0x1.476a9543891bap-3},
      {0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3}, {0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2},
      {0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2}, {0x1.767dcf5534862p-1, 0x1.ce0a44eb17bccp-2}};
  const double A0 = -0x1.712b6f70a7e4dp-2, A1 = 0x1.ecabf496832ep-2, A2 = -0x1.715479ffae3dep-1,
               A3 = 0x1.715475f35c8b8p0;
  u32 ix = tm_f2u(x);
  if (ix == 0x3f800000u) return 0.0f;
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2u == 0u) return -__builtin_inff();
    if (ix == 0x7f800000u) return x;
    if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return __builtin_nanf("");
    ix = tm_f2u(x * 0x1p23f);
    ix -= 23u << 23;
  }
  const u32 tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> 19) % 16u);
  const u32 top = tmp & 0xff800000u;
  const u32 iz = ix - top;
  const int k = (i32)tmp >> 23;
  const double z = (double)tm_u2f(iz);
  const double r = __builtin_fma(z, T[i][0], -1.0);
  const double y0 = T[i][1] + (double)k;
  const double r2 = r * r;
  double y = __builtin_fma(A1, r, A2);
  y = __builtin_fma(A0, r2, y);
  const double p = __builtin_fma(A3, r, y0);
  y = __builtin_fma(y, r2, p);
  return (float)y;
}

// ---------------------------------------------------------------------------------------------- expm1f
// fdlibm's float expm1f as glibc 2.35 builds it (generic code, float arithmetic, no contraction): x = k ln2 + r,
// |r| <= ln2 / 2 (hi / lo parts), expm1(r) by a rational form with R(r^2/2) (five coefficients), then
// 2^k (1 + expm1(r)) - 1 assembled so that no cancellation loses bits.
TM_FN float tm_expm1f(float x) {
  const float huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f,
              ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f, Q1 = -3.3333335072e-02f,
              Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  i32 k;
  u32 hx = tm_f2u(x);
  const u32 xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {                       // |x| >= 27 ln2
    if (hx >= 0x42b17218u) {                     // |x| >= 88.721...
      if (hx > 0x7f800000u) return x + x;
      if (hx == 0x7f800000u) return xsb == 0u ? x : -1.0f;
      if (x > o_threshold) return huge * huge;
    }
    if (xsb != 0u) {                             // x < -27 ln2
      if (x + tiny < 0.0f) return tiny - 1.0f;
    }
  }
  if (hx > 0x3eb17218u) {                        // |x| > 0.5 ln2
    if (hx < 0x3F851592u) {                      // and |x| < 1.5 ln2
      if (xsb == 0u) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
      else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
    } else {
      k = (i32)(invln2 * x + (xsb == 0u ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {                 // |x| < 2^-25
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0f - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return 1.0f + 2.0f * (x - e);
  }
  if (k <= -2 || k > 56) {                       // suffice to return exp(x) - 1
    i32 i;
    y = 1.0f - (e - x);
    i = (i32)tm_f2u(y);
    y = tm_u2f((u32)(i + (k << 23)));
    return y - 1.0f;
  }
  if (k < 23) {
    t = tm_u2f(0x3f800000u - (0x1000000u >> k));   // 1 - 2^-k
    y = t - (e - x);
    y = tm_u2f((u32)((i32)tm_f2u(y) + (k << 23)));
  } else {
    t = tm_u2f((u32)((0x7f - k) << 23));         // 2^-k
    y = x - (e + t);
    y += 1.0f;
    y = tm_u2f((u32)((i32)tm_f2u(y) + (k << 23)));
  }
  return y;
}

// ---------------------------------------------------------------------------------------------- log1pf
// fdlibm's float log1pf as glibc 2.35 builds it: 1 + x = 2^k (1 + f), sqrt(2)/2 < 1 + f < sqrt(2), a correction
// term c for the rounding of 1 + x, log(1 + f) = f - s (f - R) with s = f / (2 + f) and R a polynomial in s^2.
TM_FN float tm_log1pf(float x) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, two25 = 3.355443200e+07f,
              Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
              Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f, Lp7 = 1.4798198640e-01f;
  float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
  i32 k, hu = 0;
  const i32 hx = (i32)tm_f2u(x);
  const i32 ax = hx & 0x7fffffff;
  k = 1;
  if (hx < 0x3ed413d7) {                         // x < 0.41422
    if (ax >= 0x3f800000) {                      // x <= -1
      if (x == -1.0f) return -__builtin_inff();
      return __builtin_nanf("");
    }
    if (ax < 0x31000000) {                       // |x| < 2^-29
      if (ax < 0x24800000) return x;             // |x| < 2^-54
      return x - x * x * 0.5f;
    }
    if (hx > 0 || hx <= (i32)0xbe95f61fu) { k = 0; f = x; hu = 1; }     // -0.2929 < x < 0.41422
  } else if (hx >= 0x7f800000) {
    return x + x;
  }
  if (k != 0) {
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (i32)tm_f2u(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);      // the rounding of 1 + x
      c /= u;
    } else {
      u = x;
      hu = (i32)tm_f2u(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = tm_u2f((u32)(hu | 0x3f800000));        // normalise u
    } else {
      k += 1;
      u = tm_u2f((u32)(hu | 0x3f000000));        // normalise u / 2
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  hfsq = 0.5f * f * f;
  if (hu == 0) {                                 // |f| < 2^-20
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += (float)k * ln2_lo;
      return (float)k * ln2_hi + c;
    }
    R = hfsq * (1.0f - 0.66666666666666666f * f);
    if (k == 0) return f - R;
    return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
  }
  s = f / (2.0f + f);
  z = s * s;
  R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

// ----------------------------------------------------------------------------------------------- tanhf
// fdlibm's float tanhf as glibc 2.35 builds it, on tm_expm1f: |x| < 1: -t / (t + 2) with t = expm1(-2|x|);
// 1 <= |x| < 22: 1 - 2 / (expm1(2|x|) + 2); beyond, +-1.
TM_FN float tm_tanhf(float x) {
  const i32 jx = (i32)tm_f2u(x), ix = jx & 0x7fffffff;
  float t, z;
  if (ix >= 0x7f800000) return jx >= 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
  if (ix < 0x41b00000) {                         // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000) return x * (1.0f + x);  // |x| < 2^-55
    if (ix >= 0x3f800000) {
      t = tm_expm1f(2.0f * __builtin_fabsf(x));
      z = 1.0f - 2.0f / (t + 2.0f);
    } else {
      t = tm_expm1f(-2.0f * __builtin_fabsf(x));
      z = -t / (t + 2.0f);
    }
  } else {
    z = 1.0f - 1.0e-30f;
  }
  return jx >= 0 ? z : -z;
}

// ---------------------------------------------------------------------------------------------- logistic
// lax.logistic as the reference's CPU target computes it (op_table.py:243-247): 1 / (1 + expf(-x)), IEEE.
TM_FN float tm_logisticf(float x) { return 1.0f / (1.0f + tm_expf(-x)); }

// ------------------------------------------------------------------------------------------------ powf
// the powf of glibc 2.35 (ARM optimized-routines): x^y = 2^(y log2 x), log2 x in double from tm_log2f's table by a
// quintic, 2^t from tm_exp2f's table and cubic with the result's sign folded into the table index for negative x
// with odd integer y; special cases first (y zero / inf / NaN, x zero / inf / NaN, negative x, subnormal x).
TM_FN int tm_powf_checkint(u32 iy) {              // 0: not an integer, 1: odd, 2: even
  const int e = (int)(iy >> 23 & 0xffu);
  if (e < 0x7f) return 0;
  if (e > 0x7f + 23) return 2;
  if (iy & ((1u << (0x7f + 23 - e)) - 1u)) return 0;
  if (iy & (1u << (0x7f + 23 - e))) return 1;
  return 2;
}
TM_FN bool tm_zeroinfnanf(u32 ix) { return 2u * ix - 1u >= 2u * 0x7f800000u - 1u; }
TM_FN bool tm_issnanf(u32 ix) { return (ix & 0x7fc00000u) == 0x7f800000u && (ix & 0x7fffffu) != 0u; }
TM_FN float tm_powf(float x, float y) {
  const double T[16][2] = {
      {0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2}, {0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2},
      {0x1.49539f0f010b0p+0, -0x1.7418b0a1fb77bp-2}, {0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7bp-2},
      {0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2}, {0x1.25e227b0b8ea0p+0, -0x1.97c1d1b3b7af0p-3},
      {0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3}, {0x1.12358f08ae5bap+0, -0x1.960cbbf788d5cp-4},
      {0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5}, {0x1.0000000000000p+0, 0x0.0p+0},
      {0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53dp-4}, {0x1.ca4b31f026aa0p-1, 0x1.476a9543891bap-3},
      {0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3}, {0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2},
      {0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2}, {0x1.767dcf5534862p-1, 0x1.ce0a44eb17bccp-2}};
  const double A0 = 0x1.27616c9496e0bp-2, A1 = -0x1.71969a075c67ap-2, A2 = 0x1.ec70a6ca7baddp-2,
               A3 = -0x1.7154748bef6c8p-1, A4 = 0x1.71547652ab82bp0;
  const double SHIFT = 0x1.8p+52 / 32, C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3,
               C2 = 0x1.62e42ff0c52d6p-1;
  const u64 SIGN_BIAS = 1ull << (5 + 11);
  u64 sign_bias = 0;
  u32 ix = tm_f2u(x);
  const u32 iy = tm_f2u(y);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u || tm_zeroinfnanf(iy)) {
    if (tm_zeroinfnanf(iy)) {
      if (2u * iy == 0u) return tm_issnanf(ix) ? x + y : 1.0f;
      if (ix == 0x3f800000u) return tm_issnanf(iy) ? x + y : 1.0f;
      if (2u * ix > 2u * 0x7f800000u || 2u * iy > 2u * 0x7f800000u) return x + y;
      if (2u * ix == 2u * 0x3f800000u) return 1.0f;
      if ((2u * ix < 2u * 0x3f800000u) == !(iy & 0x80000000u)) return 0.0f;
      return y * y;
    }
    if (tm_zeroinfnanf(ix)) {
      float x2 = x * x;
      if ((ix & 0x80000000u) && tm_powf_checkint(iy) == 1) x2 = -x2;
      return (iy & 0x80000000u) ? 1.0f / x2 : x2;
    }
    if (ix & 0x80000000u) {                      // finite x < 0
      const int yint = tm_powf_checkint(iy);
      if (yint == 0) return __builtin_nanf("");
      if (yint == 1) sign_bias = SIGN_BIAS;
      ix &= 0x7fffffffu;
    }
    if (ix < 0x00800000u) {                      // subnormal x: normalise
      ix = tm_f2u(x * 0x1p23f);
      ix &= 0x7fffffffu;
      ix -= 23u << 23;
    }
  }
  // log2 x
  const u32 tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> 19) % 16u);
  const u32 top = tmp & 0xff800000u;
  const u32 iz = ix - top;
  const int k = (i32)top >> 23;
  const double z = (double)tm_u2f(iz);
  const double r = __builtin_fma(z, T[i][0], -1.0);
  const double y0 = T[i][1] + (double)k;
  const double r2 = r * r;
  double yy = __builtin_fma(A0, r, A1);
  const double p = __builtin_fma(A2, r, A3);
  const double r4 = r2 * r2;
  double q = __builtin_fma(A4, r, y0);
  q = __builtin_fma(p, r2, q);
  yy = __builtin_fma(yy, r4, q);
  const double ylogx = (double)y * yy;
  if (((tm_d2u(ylogx) >> 47) & 0xffffu) >= (tm_d2u(126.0) >> 47)) {
    if (ylogx > 0x1.fffffffd1d571p+6) return sign_bias ? -__builtin_inff() : __builtin_inff();
    if (ylogx <= -150.0) return sign_bias ? -0.0f : 0.0f;
  }
  // 2^ylogx
  double kd = ylogx + SHIFT;
  const u64 ki = tm_d2u(kd);
  kd -= SHIFT;
  const double rr = ylogx - kd;
  const u64 TT[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  u64 t = TT[ki % 32u];
  t += (ki + sign_bias) << 47;
  const double s = tm_u2d(t);
  const double zz = __builtin_fma(C0, rr, C1);
  const double rr2 = rr * rr;
  double w = __builtin_fma(C2, rr, 1.0);
  w = __builtin_fma(zz, rr2, w);
  w = w * s;
  return (float)w;
}

// lax.logistic of float64 as the reference's CPU target computes it (op_table.py:243-247): 1 / (1 + exp(-x)), with
// the device's exp (float64 takes the device math library).
#if defined(__HIP__) || defined(__HIPCC_RTC__)
TM_DFN double tm_logistic_d(double x) { return 1.0 / (1.0 + exp(-x)); }
#endif

