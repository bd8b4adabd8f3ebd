// tm_device.h -- the CDNA4 device runtime of generated tallymap kernels (gfx950, wave64).
//
// Every generated module is this header + tm_libm.h + the program's own code (backend/codegen.py, kernel.py).  The
// scalar helpers are TM_FN (host + device) so that the same definitions can be compiled for the host and checked
// there; the wave-level pieces (claims, atomics, LDS) are device-only.
//
// Semantics restated from the reference's device prelude (tallymap/backends/kernel/kernel.py:26-188) and its CPU
// target (host.py:43-171), written for AMD hardware:
//   - lax max/min: NaN-propagating, a signed-zero tie gives +0 / -0 (kernel.py:78-83);
//   - lax integer div/rem: x/0 = -1 (unsigned: all ones), INT_MIN/-1 = INT_MIN; x%0 = x, INT_MIN%-1 = 0
//     (kernel.py:95-103);
//   - shifts by >= the width give 0 (logical) or the sign fill (arithmetic) (kernel.py:104-109);
//   - float -> int toward zero, saturating, NaN -> 0 (host.py:133-146; v_cvt_i32_f32 behaves so natively);
//   - threefry2x32, 20 rounds (kernel.py:137-150; Salmon et al. 2011);
//   - the subnormal-safe f32 atomic add: |v| >= 2^-102 (or non-finite) takes the native atomic, a smaller
//     nonzero v a compare-and-swap loop of the IEEE add, +-0 is skipped (kernel.py:112-135);
//   - the exact f32 sum: a bin is 5 signed int64 words of weight 2^(63 j); an emit adds <= 2 pieces with int64
//     atomics and carries +-2 into the next word on overflow; the readout rounds once (kernel.py:870-941).
#pragma once

typedef signed char i8;
typedef unsigned char u8;
typedef short i16;
typedef unsigned short u16;
typedef int i32;
typedef unsigned int u32;
typedef long long i64;
typedef unsigned long long u64;
#if defined(__clang__)
typedef u32 tm_u32x4 __attribute__((ext_vector_type(4)));     // a 16-byte unit (one dwordx4 load / store)
typedef u32 tm_u32x2 __attribute__((ext_vector_type(2)));     // an 8-byte unit
#endif

#ifdef __HIPCC_RTC__
#define TM_DEVICE_ONLY 1
#endif
#if defined(__HIP__) || defined(__HIPCC_RTC__)
#define TM_FN __host__ __device__ __forceinline__
#define TM_DFN __device__ __forceinline__
#define TM_DNOINLINE __device__ __noinline__
#else
#define TM_FN static inline
#endif

template <class To, class From> TM_FN To tm_bitcast(From x) { return __builtin_bit_cast(To, x); }
TM_FN float tm_u2f(u32 u) { return __builtin_bit_cast(float, u); }
TM_FN u32 tm_f2u(float f) { return __builtin_bit_cast(u32, f); }
TM_FN double tm_u2d(u64 u) { return __builtin_bit_cast(double, u); }
TM_FN u64 tm_d2u(double d) { return __builtin_bit_cast(u64, d); }

// ------------------------------------------------------------------------- 64-bit shifts by a variable amount
// Built from 32-bit shifts of the two halves, s in [0, 63].  gfx950 returns wrong results from a 64-bit VALU
// shift (v_lshlrev_b64 / v_lshrrev_b64 / v_ashrrev_i64) whose shift-amount VGPR is the last register of an
// 8-register allocation block (v7, v15, ..., v39 in a 40-register kernel): measured on MI355X as corrupted exact
// sums, the register placement being the register allocator's choice.  Every 64-bit shift by a non-constant amount
// in device code goes through these, so that no such instruction is emitted; backend/compile.py rejects a code
// object that still contains one.
TM_FN u64 tm_shl64(u64 x, u32 s) {
  const u32 lo = (u32)x, hi = (u32)(x >> 32);
  const u32 rh = s >= 32u ? lo << (s - 32u) : (s ? (hi << s) | (lo >> (32u - s)) : hi);
  const u32 rl = s >= 32u ? 0u : lo << s;
  return ((u64)rh << 32) | (u64)rl;
}
TM_FN u64 tm_shr64(u64 x, u32 s) {
  const u32 lo = (u32)x, hi = (u32)(x >> 32);
  const u32 rl = s >= 32u ? hi >> (s - 32u) : (s ? (lo >> s) | (hi << (32u - s)) : lo);
  const u32 rh = s >= 32u ? 0u : hi >> s;
  return ((u64)rh << 32) | (u64)rl;
}
TM_FN i64 tm_sar64(i64 x, u32 s) {
  const u32 lo = (u32)(u64)x;
  const i32 hi = (i32)(u32)((u64)x >> 32);
  const u32 rl = s >= 32u ? (u32)(hi >> (s - 32u)) : (s ? (lo >> s) | ((u32)hi << (32u - s)) : lo);
  const u32 rh = (u32)(hi >> (s >= 32u ? 31u : s));
  return (i64)(((u64)rh << 32) | (u64)rl);
}
// u64 -> f32 rounded once, through an exact double (n < 2^53): the direct conversion lowers to a 64-bit shift
TM_FN float tm_u64_f32(u64 n) { return (float)(double)n; }
// u64 / i64 -> f32 for every value, rounded once (to nearest even) from 32-bit halves: the 32 leading significant
// bits with a sticky bit for the bits below them (so the one rounding of the u32 -> f32 conversion is the rounding
// of the whole value), then an exact scaling by a power of two.  The compiler's own expansion normalises the
// operand with a 64-bit shift by its leading-zero count, a variable 64-bit shift (see tm_shl64).
TM_FN float tm_u64f(u64 u) {
  const u32 hi = (u32)(u >> 32), lo = (u32)u;
  if (hi == 0u) return (float)lo;
  const u32 n = (u32)__builtin_clz(hi);
  const u32 m = n ? (hi << n) | (lo >> (32u - n)) : hi;
  const u32 rest = n ? lo << n : lo;
  return __builtin_ldexpf((float)(m | (rest != 0u ? 1u : 0u)), (int)(32u - n));
}
TM_FN float tm_i64f(i64 x) {
  const float f = tm_u64f(x < 0 ? 0ull - (u64)x : (u64)x);
  return x < 0 ? -f : f;
}

// ------------------------------------------------------------------------------------------- lax helpers
template <class T> TM_FN T tm_fmax(T a, T b) {
  return (a > b || a != a) ? a : ((b > a || b != b) ? b : (a == (T)0 ? a + b : a));
}
template <class T> TM_FN T tm_fmin(T a, T b) {
  return (a < b || a != a) ? a : ((b < a || b != b) ? b : (a == (T)0 ? -(-a - b) : a));
}
template <class T> TM_FN T tm_imax(T a, T b) { return a > b ? a : b; }
template <class T> TM_FN T tm_imin(T a, T b) { return a < b ? a : b; }
template <class T> TM_FN T tm_fsign(T a) { return a > (T)0 ? (T)1 : (a < (T)0 ? (T)-1 : a); }

TM_FN i32 tm_idiv(i32 a, i32 b) { return b == 0 ? -1 : ((b == -1 && a == (i32)0x80000000u) ? a : a / b); }
TM_FN i32 tm_irem(i32 a, i32 b) { return b == 0 ? a : ((b == -1 && a == (i32)0x80000000u) ? 0 : a % b); }
TM_FN u32 tm_idiv(u32 a, u32 b) { return b == 0u ? 0xffffffffu : a / b; }
TM_FN u32 tm_irem(u32 a, u32 b) { return b == 0u ? a : a % b; }
TM_FN i64 tm_idiv(i64 a, i64 b) {
  return b == 0 ? -1 : ((b == -1 && a == (i64)0x8000000000000000ull) ? a : a / b);
}
TM_FN i64 tm_irem(i64 a, i64 b) {
  return b == 0 ? a : ((b == -1 && a == (i64)0x8000000000000000ull) ? 0 : a % b);
}

template <class T, class U> TM_FN T tm_shl(T a, T b) {
  if ((U)b >= (U)(sizeof(T) * 8)) return (T)0;
  if constexpr (sizeof(T) == 8) return (T)tm_shl64((u64)a, (u32)b);
  else return (T)((U)a << (U)b);
}
template <class T, class U> TM_FN T tm_shrl(T a, T b) {
  if ((U)b >= (U)(sizeof(T) * 8)) return (T)0;
  if constexpr (sizeof(T) == 8) return (T)tm_shr64((u64)a, (u32)b);
  else return (T)((U)a >> (U)b);
}
template <class T, class U> TM_FN T tm_shra(T a, T b) {
  if ((U)b >= (U)(sizeof(T) * 8)) return (T)(a < (T)0 ? (T)-1 : (T)0);
  if constexpr (sizeof(T) == 8) return (T)tm_sar64((i64)a, (u32)b);
  else return (T)(a >> (U)b);
}

// lax.rem of floats: the exact remainder x - trunc(x / y) y with x's sign (C fmod; the reference's CPU target calls
// glibc's fmodf / fmod, which are exact).  NaN for a NaN operand, an infinite x or a zero y; x itself when |x| < |y|
// (an infinite y included); +-0 when |x| == |y|.  Otherwise |x| = mx 2^ex', |y| = my 2^ey' with integer
// significands, and the remainder is (mx 2^(ex' - ey') mod my) 2^ey': the reduction runs on the significands in
// integer arithmetic (8 bits per step for f32: r < my < 2^24 keeps r << 8 within 32 bits; one bit per step for
// f64, with no variable 64-bit shift), and scaling r (< my, so exact in the format) by 2^ey' rounds nothing.
TM_FN float tm_fmodf(float x, float y) {
  const u32 ux = tm_f2u(x), ax = ux & 0x7fffffffu, ay = tm_f2u(y) & 0x7fffffffu;
  if (ax >= 0x7f800000u || ay > 0x7f800000u || ay == 0u) return __builtin_nanf("");
  if (ax <= ay) return ax == ay ? tm_u2f(ux & 0x80000000u) : x;
  int ex = (int)(ax >> 23), ey = (int)(ay >> 23);
  u32 mx = ax & 0x7fffffu, my = ay & 0x7fffffu;
  if (ex) mx |= 0x800000u; else ex = 1;        // (a subnormal: exponent field 1, no hidden bit)
  if (ey) my |= 0x800000u; else ey = 1;
  u32 r = mx % my;
  for (int d = ex - ey; d > 0;) {
    const int sh = d < 8 ? d : 8;
    r = (r << sh) % my;
    d -= sh;
  }
  if (r == 0u) return tm_u2f(ux & 0x80000000u);
  const float v = __builtin_ldexpf((float)r, ey - 150);
  return (ux >> 31) ? -v : v;
}
TM_FN double tm_fmod(double x, double y) {
  const u64 ux = tm_d2u(x), ax = ux & 0x7fffffffffffffffull, ay = tm_d2u(y) & 0x7fffffffffffffffull;
  if (ax >= 0x7ff0000000000000ull || ay > 0x7ff0000000000000ull || ay == 0ull) return __builtin_nan("");
  if (ax <= ay) return ax == ay ? tm_u2d(ux & 0x8000000000000000ull) : x;
  int ex = (int)(ax >> 52), ey = (int)(ay >> 52);
  u64 mx = ax & 0xfffffffffffffull, my = ay & 0xfffffffffffffull;
  if (ex) mx |= 1ull << 52; else ex = 1;
  if (ey) my |= 1ull << 52; else ey = 1;
  while (!(mx >> 52)) { mx <<= 1; --ex; }     // normalise: both significands in [2^52, 2^53), so ex >= ey
  while (!(my >> 52)) { my <<= 1; --ey; }
  u64 r = mx >= my ? mx - my : mx;
  for (int d = ex - ey; d > 0; --d) {
    r <<= 1;
    if (r >= my) r -= my;
  }
  if (r == 0ull) return tm_u2d(ux & 0x8000000000000000ull);
  const double v = __builtin_ldexp((double)r, ey - 1075);
  return (ux >> 63) ? -v : v;
}

// float -> integer toward zero, saturating, NaN -> 0
TM_FN i32 tm_f2i32(float x) {
  return x != x ? 0 : (x <= -2147483648.0f ? (i32)0x80000000u : (x >= 2147483648.0f ? 0x7fffffff : (i32)x));
}
TM_FN u32 tm_f2u32(float x) {
  return x != x ? 0u : (x <= 0.0f ? 0u : (x >= 4294967296.0f ? 0xffffffffu : (u32)x));
}
TM_FN i32 tm_d2i32(double x) {
  return x != x ? 0 : (x <= -2147483648.0 ? (i32)0x80000000u : (x >= 2147483647.0 ? 0x7fffffff : (i32)x));
}
TM_FN u32 tm_d2u32(double x) {
  return x != x ? 0u : (x <= 0.0 ? 0u : (x >= 4294967295.0 ? 0xffffffffu : (u32)x));
}
TM_FN i64 tm_f2i64(float x) {
  return x != x ? 0 : (x <= -9223372036854775808.0f ? (i64)0x8000000000000000ull
                                                     : (x >= 9223372036854775808.0f ? 0x7fffffffffffffffll : (i64)x));
}
TM_FN i64 tm_d2i64(double x) {
  return x != x ? 0 : (x <= -9223372036854775808.0 ? (i64)0x8000000000000000ull
                                                    : (x >= 9223372036854775808.0 ? 0x7fffffffffffffffll : (i64)x));
}

// ----------------------------------------------------------------------------------------- threefry2x32
TM_FN u32 tm_rotl(u32 x, int d) { return (x << d) | (x >> (32 - d)); }

TM_FN void tm_threefry(u32 k0, u32 k1, u32 c0, u32 c1, u32& o0, u32& o1) {
  const u32 k2 = k0 ^ k1 ^ 0x1BD11BDAu;
  u32 x0 = c0 + k0, x1 = c1 + k1;
#define TM_TFR(r) x0 += x1; x1 = tm_rotl(x1, r); x1 ^= x0;
  TM_TFR(13) TM_TFR(15) TM_TFR(26) TM_TFR(6)  x0 += k1; x1 += k2 + 1u;
  TM_TFR(17) TM_TFR(29) TM_TFR(16) TM_TFR(24) x0 += k2; x1 += k0 + 2u;
  TM_TFR(13) TM_TFR(15) TM_TFR(26) TM_TFR(6)  x0 += k0; x1 += k1 + 3u;
  TM_TFR(17) TM_TFR(29) TM_TFR(16) TM_TFR(24) x0 += k1; x1 += k2 + 4u;
  TM_TFR(13) TM_TFR(15) TM_TFR(26) TM_TFR(6)  x0 += k2; x1 += k0 + 5u;
#undef TM_TFR
  o0 = x0;
  o1 = x1;
}

#if defined(__HIP__) || defined(__HIPCC_RTC__)
// ============================================================================================ device only
// lane and wave helpers (wave64)
TM_DFN int tm_lane() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }
TM_DFN u64 tm_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
TM_DFN u32 tm_rank(u64 mask) {     // set bits of mask below this lane
  return __builtin_amdgcn_mbcnt_hi((u32)(mask >> 32), __builtin_amdgcn_mbcnt_lo((u32)mask, 0u));
}
TM_DFN u32 tm_bcast_first(u32 v) { return __builtin_amdgcn_readfirstlane(v); }

// one claim of `n` consecutive items by the first active lane -> the base, broadcast to the wave
TM_DFN u64 tm_claim(u64* ctr, u32 n) {
  u64 base = 0;
  if (tm_lane() == (int)__builtin_ctzll(tm_ballot(true))) base = atomicAdd((unsigned long long*)ctr, (u64)n);
  const u32 lo = tm_bcast_first((u32)base);
  const u32 hi = tm_bcast_first((u32)(base >> 32));
  return ((u64)hi << 32) | lo;
}

// A spawned child's row in the next generation's buffer (reference _tally.py:284-300): the lanes that spawn at this
// point take consecutive tickets with one counter atomic per wave -> the lane's ticket, or -1 (it does not spawn).
TM_DFN i64 tm_qclaim(u64* ctr, bool when) {
  const u64 m = tm_ballot(when);
  if (m == 0ull) return -1;
  const u64 b = tm_claim(ctr, (u32)__builtin_popcountll(m));
  return when ? (i64)(b + tm_rank(m)) : -1;
}

// A Records output's slot claim (reference _tally.py:141-160): a wave takes raw slots from a private batch of TM_RB
// consecutive slots, refilled from the output's slot counter with one atomic per TM_RB slots (one counter hit by
// every wave of the chip serialises at its L2 channel; per-record or per-append atomics there cost ~30x the item
// loop).  The batch state (base, slots left, records appended) lives in the wave's LDS words, read by every active
// lane and written by the first, so lanes that diverged keep one view of it.  The lanes that append take the
// batch's remaining slots in rank order, then a new batch's: only the last batch of each wave has unused slots.
// -> the lane's raw slot, or -1 (it does not append, or the slot is past rawcap).
#define TM_RB 256u
TM_DFN i64 tm_rclaim(u64* ctr, volatile u64* base_s, volatile u32* left_s, volatile u64* cnt_s, bool when,
                     u64 rawcap) {
  const u64 m = tm_ballot(when);
  if (m == 0ull) return -1;
  const u32 n = (u32)__builtin_popcountll(m), r = tm_rank(m);
  const u32 left = *left_s;
  const u64 base = *base_s;
  const u64 nb = n > left ? tm_claim(ctr, TM_RB) : 0ull;
  const u64 s = r < left ? base + (TM_RB - left) + r : nb + (r - left);
  if (tm_lane() == (int)__builtin_ctzll(tm_ballot(true))) {
    if (n > left) {
      *base_s = nb;
      *left_s = TM_RB - (n - left);
    } else {
      *left_s = left - n;
    }
    *cnt_s = *cnt_s + n;
  }
  return (when && s < rawcap) ? (i64)s : -1;
}

// A Records append inside a branch of a divergent if / else: the lanes that append take consecutive raw slots with
// one counter atomic per wave at this point; the wave's record count grows by an LDS atomic of its first lane.
// tm_rclaim's batch passes its state from one append to the next through plain LDS loads and first-lane stores,
// which is sound only where all the wave's lanes run the same code: lanes of one wave in two branches run one
// branch after the other, and the compiler, which reasons per lane (where the branches never meet), may merge the
// branches' identical trailing stores into one store after both, so the second branch would read the state from
// before the first.  An atomic add is unaffected (merged, it still adds each branch's count).
TM_DFN i64 tm_rclaim_direct(u64* ctr, u64* cnt_s, bool when, u64 rawcap) {
  const u64 m = tm_ballot(when);
  if (m == 0ull) return -1;
  const u32 n = (u32)__builtin_popcountll(m);
  const u64 b = tm_claim(ctr, n);
  if (tm_lane() == (int)__builtin_ctzll(tm_ballot(true)))
    __hip_atomic_fetch_add(cnt_s, (u64)n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const u64 s = b + tm_rank(m);
  return (when && s < rawcap) ? (i64)s : -1;
}

// f32 atomic adds that keep subnormals (2^-102 = 0x0c800000)
TM_DFN void tm_cas_addf(float* a, float v) {
  u32* const u = (u32*)a;
  u32 o = __hip_atomic_load(u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), w;
  do {
    w = o;
    const float n = tm_u2f(w) + v;
    o = atomicCAS(u, w, tm_f2u(n));
  } while (o != w);
}
TM_DFN void tm_gadd_f32(float* a, float v) {
  if (v == 0.0f) return;
  if (!(__builtin_fabsf(v) < tm_u2f(0x0c800000u))) { unsafeAtomicAdd(a, v); return; }
  tm_cas_addf(a, v);
}
TM_DFN void tm_lds_cas_addf(float* a, float v) {
  u32* const u = (u32*)a;
  u32 o = *(volatile u32*)u, w;
  do {
    w = o;
    o = atomicCAS(u, w, tm_f2u(tm_u2f(w) + v));
  } while (o != w);
}
TM_DFN void tm_ladd_f32(float* a, float v) {       // a: LDS
  if (v == 0.0f) return;
  if (!(__builtin_fabsf(v) < tm_u2f(0x0c800000u))) { atomicAdd(a, v); return; }
  tm_lds_cas_addf(a, v);
}
TM_DFN void tm_gadd_i32(i32* a, i32 v) { atomicAdd(a, v); }
// f64 atomic adds that keep subnormals: a CAS loop of the IEEE add below 2^-970 (where a sum of two addends can
// be subnormal), the native add above
TM_DFN void tm_cas_addd(double* a, double v) {
  u64* const u = (u64*)a;
  u64 o = __hip_atomic_load(u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), w;
  do {
    w = o;
    o = atomicCAS((unsigned long long*)u, (unsigned long long)w, (unsigned long long)tm_d2u(tm_u2d(w) + v));
  } while (o != w);
}
TM_DFN void tm_gadd_f64(double* a, double v) {
  if (v == 0.0) return;
  if (!(__builtin_fabs(v) < 0x1p-970)) { unsafeAtomicAdd(a, v); return; }
  tm_cas_addd(a, v);
}
TM_DFN void tm_ladd_f64(double* a, double v) {     // a: LDS
  if (v == 0.0) return;
  if (!(__builtin_fabs(v) < 0x1p-970)) { atomicAdd(a, v); return; }
  u64* const u = (u64*)a;
  u64 o = *(volatile u64*)u, w;
  do {
    w = o;
    o = atomicCAS((unsigned long long*)u, (unsigned long long)w, (unsigned long long)tm_d2u(tm_u2d(w) + v));
  } while (o != w);
}
TM_DFN void tm_gadd_u64(u64* a, u64 v) { atomicAdd((unsigned long long*)a, (unsigned long long)v); }

#endif  // device only

// -------------------------------------------------------------------------- the exact f32 sum (5 words)
// A finite f32 v = m * 2^(p - 149), m < 2^24, p = max(biased exponent - 1, 0): an integer below 2^277 in units of
// 2^-149, kept as 5 signed int64 words of weight 2^(63 j).  An emit adds the signed pieces of m << (p % 63) into
// words p/63 and p/63 + 1; an add that overflows int64 (seen in the old value the add returns) carries +-2 into the
// next word (2^64 = 2 * 2^63); a carry out of word 4 is lost and flags the bin.  Integer adds commute: the total is
// bitwise independent of the order of the emits.  `add(a, j, q)` adds q to word j and returns the word's old value
// (the device passes an int64 atomic; the host checks pass a plain add).
template <class Add> TM_FN bool tm_xcarry(u64* a, int j, i64 c, Add add) {
  for (; j < 5; ++j) {
    const i64 o = add(a, j, c);
    const i64 r = (i64)((u64)o + (u64)c);
    if (!((c > 0 && r < o) || (c < 0 && r > o))) return false;
  }
  return true;
}
template <class Add> TM_FN bool tm_xadd_with(u64* a, int j, i64 q, Add add) {
  const i64 o = add(a, j, q);
  const i64 r = (i64)((u64)o + (u64)q);
  if (q > 0 && r < o) return tm_xcarry(a, j + 1, 2, add);
  if (q < 0 && r > o) return tm_xcarry(a, j + 1, -2, add);
  return false;
}
// true: flag the bin (a non-finite emit or a lost carry)
template <class Add> TM_FN bool tm_xemit_with(u64* a, float v, Add add) {
  const u32 b = tm_f2u(v), e = (b >> 23) & 255u;
  if (e == 255u) return true;
  const u64 m = (u64)(b & 0x7fffffu) | (e ? 0x800000ull : 0ull);
  if (m == 0ull) return false;
  const u32 p = e ? e - 1u : 0u, j = p / 63u, s = p - 63u * j;
  const i64 lo = (i64)(tm_shl64(m, s) & 0x7fffffffffffffffull), hi = s >= 40u ? (i64)tm_shr64(m, 63u - s) : 0ll;
  const bool neg = (b >> 31) != 0u;
  bool lost = false;
  if (lo) lost = tm_xadd_with(a, (int)j, neg ? -lo : lo, add);
  if (hi) lost = tm_xadd_with(a, (int)j + 1, neg ? -hi : hi, add) || lost;
  return lost;
}

#if defined(__HIP__) || defined(__HIPCC_RTC__)
struct TmAtomicAdd64 {
  __device__ i64 operator()(u64* a, int j, i64 q) const {
    return (i64)atomicAdd((unsigned long long*)&a[j], (unsigned long long)q);
  }
};
TM_DFN bool tm_xadd(u64* a, int j, i64 q) { return tm_xadd_with(a, j, q, TmAtomicAdd64()); }
TM_DFN bool tm_xemit(u64* a, float v) { return tm_xemit_with(a, v, TmAtomicAdd64()); }
// a lane's own exact accumulator (the words in registers: a tally of one bin privatised per lane)
struct TmLaneAdd64 {
  __device__ i64 operator()(u64* a, int j, i64 q) const {
    const i64 o = (i64)a[j];
    a[j] = (u64)(o + q);
    return o;
  }
};
TM_DFN bool tm_xemit_lane(u64* a, float v) { return tm_xemit_with(a, v, TmLaneAdd64()); }
#endif  // device only

// the readout: sum_j word_j 2^(63 j) as a 384-bit two's-complement integer, its magnitude rounded once to f32
// (nearest, ties to even); *bad when beyond f32 (host + device: the host build checks it against Python integers)
TM_FN float tm_xread(const u64* a, bool* bad) {
  u64 d[6] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
  for (int j = 0; j < 5; ++j) {
    const i64 w = (i64)a[j];
    const int sh = 63 * j, l = sh >> 6, b = sh & 63;
    const u64 ext = w < 0 ? ~0ull : 0ull;
    const u64 x0 = tm_shl64((u64)w, (u32)b), x1 = b ? (u64)tm_sar64(w, (u32)(64 - b)) : ext;
    u64 c = 0ull;
    for (int k = l; k < 6; ++k) {
      const u64 y = k == l ? x0 : (k == l + 1 ? x1 : ext);
      const u64 t = d[k] + y, u = t + c;
      c = (t < y ? 1ull : 0ull) + (u < t ? 1ull : 0ull);
      d[k] = u;
    }
  }
  const bool neg = (i64)d[5] < 0;
  if (neg) {
    u64 k = 1ull;
    for (int j = 0; j < 6; ++j) {
      d[j] = ~d[j] + k;
      k = (k && d[j] == 0ull) ? 1ull : 0ull;
    }
  }
  int t = 5;
  while (t >= 0 && d[t] == 0ull) --t;
  if (t < 0) return 0.0f;
  const int s = __builtin_clzll(d[t]);
  const u64 d1 = t >= 1 ? d[t - 1] : 0ull;
  const u64 top = s ? tm_shl64(d[t], (u32)s) | tm_shr64(d1, (u32)(64 - s)) : d[t];
  bool st = s ? tm_shl64(d1, (u32)s) != 0ull : d1 != 0ull;
  for (int j = 0; j < t - 1; ++j) st = st || d[j] != 0ull;
  u64 q = top >> 40;
  const u64 r = top & 0xffffffffffull, half = 0x8000000000ull;
  if (r > half || (r == half && (st || (q & 1ull)))) ++q;
  // q * 2^(64 t + 40 - s - 149): exact in double (q <= 2^24), then to f32 exactly unless out of range
  const int ex = 64 * t + 40 - s - 149;
  double o = (double)q;
  // scale by 2^ex in two exact steps (ex can reach ~250 or fall to ~-149)
  const int e1 = ex / 2, e2 = ex - e1;
  o = o * tm_u2d((u64)(1023 + e1) << 52) * tm_u2d((u64)(1023 + e2) << 52);
  if (!(o <= 3.4028234663852886e38)) *bad = true;
  const float f = (float)o;
  return neg ? -f : f;
}

// --------------------------------------------------------------------- the scaled fixed-point sum (WIDE)
// A bin is an int64 low word (two's complement, wrapping) and an i32 carry word, the net signed carry out of the
// low word: an add of q whose old value o wraps (q > 0 and o + q < o: +1; q < 0 and o + q > o: -1) adds its carry,
// so the exact total low + carry * 2^64 does not depend on the order of the adds.  An emit adds round(v * scale)
// (nearest, ties to even); |v * scale| >= 9.2e18 is not representable: the emit is dropped and flags its bin
// (reference kernel.py:844-869, _api.py:55-84).  `add(lo, q)` adds q and returns the old value.
template <class Add> TM_FN int tm_wadd_with(u64* lo, i64 q, Add add) {      // -> the carry: -1, 0 or +1
  const i64 o = add(lo, q);
  const i64 r = (i64)((u64)o + (u64)q);
  return (q > 0 && r < o) ? 1 : ((q < 0 && r > o) ? -1 : 0);
}
// round(v * scale) -> *q; false when not representable
TM_FN bool tm_wvalue(double v, double scale, i64* q) {
  const double x = v * scale;
  if (!(__builtin_fabs(x) < 9.2e18)) return false;
  *q = (i64)__builtin_rint(x);
  return true;
}
// low + carry * 2^64 rounded once to double (nearest, ties to even)
TM_FN double tm_wide_f64(u64 lo, i32 c) {
  if (c == 0) return (double)(i64)lo;
  u64 h = (u64)((i64)c - (i64)(lo >> 63)), l = lo;       // the 128-bit two's complement h:l
  const bool neg = (i64)h < 0;
  if (neg) {
    l = ~l + 1ull;
    h = ~h + (l == 0ull ? 1ull : 0ull);
  }
  if (h == 0ull) {
    const double m = (double)l;
    return neg ? -m : m;
  }
  const int e = 64 - __builtin_clzll(h);                   // the magnitude has 64 + e bits
  const u64 t = e == 64 ? h : (tm_shl64(h, (u32)(64 - e)) | tm_shr64(l, (u32)e));   // its top 64 bits
  const u64 sticky = e == 64 ? l : tm_shl64(l, (u32)(64 - e));                      // the bits below them
  const double m = (double)(t | (sticky != 0ull ? 1ull : 0ull)) * tm_u2d((u64)(1023 + e) << 52);
  return neg ? -m : m;
}
TM_FN u64 tm_d2u64(double x) {
  return x != x ? 0ull : (x <= 0.0 ? 0ull : (x >= 18446744073709551616.0 ? ~0ull : (u64)x));
}

#if defined(__HIP__) || defined(__HIPCC_RTC__)
struct TmAtomicAddW {
  __device__ i64 operator()(u64* a, i64 q) const {
    return (i64)atomicAdd((unsigned long long*)a, (unsigned long long)q);
  }
};
TM_DFN void tm_wadd(u64* lo, i32* c, i64 q) {
  const int k = tm_wadd_with(lo, q, TmAtomicAddW());
  if (k) atomicAdd(c, k);
}
// one emit of v: false when v * scale is not representable (the caller counts it and flags the bin)
TM_DFN bool tm_wemit(u64* lo, i32* c, double v, double scale) {
  i64 q = 0;
  if (!tm_wvalue(v, scale, &q)) return false;
  if (q != 0) tm_wadd(lo, c, q);
  return true;
}
#endif  // device only
