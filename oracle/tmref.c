/* tmref -- the parity ORACLE and the CPU baseline.  TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only as the checker.  The product path (tallymap_amd) never
 * links, loads or calls anything here.
 *
 * A plain-C restatement of what the reference's CPU kernel backend computes for the benchmark item programs:
 *   - an OpenMP team, each thread claiming ONE item at a time from a shared counter
 *     (reference tallymap/backends/kernel/host_shim.cc:83-138, kernel.py:727-760);
 *   - per-thread privatised f32 tallies when a program's tallies fit 4096 bytes, flushed with an IEEE
 *     compare-and-swap add; larger tallies take the CAS add directly (kernel.py:300, 313-324, 681-688;
 *     host.py:57, 158-161);
 *   - the IEEE environment per thread (host_shim.cc:116-121), no FMA contraction (host.py:35: -ffp-contract=off);
 *   - glibc libm for transcendentals and, for f32 erf_inv, Giles' polynomial evaluated in double with libm log and
 *     sqrt, rounded once to f32 (host.py:102-132);
 *   - float->int conversion toward zero, saturating, NaN -> 0 (host.py:133-146);
 *   - lax.max: NaN-propagating, a signed-zero tie gives +0 (kernel.py:78-83);
 *   - out-of-range emits dropped and counted in stats[4] (kernel.py:987-988, _tally.py:32-38);
 *   - the max_steps cap: the loop runs while k < M && cond, truncated = k >= M && cond(final)
 *     (_rewrite.py:517-527);
 *   - jax.random's threefry2x32 and its partitionable layering (fold_in, split, random_bits, uniform, normal):
 *     kernel.py:137-150 for the core, jax's PRNGImpl via _compat.py:119-154 for the layering.
 * Gradients are computed here in FORWARD mode (dual numbers carried through the same item), so the oracle is
 * independent of the product's reverse-mode replay; per-item cotangent contributions are summed EXACTLY (an integer
 * in units of 2^-149, rounded once: the reference's exact broadcast cotangents, _reverse.py:1172-1177,
 * kernel.py:870-941) by a multi-limb magnitude accumulator that shares no code or format with the product's.
 * Every float tally also gets a float64 shadow sum of the same emits: the re-summation the tolerances are
 * measured against.
 */
#include <fenv.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint32_t u32;
typedef uint64_t u64;
typedef int32_t i32;
typedef int64_t i64;

/* ------------------------------------------------------------------------------------------ bit helpers */
static inline float asf(u32 u) { float f; memcpy(&f, &u, 4); return f; }
static inline u32 asu(float f) { u32 u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------- threefry2x32 (Salmon et al. 2011) */
/* 20 rounds, rotation constants R_{2x32} = 13 15 26 6 17 29 16 24, key schedule every 4 rounds with the parity
 * constant 0x1BD11BDA (Random123 threefry.h); reference kernel.py:137-150. */
static inline u32 rotl32(u32 x, int d) { return (x << d) | (x >> (32 - d)); }

void tmref_threefry(u32 k0, u32 k1, u32 c0, u32 c1, u32* out) {
  static const int R[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  const u32 ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  u32 x0 = c0 + ks[0], x1 = c1 + ks[1];
  for (int blk = 0; blk < 5; ++blk) {
    for (int r = 0; r < 4; ++r) {
      x0 += x1;
      x1 = rotl32(x1, R[(blk & 1) * 4 + r]);
      x1 ^= x0;
    }
    x0 += ks[(blk + 1) % 3];
    x1 += ks[(blk + 2) % 3] + (u32)(blk + 1);
  }
  out[0] = x0;
  out[1] = x1;
}

/* ------------------------------------------------------------ jax.random layering (threefry, partitionable) */
/* fold_in(key, d) = threefry(key; (0, u32(d))): _threefry_fold_in = threefry_2x32(key, threefry_seed(d)), and the
 * seed of a 32-bit integer is (d >> 32 = 0, d). */
static inline void fold_in(const u32* k, u32 d, u32* o) { tmref_threefry(k[0], k[1], 0u, d, o); }
/* split(key, n)[i] = threefry(key; (hi(i), lo(i))) (iota_2x32_shape) */
static inline void split_i(const u32* k, u64 i, u32* o) { tmref_threefry(k[0], k[1], (u32)(i >> 32), (u32)i, o); }
/* random_bits(key, 32, ()) = o0 ^ o1 of threefry(key; (0, 0)) */
static inline u32 bits32(const u32* k) { u32 o[2]; tmref_threefry(k[0], k[1], 0u, 0u, o); return o[0] ^ o[1]; }

/* lax.max of f32: NaN-propagating, +0 on a signed-zero tie (kernel.py:78-80) */
static inline float lax_fmax(float a, float b) {
  return (a > b || a != a) ? a : ((b > a || b != b) ? b : (a == 0.0f ? a + b : a));
}

/* jax.random.uniform(key, (), f32, lo, hi): ((bits >> 9) | 1.0f bits) as float - 1, times (hi - lo), plus lo,
 * then lax.max(lo, .) -- every operation in f32, separately rounded */
static inline float uniform_f32(const u32* k, float lo, float hi) {
  const float f = asf((bits32(k) >> 9) | 0x3f800000u) - 1.0f;
  const float span = hi - lo;
  const float r = f * span;
  return lax_fmax(lo, r + lo);
}

/* f32 erf_inv of the reference CPU target: Giles (2010) single-precision polynomial evaluated in double, libm
 * log / sqrt, rounded once to f32 (host.py:102-132). */
static double giles(double y) {
  const double a = fabs(y);
  double w = -log((1.0 - a) * (1.0 + a)), p;
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
    w = sqrt(w) - 3.0;
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

float tmref_erfinvf(float y) {
  if (!(y > -1.0f && y < 1.0f)) return y == 1.0f ? INFINITY : (y == -1.0f ? -INFINITY : NAN);
  return y == 0.0f ? y : (float)copysign(giles((double)y), (double)y);
}

/* jax.random.normal(key, (), f32): sqrt(2) (as f32) * erf_inv(uniform(key, nextafter(-1, 0), 1)) (_normal_real) */
static inline float normal_f32(const u32* k) {
  const float lo = asf(0xbf7fffffu);             /* nextafter(-1.0f, 0.0f) = -(1 - 2^-24) */
  const float u = uniform_f32(k, lo, 1.0f);
  return asf(0x3fb504f3u) * tmref_erfinvf(u);    /* float32(sqrt(2)) */
}

/* f32 -> int32 toward zero, saturating, NaN -> 0 (host.py:133-146) */
static inline i32 f2i(float x) {
  if (x != x) return 0;
  if (x <= -2147483648.0f) return INT32_MIN;
  if (x >= 2147483648.0f) return INT32_MAX;
  return (i32)x;
}

/* exported scalar helpers (golden tests pin them) */
void tmref_fold_in(const u32* k, u32 d, u32* o) { fold_in(k, d, o); }
void tmref_split(const u32* k, u64 n, u32* out) { for (u64 i = 0; i < n; ++i) split_i(k, i, out + 2 * i); }
float tmref_uniform(const u32* k, float lo, float hi) { return uniform_f32(k, lo, hi); }
float tmref_normal(const u32* k) { return normal_f32(k); }
u32 tmref_bits32(const u32* k) { return bits32(k); }

/* -------------------------------------------------------------------------------- exact f32 summation */
/* A finite f32 is m * 2^(p - 149) with m < 2^24, p = max(biased exponent - 1, 0): an integer below 2^277 in units of
 * 2^-149.  Positive and negative parts are kept as separate 384-bit magnitudes (6 x 64-bit limbs: room for 2^107
 * emits of the largest f32), and the result is |pos - neg| rounded once to f32, nearest, ties to even -- the meaning
 * of the reference's exact accumulator (kernel.py:870-941), in an unrelated representation. */
#define XL 6
typedef struct { u64 p[XL], n[XL]; int bad; } exsum;

static void ex_addmag(u64* a, u64 m, unsigned s) {
  unsigned l = s >> 6, b = s & 63u;
  u64 lo = m << b, hi = b ? (m >> (64 - b)) : 0;
  u64 c = 0;
  for (unsigned j = l; j < XL; ++j) {
    u64 add = (j == l) ? lo : (j == l + 1 ? hi : 0);
    u64 t = a[j] + add;
    u64 c1 = t < add;
    u64 u = t + c;
    u64 c2 = u < t;
    a[j] = u;
    c = c1 + c2;
    if (!c && j > l) break;
  }
}

static inline void ex_add(exsum* e, float v) {
  const u32 b = asu(v), ex = (b >> 23) & 255u;
  if (ex == 255u) { e->bad = 1; return; }
  const u64 m = (u64)(b & 0x7fffffu) | (ex ? 0x800000ull : 0ull);
  if (!m) return;
  const unsigned p = ex ? ex - 1u : 0u;
  ex_addmag((b >> 31) ? e->n : e->p, m, p);
}

static void ex_merge(exsum* dst, const exsum* src) {
  for (unsigned j = 0; j < XL; ++j) {
    /* add limb by limb through the same magnitude adder (64 bits at a time) */
    if (src->p[j]) ex_addmag(dst->p, src->p[j], 64u * j);
    if (src->n[j]) ex_addmag(dst->n, src->n[j], 64u * j);
  }
  dst->bad |= src->bad;
}

static float ex_read(const exsum* e, int* bad) {
  if (e->bad) { *bad = 1; return NAN; }
  u64 d[XL];
  int neg = 0;
  int cmp = 0;
  for (int j = XL - 1; j >= 0 && !cmp; --j) cmp = (e->p[j] > e->n[j]) - (e->p[j] < e->n[j]);
  const u64* A = e->p; const u64* B = e->n;
  if (cmp < 0) { neg = 1; A = e->n; B = e->p; }
  u64 br = 0;
  for (int j = 0; j < XL; ++j) {
    u64 t = A[j] - B[j];
    u64 b1 = A[j] < B[j];
    u64 u = t - br;
    u64 b2 = t < br;
    d[j] = u;
    br = b1 + b2;
  }
  int t = XL - 1;
  while (t >= 0 && d[t] == 0) --t;
  if (t < 0) return 0.0f;
  const int top = 64 * t + 63 - __builtin_clzll(d[t]);   /* index of the leading bit */
  if (top < 24) {                                           /* exact: an f32 subnormal or small normal in units */
    float r = (float)ldexp((double)d[0], -149);
    return neg ? -r : r;
  }
  /* q = bits [top-23, top], r = the rest */
  const int lsb = top - 23;
  u64 q = 0;
  for (int i = 0; i < 24; ++i) {
    const int bit = lsb + i;
    q |= ((d[bit >> 6] >> (bit & 63)) & 1ull) << i;
  }
  const int hb = lsb - 1;
  const int half = (d[hb >> 6] >> (hb & 63)) & 1ull;
  int sticky = 0;
  for (int bit = 0; bit < hb && !sticky; ++bit) sticky = (d[bit >> 6] >> (bit & 63)) & 1ull;
  if (half && (sticky || (q & 1ull))) ++q;
  const double r = ldexp((double)q, lsb - 149);
  if (!(r <= 3.4028234663852886e38)) { *bad = 1; return NAN; }
  return neg ? -(float)r : (float)r;
}

/* exact sum of n f32 values (the golden tests pin it against Python integers) */
float tmref_exact_sum(const float* v, i64 n, int* bad) {
  exsum e;
  memset(&e, 0, sizeof(e));
  *bad = 0;
  for (i64 i = 0; i < n; ++i) ex_add(&e, v[i]);
  return ex_read(&e, bad);
}

/* ----------------------------------------------------------------------------------------- the runner */
/* stats slots (reference _api.py:194-195): spawned, children_dropped, children_truncated, fixed_point_overflow,
 * dropped_emits */
enum { ST_DROPPED = 4 };
#define PRIV_BYTES 4096

typedef struct {
  int nt;                 /* sum tallies */
  const i64* size;        /* bins per tally */
  float** out;            /* the f32 tallies (zeroed by the caller) */
  double** shadow;        /* float64 re-summation of the same emits, or NULL */
  int priv;               /* privatise per thread (total bytes <= PRIV_BYTES) */
} tm_tallies;

typedef struct {
  float* f[8];
  double* d[8];
  const tm_tallies* T;
  i64 dropped;
} tm_thr;

/* an IEEE compare-and-swap add (host.py:158-161) */
static inline void cas_addf(float* a, float v) {
  u32* u = (u32*)a;
  u32 o = __atomic_load_n(u, __ATOMIC_RELAXED), n;
  do { n = asu(asf(o) + v); } while (!__atomic_compare_exchange_n(u, &o, n, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED));
}
static inline void cas_addd(double* a, double v) {
  u64* u = (u64*)a;
  u64 o = __atomic_load_n(u, __ATOMIC_RELAXED), n;
  do { double x; memcpy(&x, &o, 8); x += v; memcpy(&n, &x, 8); }
  while (!__atomic_compare_exchange_n(u, &o, n, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED));
}

static inline void emit(tm_thr* t, int k, i64 idx, float v) {
  if ((u64)idx >= (u64)t->T->size[k]) { t->dropped++; return; }
  if (t->T->priv) t->f[k][idx] += v; else cas_addf(&t->T->out[k][idx], v);
  if (t->d[k]) t->d[k][idx] += (double)v;
}

static void thr_init(tm_thr* t, const tm_tallies* T) {
  memset(t, 0, sizeof(*t));
  t->T = T;
  for (int k = 0; k < T->nt; ++k) {
    if (T->priv) t->f[k] = (float*)calloc((size_t)T->size[k], sizeof(float));
    if (T->shadow) t->d[k] = (double*)calloc((size_t)T->size[k], sizeof(double));
  }
}

static void thr_flush(tm_thr* t, i32* stats) {
  const tm_tallies* T = t->T;
  for (int k = 0; k < T->nt; ++k) {
    for (i64 i = 0; i < T->size[k]; ++i) {
      if (t->f[k] && t->f[k][i] != 0.0f) cas_addf(&T->out[k][i], t->f[k][i]);
      if (t->d[k] && t->d[k][i] != 0.0) cas_addd(&T->shadow[k][i], t->d[k][i]);
    }
    free(t->f[k]);
    free(t->d[k]);
  }
  if (t->dropped) __atomic_fetch_add(&stats[ST_DROPPED], (i32)t->dropped, __ATOMIC_RELAXED);
}

static int team_size(int nthreads) {
  if (nthreads > 0) return nthreads;
  return omp_get_max_threads();
}

/* ------------------------------------------------------------------------------- C1: quickstart walker */
/* reference examples/quickstart.py:19-28: per step k, u = uniform(fold_in(key, k)); add
 * theta * (1 - x) to hist[int32(x * 16)]; x *= 0.5 + 0.5 u; while x > 0.05.  Gradient: d(sum_b ct[b] hist[b]) /
 * d theta in forward mode, tangent of theta = 1. */
typedef struct { i32 k; u32 trunc; float g, gx; } c1_res;

static inline c1_res c1_item(const float* xs, const u32* keys, float theta, i64 i, int M, tm_thr* t,
                             const float* ct) {
  const u32* key = keys + 2 * i;
  float x = xs[i];
  float dx = 1.0f;          /* tangent of x w.r.t. its own start value x0 */
  i32 k = 0, cap = 0;
  float g = 0.0f, gx = 0.0f;
  while (cap < M && x > 0.05f) {
    u32 fk[2];
    fold_in(key, (u32)k, fk);
    const float u = uniform_f32(fk, 0.0f, 1.0f);
    const i32 idx = f2i(x * 16.0f);
    const float omx = 1.0f - x;
    const float f = 0.5f + 0.5f * u;
    if (t) emit(t, 0, idx, theta * omx);
    if (ct && (u32)idx < 16u) {
      g = g + ct[idx] * omx;               /* d(theta * (1 - x)) / d theta = 1 - x */
      gx = gx + ct[idx] * (-theta * dx);   /* d(theta * (1 - x)) / d x0 = -theta dx */
    }
    k = k + 1;
    x = x * f;
    dx = dx * f;
    ++cap;
  }
  c1_res r = {k, (u32)(cap >= M && x > 0.05f), g, gx};
  return r;
}

int tmref_c1_fwd(const float* xs, const u32* keys, float theta, i64 n, int M, int nthreads, float* hist,
                 double* hist64, i32* ks, uint8_t* trunc, i32* stats) {
  const i64 sz[1] = {16};
  float* outs[1] = {hist};
  double* sh[1] = {hist64};
  tm_tallies T = {1, sz, outs, hist64 ? sh : NULL, 16 * 4 <= PRIV_BYTES};
  i64 ctr = 0;
#pragma omp parallel num_threads(team_size(nthreads))
  {
    fenv_t saved;
    fegetenv(&saved);
    fesetenv(FE_DFL_ENV);
    tm_thr t;
    thr_init(&t, &T);
    for (;;) {
      const i64 i = __atomic_fetch_add(&ctr, 1, __ATOMIC_RELAXED);
      if (i >= n) break;
      const c1_res r = c1_item(xs, keys, theta, i, M, &t, NULL);
      ks[i] = r.k;
      trunc[i] = (uint8_t)r.trunc;
    }
    thr_flush(&t, stats);
    fesetenv(&saved);
  }
  return 0;
}

/* gradient: exact sum over items of each item's f32 forward-mode cotangent; out[0] = d/d theta; per-item trip
 * counts and truncation flags as in the forward pass (the adjoint's own replay flags) */
int tmref_c1_grad(const float* xs, const u32* keys, float theta, i64 n, int M, int nthreads, const float* ct,
                  float* dtheta, float* dxs, i32* ntrunc) {
  exsum tot;
  memset(&tot, 0, sizeof(tot));
  i64 ctr = 0;
  i32 ntr = 0;
#pragma omp parallel num_threads(team_size(nthreads))
  {
    fenv_t saved;
    fegetenv(&saved);
    fesetenv(FE_DFL_ENV);
    exsum e;
    memset(&e, 0, sizeof(e));
    i32 mytr = 0;
    for (;;) {
      const i64 i = __atomic_fetch_add(&ctr, 1, __ATOMIC_RELAXED);
      if (i >= n) break;
      const c1_res r = c1_item(xs, keys, theta, i, M, NULL, ct);
      ex_add(&e, r.g);
      if (dxs) dxs[i] = r.gx;
      mytr += (i32)r.trunc;
    }
#pragma omp critical
    {
      ex_merge(&tot, &e);
      ntr += mytr;
    }
    fesetenv(&saved);
  }
  int bad = 0;
  dtheta[0] = ex_read(&tot, &bad);
  *ntrunc = ntr;
  return bad;
}

/* ---------------------------------------------------------------------------------- C2: 1-D random walk */
/* BASELINE config 2: while 0 <= x <= 1: add 1 to occ[int32(x * 128)], n = normal(fold_in(key, k)),
 * x = x + (drift + 0.02 n).  After the loop add 1 to wall[int32(x > 1)].  Per-item result: k. */
typedef struct { i32 k; u32 trunc; float g; } c2_res;

static inline c2_res c2_item(const float* x0, const u32* keys, float drift, i64 i, int M, tm_thr* t,
                             const float* ct_occ, const float* ct_wall) {
  const u32* key = keys + 2 * i;
  float x = x0[i];
  /* the emitted values are the constant 1: their tangent w.r.t. drift is a symbolic zero, so the cotangent of
   * drift is exactly 0 whatever ct_occ / ct_wall hold (x's tangent only reaches integer bins and the exit test) */
  const float g = 0.0f;
  i32 k = 0, cap = 0;
  while (cap < M && (x >= 0.0f && x <= 1.0f)) {
    const i32 idx = f2i(x * 128.0f);
    if (t) emit(t, 0, idx, 1.0f);
    u32 fk[2];
    fold_in(key, (u32)k, fk);
    const float nz = normal_f32(fk);
    k = k + 1;
    x = x + (drift + 0.02f * nz);
    ++cap;
  }
  const i32 w = x > 1.0f ? 1 : 0;
  if (t) emit(t, 1, w, 1.0f);
  (void)ct_occ;
  (void)ct_wall;
  c2_res r = {k, (u32)(cap >= M && (x >= 0.0f && x <= 1.0f)), g};
  return r;
}

int tmref_c2_fwd(const float* x0, const u32* keys, float drift, i64 n, int M, int nthreads, float* occ,
                 float* wall, double* occ64, double* wall64, i32* ks, uint8_t* trunc, i32* stats) {
  const i64 sz[2] = {128, 2};
  float* outs[2] = {occ, wall};
  double* sh[2] = {occ64, wall64};
  tm_tallies T = {2, sz, outs, occ64 ? sh : NULL, (128 + 2) * 4 <= PRIV_BYTES};
  i64 ctr = 0;
#pragma omp parallel num_threads(team_size(nthreads))
  {
    fenv_t saved;
    fegetenv(&saved);
    fesetenv(FE_DFL_ENV);
    tm_thr t;
    thr_init(&t, &T);
    for (;;) {
      const i64 i = __atomic_fetch_add(&ctr, 1, __ATOMIC_RELAXED);
      if (i >= n) break;
      const c2_res r = c2_item(x0, keys, drift, i, M, &t, NULL, NULL);
      if (ks) ks[i] = r.k;
      if (trunc) trunc[i] = (uint8_t)r.trunc;
    }
    thr_flush(&t, stats);
    fesetenv(&saved);
  }
  return 0;
}

int tmref_c2_grad(const float* x0, const u32* keys, float drift, i64 n, int M, int nthreads, const float* ct_occ,
                  const float* ct_wall, float* ddrift, i32* ntrunc) {
  exsum tot;
  memset(&tot, 0, sizeof(tot));
  i64 ctr = 0;
  i32 ntr = 0;
#pragma omp parallel num_threads(team_size(nthreads))
  {
    fenv_t saved;
    fegetenv(&saved);
    fesetenv(FE_DFL_ENV);
    exsum e;
    memset(&e, 0, sizeof(e));
    i32 mytr = 0;
    for (;;) {
      const i64 i = __atomic_fetch_add(&ctr, 1, __ATOMIC_RELAXED);
      if (i >= n) break;
      const c2_res r = c2_item(x0, keys, drift, i, M, NULL, ct_occ, ct_wall);
      ex_add(&e, r.g);
      mytr += (i32)r.trunc;
    }
#pragma omp critical
    {
      ex_merge(&tot, &e);
      ntr += mytr;
    }
    fesetenv(&saved);
  }
  int bad = 0;
  ddrift[0] = ex_read(&tot, &bad);
  *ntrunc = ntr;
  return bad;
}

/* the C2 starting points: x0_i = uniform(fold_in(key_i, 0xFFFFFFFF), 0.2, 0.8) (pins the host input generator) */
void tmref_c2_x0(const u32* keys, i64 n, float* x0) {
  for (i64 i = 0; i < n; ++i) {
    u32 fk[2];
    fold_in(keys + 2 * i, 0xFFFFFFFFu, fk);
    x0[i] = uniform_f32(fk, 0.2f, 0.8f);
  }
}

int tmref_max_threads(void) { return omp_get_max_threads(); }
