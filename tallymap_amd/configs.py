"""The benchmark item programs and their synthetic inputs.

Each config gives: the item function (written against tallymap_amd's jax-shaped API, as a reference user writes
it against JAX), its `vmap` outputs / in_axes / max_steps, a seeded input generator, and the cotangent of the
gradient the config asks for.  Inputs are generated on the host with tallymap_amd.random (numpy threefry), so the
GPU and the oracle see the same arrays.

C1  the reference's quickstart walker (reference examples/quickstart.py:19-30).
C2  1-D random walk with absorbing walls: per step one occupancy emit at int32(x * 128), then
    x += drift + 0.02 * normal(fold_in(key, k)); after the loop one emit into the wall histogram.
C3  photon transport in a slab 0 <= z <= 5 (mu_a = 0.1, mu_s = 0.9): exponential flights, a deposit of
    w * mu_a / mu_t per interaction into a (depth, radius) 64 x 64 histogram, Henyey-Greenstein scattering
    (g = 0.8), Russian roulette below w = 0.01 (survival 0.1).  Gradient w.r.t. mu_a.
C4  walk on spheres for the Laplace equation in the unit disk: hop to a uniform point of the largest inscribed
    circle until within 1e-3 of the boundary, score a * sin(3 theta_exit) into a per-walker (N, 1) tally and into
    a 256 x 256 histogram of start positions.  Gradient w.r.t. a.
C5  damped driven pendulums theta'' = -0.1 theta' - sin(theta) + A cos(2t / 3), adaptive Dormand-Prince 5(4)
    (rtol 1e-6, atol 1e-8) from t = 0 to 50; final (theta, omega) into a per-item (N, 2) tally.  Gradient of the
    summed final energy w.r.t. A.
"""
import numpy as np

from . import lax, random
from . import numpy as jnp
from ._api import Sum

NB = 16


# ------------------------------------------------------------------------------------------------- C1
def c1_item(t, x, key, theta):
    """ONE walker (reference examples/quickstart.py:19-26)."""
    def body(c):
        k, x, t = c
        u = random.uniform(random.fold_in(key, k))
        t = t.add("hist", (x * NB).astype(jnp.int32), theta * (1.0 - x))
        return k + 1, x * (0.5 + 0.5 * u), t
    k, x, t = lax.while_loop(lambda c: c[1] > 0.05, body, (0, x, t))
    return t, k


C1 = dict(item=c1_item, outputs={"hist": Sum((NB,))}, in_axes=(0, 0, None), max_steps=100)


def c1_inputs(n=10_000, seed=0):
    """xs = linspace(0.1, 0.99, N) as float32 (computed in float64, rounded once), keys = split(PRNGKey(seed), N),
    theta = 2."""
    xs = np.linspace(0.1, 0.99, n, dtype=np.float64).astype(np.float32)
    keys = random.split(random.PRNGKey(seed), n)
    return xs, keys, np.float32(2.0)


# ------------------------------------------------------------------------------------------------- C2
def c2_item(t, x, key, drift):
    """ONE walker on [0, 1]: occupancy of its bin every step, absorbed at either wall."""
    def cond(c):
        k, x, t = c
        return (x >= 0.0) & (x <= 1.0)

    def body(c):
        k, x, t = c
        t = t.add("occ", (x * 128).astype(jnp.int32), 1.0)
        n = random.normal(random.fold_in(key, k))
        return k + 1, x + (drift + 0.02 * n), t
    k, x, t = lax.while_loop(cond, body, (0, x, t))
    t = t.add("wall", (x > 1.0).astype(jnp.int32), 1.0)
    return t, k


C2 = dict(item=c2_item, outputs={"occ": Sum((128,)), "wall": Sum((2,))}, in_axes=(0, 0, None), max_steps=65_536)


def c2_inputs(n=4_194_304, seed=0):
    """keys = split(PRNGKey(seed), N); x0_i = uniform(fold_in(key_i, 0xFFFFFFFF), 0.2, 0.8) (a stream disjoint from
    the steps' fold_in(key_i, k)); drift = 1e-3."""
    keys = random.split(random.PRNGKey(seed), n)
    x0 = random.uniform(random.fold_in(keys, 0xFFFFFFFF), (), np.float32, 0.2, 0.8)
    return x0.astype(np.float32), keys, np.float32(1e-3)


# ------------------------------------------------------------------------------------------------- C3
C3_MU_S = 0.9           # scattering coefficient (1/length)
C3_G = 0.8              # Henyey-Greenstein anisotropy
C3_DEPTH = 5.0          # slab thickness
C3_NB = 64              # bins per axis: depth z in [0, 5), radius r in [0, 5)


def c3_item(t, key, mu_a):
    """ONE photon packet entering the slab at the origin along +z with weight 1."""
    mu_t = mu_a + C3_MU_S
    frac = mu_a / mu_t
    albedo = C3_MU_S / mu_t
    g = C3_G

    def body(c):
        k, p, d, w, t = c
        u = random.uniform(random.fold_in(key, k), (4,))
        s = -jnp.log(1.0 - u[0]) / mu_t                          # exponential free path, mean 1 / mu_t
        p = p + s * d
        esc = (p[2] < 0.0) | (p[2] > C3_DEPTH)
        r = jnp.sqrt(p[0] * p[0] + p[1] * p[1])
        iz = (p[2] * (C3_NB / C3_DEPTH)).astype(jnp.int32)
        ir = (r * (C3_NB / C3_DEPTH)).astype(jnp.int32)
        t = t.add("absorbed", (jnp.where(esc, -1, iz), ir), w * frac)   # escaped: index -1, dropped
        w = w * albedo
        # Henyey-Greenstein deflection cos(theta), azimuth phi, direction update (MCML's formulas)
        tmp = (1.0 - g * g) / (1.0 - g + 2.0 * g * u[1])
        cost = (1.0 + g * g - tmp * tmp) / (2.0 * g)
        sint = jnp.sqrt(jnp.maximum(0.0, 1.0 - cost * cost))
        phi = (2.0 * jnp.pi) * u[2]
        cp, sp = jnp.cos(phi), jnp.sin(phi)
        ux, uy, uz = d[0], d[1], d[2]
        temp = jnp.sqrt(jnp.maximum(0.0, 1.0 - uz * uz))
        near = jnp.abs(uz) > 0.99999
        den = jnp.where(near, 1.0, temp)
        nx = jnp.where(near, sint * cp, sint * (ux * uz * cp - uy * sp) / den + ux * cost)
        ny = jnp.where(near, sint * sp, sint * (uy * uz * cp + ux * sp) / den + uy * cost)
        nz = jnp.where(near, jnp.sign(uz) * cost, -sint * cp * temp + uz * cost)
        d = jnp.stack([nx, ny, nz])
        # Russian roulette
        w = jnp.where(w < 0.01, jnp.where(u[3] < 0.1, w * 10.0, 0.0), w)
        w = jnp.where(esc, 0.0, w)
        return k + 1, p, d, w, t
    init = (0, jnp.array([0.0, 0.0, 0.0], jnp.float32), jnp.array([0.0, 0.0, 1.0], jnp.float32),
            jnp.float32(1.0), t)
    k, p, d, w, t = lax.while_loop(lambda c: c[3] > 0.0, body, init)
    return t, k


# (opts: the replay gradient's refill -- photon histories of very different lengths, so a wave takes new items as
# soon as 8 of its lanes are free)
C3 = dict(item=c3_item, outputs={"absorbed": Sum((C3_NB, C3_NB))}, in_axes=(0, None), max_steps=1024,
          opts={"rev_refill": 8})


def c3_inputs(n=4_194_304, seed=0):
    """keys = split(PRNGKey(seed), N); mu_a = 0.1."""
    return random.split(random.PRNGKey(seed), n), np.float32(0.1)


# ------------------------------------------------------------------------------------------------- C4
C4_EPS = 1e-3
C4_NB = 256


def c4_item(t, p0, key, item_id, a):
    """ONE walker from p0 (|p0| < 0.95) until it is within 1e-3 of the unit circle."""
    def cond(c):
        k, p = c
        return 1.0 - jnp.sqrt(p[0] * p[0] + p[1] * p[1]) >= C4_EPS

    def body(c):
        k, p = c
        R = 1.0 - jnp.sqrt(p[0] * p[0] + p[1] * p[1])           # radius of the largest inscribed circle
        phi = (2.0 * jnp.pi) * random.uniform(random.fold_in(key, k))
        return k + 1, p + R * jnp.stack([jnp.cos(phi), jnp.sin(phi)])
    k, p = lax.while_loop(cond, body, (0, p0))
    score = a * jnp.sin(3.0 * jnp.arctan2(p[1], p[0]))
    t = t.add("walker", (item_id, 0), score)
    ix = ((p0[0] + 1.0) * (C4_NB / 2.0)).astype(jnp.int32)
    iy = ((p0[1] + 1.0) * (C4_NB / 2.0)).astype(jnp.int32)
    t = t.add("grid", (ix, iy), score)
    return t, k


def c4_config(n):
    return dict(item=c4_item, outputs={"walker": Sum((n, 1)), "grid": Sum((C4_NB, C4_NB))},
                in_axes=(0, 0, 0, None), max_steps=1024)


C4 = c4_config(4_194_304)


def c4_inputs(n=4_194_304, seed=0):
    """start points uniform in the disk of radius 0.95 (r = 0.95 sqrt(u1), angle 2 pi u2 in float64 from numpy's
    PCG64 with `seed`, rounded to float32), keys = split(PRNGKey(seed), N), item_id = arange(N), a = 0.75."""
    rng = np.random.default_rng(seed)
    r = 0.95 * np.sqrt(rng.uniform(0.0, 1.0, n))
    th = rng.uniform(0.0, 2.0 * np.pi, n)
    p0 = np.stack([r * np.cos(th), r * np.sin(th)], 1).astype(np.float32)
    return p0, random.split(random.PRNGKey(seed), n), np.arange(n, dtype=np.int32), np.float32(0.75)


# ------------------------------------------------------------------------------------------------- C5
C5_DAMP = 0.1
C5_WD = 2.0 / 3.0
C5_T1 = 50.0
C5_RTOL = 1e-6
C5_ATOL = 1e-8
C5_H0 = 0.01
# Dormand & Prince (1980) RK5(4)7M: nodes, stage weights, 5th-order weights (= the last stage row), error weights
DP_C = (1.0 / 5, 3.0 / 10, 4.0 / 5, 8.0 / 9)
DP_A = ((1.0 / 5,),
        (3.0 / 40, 9.0 / 40),
        (44.0 / 45, -56.0 / 15, 32.0 / 9),
        (19372.0 / 6561, -25360.0 / 2187, 64448.0 / 6561, -212.0 / 729),
        (9017.0 / 3168, -355.0 / 33, 46732.0 / 5247, 49.0 / 176, -5103.0 / 18656))
DP_B = (35.0 / 384, 500.0 / 1113, 125.0 / 192, -2187.0 / 6784, 11.0 / 84)          # stages 1, 3, 4, 5, 6
DP_E = (71.0 / 57600, -71.0 / 16695, 71.0 / 1920, -17253.0 / 339200, 22.0 / 525, -1.0 / 40)  # 1, 3, 4, 5, 6, 7


def c5_rhs(t, y, A):
    th, om = y[0], y[1]
    return jnp.stack([om, -C5_DAMP * om - jnp.sin(th) + A * jnp.cos(C5_WD * t)])


def c5_item(t, th0, om0, item_id, A):
    """ONE pendulum from (th0, om0): adaptive DP5(4) with FSAL to t = 50, final state into `state`."""
    def cond(c):
        return c[1] < C5_T1

    def body(c):
        k, tt, y, f0, h = c
        h = jnp.minimum(h, C5_T1 - tt)
        a = DP_A
        k1 = f0
        k2 = c5_rhs(tt + DP_C[0] * h, y + h * (a[0][0] * k1), A)
        k3 = c5_rhs(tt + DP_C[1] * h, y + h * (a[1][0] * k1 + a[1][1] * k2), A)
        k4 = c5_rhs(tt + DP_C[2] * h, y + h * (a[2][0] * k1 + a[2][1] * k2 + a[2][2] * k3), A)
        k5 = c5_rhs(tt + DP_C[3] * h, y + h * (a[3][0] * k1 + a[3][1] * k2 + a[3][2] * k3 + a[3][3] * k4), A)
        k6 = c5_rhs(tt + h, y + h * (a[4][0] * k1 + a[4][1] * k2 + a[4][2] * k3 + a[4][3] * k4 + a[4][4] * k5), A)
        b = DP_B
        y5 = y + h * (b[0] * k1 + b[1] * k3 + b[2] * k4 + b[3] * k5 + b[4] * k6)
        k7 = c5_rhs(tt + h, y5, A)
        e = DP_E
        ev = h * (e[0] * k1 + e[1] * k3 + e[2] * k4 + e[3] * k5 + e[4] * k6 + e[5] * k7)
        sc = C5_ATOL + C5_RTOL * jnp.maximum(jnp.abs(y), jnp.abs(y5))
        q = ev / sc
        err = jnp.sqrt((q[0] * q[0] + q[1] * q[1]) * 0.5)
        ok = err <= 1.0
        fac = lax.stop_gradient(jnp.clip(0.9 * jnp.exp(-0.2 * jnp.log(err)), 0.2, 10.0))
        return (k + 1, jnp.where(ok, tt + h, tt), jnp.where(ok, y5, y), jnp.where(ok, k7, f0), h * fac)
    y0 = jnp.stack([th0, om0])
    f0 = jnp.stack([om0, -C5_DAMP * om0 - jnp.sin(th0) + A])    # c5_rhs at t = 0: A * cos(0) = A exactly
    init = (0, jnp.float32(0.0), y0, f0, jnp.float32(C5_H0))
    k, tt, y, f, h = lax.while_loop(cond, body, init)
    t = t.add("state", (item_id, 0), y[0])
    t = t.add("state", (item_id, 1), y[1])
    return t, k


def c5_config(n):
    # (opts: every pendulum integrates the same interval, so its step count falls in a narrow band: the replay
    # gradient refills a wave only when all 64 lanes are free, keeping counting and reversing lanes apart)
    return dict(item=c5_item, outputs={"state": Sum((n, 2))}, in_axes=(0, 0, 0, None), max_steps=20_000,
                opts={"rev_refill": 64})


C5 = c5_config(1_048_576)


def c5_inputs(n=1_048_576, seed=0):
    """theta0 ~ U(-pi, pi), omega0 ~ U(-2, 2) in float64 from numpy's PCG64 with `seed`, rounded to float32;
    item_id = arange(N); A = 1.2."""
    rng = np.random.default_rng(seed)
    th0 = rng.uniform(-np.pi, np.pi, n).astype(np.float32)
    om0 = rng.uniform(-2.0, 2.0, n).astype(np.float32)
    return th0, om0, np.arange(n, dtype=np.int32), np.float32(1.2)


def c5_energy_ct(state):
    """the cotangent of sum_i E_i, E = omega^2 / 2 + 1 - cos(theta), at the final states (N, 2): (sin theta,
    omega) per item, in float32."""
    st = np.asarray(state, np.float32)
    return np.stack([np.sin(st[:, 0].astype(np.float64)), st[:, 1].astype(np.float64)], 1).astype(np.float32)


CONFIGS = {"c1": C1, "c2": C2, "c3": C3, "c4": C4, "c5": C5}
SIZED = {"c4": c4_config, "c5": c5_config}
# the modules built ahead of time (the benchmark and the GPU tests' sizes; other sizes compile on first use)
PREBUILD = [("c1", C1), ("c2", C2), ("c3", C3), ("c4", c4_config(65_536)), ("c4", C4), ("c5", c5_config(16_384)),
            ("c5", C5)]
