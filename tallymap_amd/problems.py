"""The reference's own benchmark problems, as tallymap_amd items: the "natural" group of its plain-JAX comparison
suite, whose kernel-backend timings it publishes (NVIDIA L40S, JAX 0.5.3, divergence level "mid";
docs/performance_detail.md).  Each is written here from the problem's description and arithmetic in
benchmarks/vs_jax/problems/<name>.py -- same item, same inputs (seeded as there), same loss -- so the MI355X
timings can be set beside the published ones:

    random_walk       4,194,304 walkers, 64-bin histogram, per-step emits      fwd 3.1 ms, grad 8.84 ms
    transport         4,194,304 photon packets, 32 sensors, one emit per item   fwd 1.77 ms, grad 16.3 ms
    walk_on_spheres   4,194,304 walkers, 64 evaluation points (Poisson, 2-D)    fwd 1.27 ms, grad 8.68 ms
    ode_ensemble      1,048,576 Van der Pol trajectories, Bogacki-Shampine 3(2)  fwd 5.32 ms, grad 25.9 ms
    barrier           4,194,304 up-and-out call paths, 252 daily steps          fwd 8.16 ms, grad 38.3 ms
    gillespie         1,048,576 Schloegl SSA realisations (forward only)        fwd 30 ms
    shower            262,144 roots of a branching shower (spawn)               fwd 1.66 ms, grad 14.9 ms

"grad" there is jax.grad of the problem's scalar loss of the tally w.r.t. theta: the forward call plus the
adjoint, whose cotangent is the loss's derivative at the forward's tally.  PROBLEMS[name] holds: item, outputs,
in_axes, argnum (theta's position), inputs(n) (numpy arrays: per-item operands, then broadcast ones), ct(tallies,
n, inputs) (the loss's cotangent of each tally output), loss(tallies, n, inputs), published (ms), n (the published
size).  The JAX PRNG calls are this package's restatement (tallymap_amd.random); the keys are split from the same
seeds as the reference's setup()."""
import math

import numpy as np

from . import _api, lax
from . import numpy as jnp
from . import random as R

F32 = np.float32


def _like(x, a):
    """the host array `a` as an array of x's kind (a torch tensor on x's device, or numpy)"""
    if type(x).__module__.startswith("torch"):
        import torch
        return torch.as_tensor(a, device=x.device)
    return np.asarray(a)


# ----------------------------------------------------------------------------------------------- random_walk
# reference benchmarks/vs_jax/problems/random_walk.py:36-63, 91-94 (step, setup, sim_of, loss)
RW_NB, RW_WMIN = 64, 0.01


def rw_item(t, key, decay, th):
    """one walker of weight w = decay^k: each step draws u, adds w th0 + th1 u + th2 w^2 to bin floor(64 u)."""
    def body(c):
        k, w, t = c
        u = R.uniform(R.fold_in(key, k))
        b = (u * RW_NB).astype(jnp.int32)
        t = t.add("hist", b, w * th[0] + th[1] * u + th[2] * w * w)
        return k + 1, w * decay, t
    k, _, t = lax.while_loop(lambda c: c[1] > RW_WMIN, body, (np.int32(0), F32(1.0), t))
    return t, k


def rw_inputs(n):
    rng = np.random.default_rng(0)
    decay = rng.uniform(0.60, 0.95, n).astype(F32)
    wq = rng.uniform(0.5, 1.5, RW_NB).astype(F32)
    return (R.split(R.PRNGKey(0), n), decay, np.array([1.0, 0.5, 0.25], F32)), {"wq": wq}


def rw_loss(tal, n, extra):
    return (_like(tal["hist"], extra["wq"]) * tal["hist"] ** 2).sum() / RW_NB


def rw_ct(tal, n, extra):
    return {"hist": 2.0 * _like(tal["hist"], extra["wq"]) * tal["hist"] / RW_NB}


# ------------------------------------------------------------------------------------------------- transport
# reference benchmarks/vs_jax/problems/transport.py:36-75, 131-136
TR_NS, TR_WMIN = 32, 1e-3


def tr_item(t, p0, key, th, eff):
    """one packet in the unit disk: exponential flights of mean th0 with isotropic scattering, weight times
    exp(-th1 s) per flight, until it leaves the disk (deposit w eff[sensor] at its exit angle) or w < 1e-3."""
    def alive(c):
        return (~c[4]) & (c[2] > TR_WMIN)

    def body(c):
        p, d, w, k, _ = c
        u = R.uniform(R.fold_in(key, k), (2,))
        s = -jnp.log1p(-u[0]) * th[0]
        p2 = p + s * d
        esc = jnp.sum(p2 * p2) >= 1.0
        phi = 2.0 * jnp.pi * u[1]
        return p2, jnp.stack([jnp.cos(phi), jnp.sin(phi)]), w * jnp.exp(-th[1] * s), k + 1, esc
    c0 = (p0, np.array([1.0, 0.0], F32), F32(1.0), np.int32(0), np.bool_(False))
    p, _, w, k, esc = lax.while_loop(alive, body, c0)
    i = ((jnp.arctan2(p[1], p[0]) + jnp.pi) * (TR_NS / (2.0 * jnp.pi))).astype(jnp.int32) % TR_NS
    return t.add("Q", jnp.where(esc, i, -1), w * eff[i]), k


def tr_inputs(n):
    rng = np.random.default_rng(0)
    r = np.sqrt(rng.uniform(0, 0.25, n))
    a = rng.uniform(0, 2 * np.pi, n)
    p0 = np.stack([r * np.cos(a), r * np.sin(a)], 1).astype(F32)
    eff = (0.8 + 0.2 * np.cos(np.arange(TR_NS))).astype(F32)
    tgt = rng.uniform(5.0, 30.0, TR_NS).astype(F32)
    return (p0, R.split(R.PRNGKey(0), n), np.array([0.2, 0.5], F32), eff), {"tgt": tgt}


def tr_loss(tal, n, extra):
    return ((tal["Q"] - _like(tal["Q"], extra["tgt"])) ** 2).sum() / TR_NS


def tr_ct(tal, n, extra):
    return {"Q": 2.0 * (tal["Q"] - _like(tal["Q"], extra["tgt"])) / TR_NS}


# ------------------------------------------------------------------------------------------- walk_on_spheres
# reference benchmarks/vs_jax/problems/walk_on_spheres.py:40-83, 98-110, 126-128
WS_M, WS_EPS = 64, 1e-3


def _ws_sdf(x):
    return jnp.minimum(jnp.minimum(x[0], 1.0 - x[0]), jnp.minimum(x[1], 1.0 - x[1]))


def ws_item(t, x0, pid, key, th):
    """one walk-on-spheres walker in the unit square (Poisson, laplacian u = -th0 exp(-th1 |y - c|^2), boundary
    th2 + th3 cos(th4 pi (x + y))): hops to the largest inscribed circle until within 1e-3 of the boundary, each
    ball adding the single-sample source estimate (R^2 / 2) ln(R / r) f(y); then the boundary value at the
    nearest boundary point.  One emit per walker into its evaluation point."""
    def body(c):
        x, acc, k = c
        Rr = _ws_sdf(x)
        u = R.uniform(R.fold_in(key, k), (3,))
        r = Rr * jnp.sqrt(u[0])
        a = 2.0 * jnp.pi * u[1]
        y = x + r * jnp.stack([jnp.cos(a), jnp.sin(a)])
        g = -0.5 * jnp.log(jnp.maximum(u[0], 1e-20))
        f = th[0] * jnp.exp(-th[1] * ((y[0] - 0.5) ** 2 + (y[1] - 0.5) ** 2))
        acc = acc + 0.5 * Rr * Rr * g * f
        a2 = 2.0 * jnp.pi * u[2]
        return x + Rr * jnp.stack([jnp.cos(a2), jnp.sin(a2)]), acc, k + 1
    x, acc, k = lax.while_loop(lambda c: _ws_sdf(c[0]) > WS_EPS, body, (x0, F32(0.0), np.int32(0)))
    i = jnp.argmin(jnp.stack([x[0], 1.0 - x[0], x[1], 1.0 - x[1]]))
    xb = jnp.stack([jnp.where(i == 0, 0.0, jnp.where(i == 1, 1.0, x[0])),
                    jnp.where(i == 2, 0.0, jnp.where(i == 3, 1.0, x[1]))])
    acc = acc + (th[2] + th[3] * jnp.cos(th[4] * jnp.pi * (xb[0] + xb[1])))
    return t.add("u", pid, acc), k


def ws_inputs(n):
    rng = np.random.default_rng(0)
    x0 = rng.uniform(0.02, 0.98, (n, 2)).astype(F32)
    pid = (np.arange(n) % WS_M).astype(np.int32)
    wts = rng.uniform(0.5, 1.5, WS_M).astype(F32)
    tgt = rng.uniform(0.0, 1.0, WS_M).astype(F32)
    return (x0, pid, R.split(R.PRNGKey(1), n), np.array([1.0, 4.0, 0.3, 0.5, 2.0], F32)), {"wts": wts, "tgt": tgt}


def ws_loss(tal, n, extra):
    u = tal["u"]
    return (_like(u, extra["wts"]) * (u / (n / WS_M) - _like(u, extra["tgt"])) ** 2).sum() / WS_M


def ws_ct(tal, n, extra):
    w = n / WS_M
    u = tal["u"]
    return {"u": 2.0 * _like(u, extra["wts"]) * (u / w - _like(u, extra["tgt"])) / (WS_M * w)}


# ---------------------------------------------------------------------------------------------- ode_ensemble
# reference benchmarks/vs_jax/problems/ode_ensemble.py:37-86, 94-101, 139-151, 154-156
OD_G, OD_T, OD_RTOL, OD_ATOL = 32, 20.0, 1e-3, 1e-5


def _od_rhs(t, y, mu, th):
    return jnp.stack([y[1], mu * th[0] * (1.0 - y[0] * y[0]) * y[1] - y[0] - th[1] * y[1] + th[2] * jnp.sin(2.0 * t)])


def od_item(t_, y0, mu, gid, th):
    """one forced Van der Pol trajectory on [0, 20], Bogacki-Shampine 3(2) trial steps (accepted when the scaled
    error norm is <= 1; h *= clip(0.9 err^(-1/3), 0.2, 5), the factor held constant in derivatives); the item
    emits tanh(y0) + 0.5 y1 exp(-0.1 y1^2) at the end into its group."""
    def body(c):
        t, y, h, na, nr = c
        h = jnp.minimum(h, OD_T - t)
        k1 = _od_rhs(t, y, mu, th)
        k2 = _od_rhs(t + 0.5 * h, y + 0.5 * h * k1, mu, th)
        k3 = _od_rhs(t + 0.75 * h, y + 0.75 * h * k2, mu, th)
        yn = y + h * (2.0 / 9.0 * k1 + 1.0 / 3.0 * k2 + 4.0 / 9.0 * k3)
        k4 = _od_rhs(t + h, yn, mu, th)
        e = h * ((2.0 / 9.0 - 7.0 / 24.0) * k1 + (1.0 / 3.0 - 0.25) * k2 + (4.0 / 9.0 - 1.0 / 3.0) * k3
                 + (-0.125) * k4)
        sc = OD_ATOL + OD_RTOL * jnp.maximum(jnp.abs(y), jnp.abs(yn))
        err = jnp.max(jnp.abs(e) / sc)
        ok = err <= 1.0
        fac = lax.stop_gradient(jnp.clip(0.9 * jnp.power(jnp.maximum(err, 1e-10), -1.0 / 3.0), 0.2, 5.0))
        return (jnp.where(ok, t + h, t), jnp.where(ok, yn, y), jnp.maximum(h * fac, 1e-7),
                na + ok.astype(jnp.int32), nr + (~ok).astype(jnp.int32))
    c0 = (F32(0.0), y0, F32(1e-2), np.int32(0), np.int32(0))
    _, y, _, na, nr = lax.while_loop(lambda c: c[0] < OD_T, body, c0)
    o = jnp.tanh(y[0]) + 0.5 * y[1] * jnp.exp(-0.1 * y[1] * y[1])
    return t_.add("obs", gid, o), na + nr


def od_inputs(n):
    rng = np.random.default_rng(0)
    y0 = np.stack([rng.uniform(-2.0, 2.0, n), rng.uniform(-1.0, 1.0, n)], 1).astype(F32)
    mu = np.exp(rng.uniform(np.log(0.5), np.log(6.0), n)).astype(F32)
    gid = (np.arange(n) % OD_G).astype(np.int32)
    w = rng.uniform(0.5, 1.5, OD_G).astype(F32)
    return (y0, mu, gid, np.array([1.0, 0.05, 0.3], F32)), {"w": w}


def od_loss(tal, n, extra):
    return (_like(tal["obs"], extra["w"]) * (tal["obs"] / (n / OD_G)) ** 2).sum()


def od_ct(tal, n, extra):
    wn = n / OD_G
    return {"obs": 2.0 * _like(tal["obs"], extra["w"]) * tal["obs"] / (wn * wn)}


# --------------------------------------------------------------------------------------------------- barrier
# reference benchmarks/vs_jax/problems/barrier.py:36-63, 72-100, 104-106
BA_NK, BA_KSTEPS, BA_T, BA_BAR = 8, 252, 1.0, 1.3
BA_DT = BA_T / BA_KSTEPS
BA_SQDT = math.sqrt(BA_DT)


def ba_item(t, key, th, strikes):
    """one price path of an up-and-out call, 252 daily log-normal steps (th = sigma, r, S0), stopped once S reaches
    1.3 S0; the discounted payoff ladder over 8 strikes (0 when knocked out) and the knock-out count."""
    def body(c):
        k, S, alive = c
        z = R.normal(R.fold_in(key, k))
        S = S * jnp.exp((th[1] - 0.5 * th[0] * th[0]) * BA_DT + th[0] * BA_SQDT * z)
        return k + 1, S, alive & (S < BA_BAR * th[2])
    k, S, alive = lax.while_loop(lambda c: (c[0] < BA_KSTEPS) & c[2], body, (np.int32(0), th[2], np.bool_(True)))
    pay = jnp.exp(-th[1] * BA_T) * jnp.maximum(S - strikes * th[2], 0.0) * alive.astype(jnp.float32)
    t = t.add("price", jnp.arange(BA_NK, dtype=jnp.int32), pay)
    t = t.add("ko", 0, (~alive).astype(jnp.float32))
    return t, (pay[BA_NK // 2], k)


def ba_inputs(n):
    return ((R.split(R.PRNGKey(3), n), np.array([0.25, 0.03, 100.0], F32),
             np.linspace(0.8, 1.2, BA_NK).astype(F32)), {"w": np.linspace(1.0, 2.0, BA_NK).astype(F32)})


def ba_loss(tal, n, extra):
    return (_like(tal["price"], extra["w"]) * tal["price"] / n).sum()


def ba_ct(tal, n, extra):
    return {"price": _like(tal["price"], extra["w"]) / n}


# ------------------------------------------------------------------------------------------------- gillespie
# reference benchmarks/vs_jax/problems/gillespie.py:37-95, 101-116 (forward only: a jump process has no pathwise
# derivative)
GI_NB, GI_T, GI_A, GI_B, GI_XMAX = 32, 0.5, 1.0e5, 2.0e5, 1000.0


def gi_item(t_, x0, key, c):
    """one exact SSA realisation of the Schloegl network (A + 2X -> 3X, 3X -> A + 2X, B -> X, X -> B with A, B
    buffered) until t = 0.5: per event tau = -ln(u0) / a0 and the reaction by a linear search of u1 a0 over the
    cumulative propensities; the histogram of X(T) and the sum of X(T)."""
    def body(s):
        tt, x, n = s
        xf = x.astype(jnp.float32)
        a = jnp.maximum(jnp.stack([c[0] * GI_A * xf * (xf - 1.0) * 0.5, c[1] * xf * (xf - 1.0) * (xf - 2.0) / 6.0,
                                   c[2] * GI_B, c[3] * xf]), 0.0)
        a0 = jnp.sum(a)
        u = R.uniform(R.fold_in(key, n), (2,))
        tau = -jnp.log(jnp.maximum(u[0], 1e-20)) / jnp.maximum(a0, 1e-20)
        r = jnp.clip(jnp.sum((u[1] * a0 > jnp.cumsum(a)).astype(jnp.int32)), 0, 3)
        dx = 1 - 2 * (r & 1)                        # the stoichiometry (+1, -1, +1, -1)[r]
        return tt + tau, jnp.clip(x + dx, 0, 2000), n + 1
    _, x, n = lax.while_loop(lambda s: s[0] < GI_T, body, (F32(0.0), x0, np.int32(0)))
    b = jnp.clip((x.astype(jnp.float32) * (GI_NB / GI_XMAX)).astype(jnp.int32), 0, GI_NB - 1)
    t_ = t_.add("hist", b, 1.0)
    t_ = t_.add("mean", 0, x.astype(jnp.float32))
    return t_, (x, n)


def gi_inputs(n):
    rng = np.random.default_rng(0)
    x0 = rng.integers(100, 501, n).astype(np.int32)
    return (x0, R.split(R.PRNGKey(2), n), np.array([3.0e-7, 1.0e-4, 1.0e-3, 3.5], F32)), {}


# ---------------------------------------------------------------------------------------------------- shower
# reference benchmarks/vs_jax/problems/shower.py:55-90, 130-150, 160-165 (its Queue holds every child of the call;
# here a Queue holds one generation, and a generation of this binary tree has at most n particles)
SH_NZ, SH_DEPTH, SH_KMAX, SH_EMIN, SH_PSPLIT = 16, 6, 24, 1e-3, 0.03


def sh_item(t, s, th):
    """one particle: steps along z (exponential, mean 0.5) depositing th0 of its energy per step, until E <= 1e-3
    or 24 steps; at most once, with probability 0.03 per step below generation 6, it splits off a child carrying
    th1 x (0.5 .. 1) of the energy left.  The deposit profile over every particle of the tree.  (`did`, whether
    the particle has split, is an int32 0 / 1 here, a bool there.)"""
    def body(c):
        s, t = c
        k = R.fold_in(s["key"], s["n"])
        u = R.uniform(k, (3,))
        z = s["z"] - jnp.log1p(-u[0]) * 0.5
        dep = s["E"] * th[0]
        split = (u[1] < SH_PSPLIT) & (s["g"] < SH_DEPTH) & (s["did"] == 0) & (s["E"] > SH_EMIN)
        ec = (s["E"] - dep) * th[1] * (0.5 + 0.5 * u[2])
        t = t.add("dep", jnp.clip(jnp.floor(z * 2.0).astype(jnp.int32), 0, SH_NZ - 1), dep)
        t = t.spawn(dict(E=ec, z=z, key=R.fold_in(k, 1), g=s["g"] + 1, n=np.int32(0), did=np.int32(0)), when=split)
        e = s["E"] - dep - jnp.where(split, ec, 0.0)
        return dict(E=e, z=z, key=s["key"], g=s["g"], n=s["n"] + 1,
                    did=jnp.where(split, 1, s["did"])), t
    s, t = lax.while_loop(lambda c: (c[0]["E"] > SH_EMIN) & (c[0]["n"] < SH_KMAX), body, (s, t))
    return t


def sh_inputs(n):
    rng = np.random.default_rng(0)
    roots = dict(E=rng.uniform(1.0, 2.0, n).astype(F32), z=np.zeros(n, F32), key=R.split(R.PRNGKey(0), n),
                 g=np.zeros(n, np.int32), n=np.zeros(n, np.int32), did=np.zeros(n, np.int32))
    wz = rng.uniform(0.5, 1.5, SH_NZ).astype(F32)
    return (roots, np.array([0.2, 0.6], F32)), {"wz": wz}


def sh_loss(tal, n, extra):
    return (_like(tal["dep"], extra["wz"]) * tal["dep"]).sum()


def sh_ct(tal, n, extra):
    return {"dep": _like(tal["dep"], extra["wz"])}


PROBLEMS = {
    "random_walk": dict(item=rw_item, outputs={"hist": _api.Sum((RW_NB,))}, in_axes=(0, 0, None), argnum=2,
                        inputs=rw_inputs, ct=rw_ct, loss=rw_loss, n=4_194_304,
                        published={"fwd_ms": 3.1, "grad_ms": 8.84, "jvp_ms": 3.14, "jacfwd_ms": 3.24,
                                   "source": "docs/performance_detail.md:93, 114, 156, 165"}),
    "transport": dict(item=tr_item, outputs={"Q": _api.Sum((TR_NS,))}, in_axes=(0, 0, None, None), argnum=2,
                      inputs=tr_inputs, ct=tr_ct, loss=tr_loss, n=4_194_304,
                      published={"fwd_ms": 1.77, "grad_ms": 16.3, "jvp_ms": 1.78, "jacfwd_ms": 1.79,
                                 "source": "docs/performance_detail.md:200, 221, 263, 272"}),
    "walk_on_spheres": dict(item=ws_item, outputs={"u": _api.Sum((WS_M,))}, in_axes=(0, 0, 0, None), argnum=3,
                            inputs=ws_inputs, ct=ws_ct, loss=ws_loss, n=4_194_304,
                            published={"fwd_ms": 1.27, "grad_ms": 8.68, "jvp_ms": 1.37, "jacfwd_ms": 1.47,
                                       "source": "docs/performance_detail.md:307, 328, 370, 379"}),
    "ode_ensemble": dict(item=od_item, outputs={"obs": _api.Sum((OD_G,))}, in_axes=(0, 0, 0, None), argnum=3,
                         inputs=od_inputs, ct=od_ct, loss=od_loss, n=1_048_576,
                         published={"fwd_ms": 5.32, "grad_ms": 25.9, "jvp_ms": 3.83, "jacfwd_ms": 4.83,
                                    "source": "docs/performance_detail.md:414, 435, 477, 486"}),
    "barrier": dict(item=ba_item, outputs={"price": _api.Sum((BA_NK,)), "ko": _api.Sum((1,))}, in_axes=(0, None, None),
                    argnum=1, inputs=ba_inputs, ct=ba_ct, loss=ba_loss, n=4_194_304,
                    published={"fwd_ms": 8.16, "grad_ms": 38.3, "jvp_ms": 9.12, "jacfwd_ms": 11.3,
                               "source": "docs/performance_detail.md:684, 705, 747, 756"}),
    "gillespie": dict(item=gi_item, outputs={"hist": _api.Sum((GI_NB,)), "mean": _api.Sum((1,))}, in_axes=(0, 0, None),
                      argnum=None, inputs=gi_inputs, ct=None, loss=None, n=1_048_576,
                      published={"fwd_ms": 30.0, "source": "docs/performance_detail.md:523"}),
    "shower": dict(item=sh_item, outputs={"dep": _api.Sum((SH_NZ,))}, in_axes=(0, None), argnum=1, inputs=sh_inputs,
                   ct=sh_ct, loss=sh_loss, n=262_144, queue=262_144,
                   published={"fwd_ms": 1.66, "grad_ms": 14.9, "source": "docs/performance_detail.md:593, 614"}),
}


def mapped(name, **opts):
    """the problem's tallymap call (uncapped loops, as the reference's benchmark calls)."""
    p = PROBLEMS[name]
    if p.get("queue"):
        opts = dict(opts, spawn=_api.Queue(p["queue"]))
    return _api.vmap(p["item"], outputs=p["outputs"], in_axes=p["in_axes"], **opts)
