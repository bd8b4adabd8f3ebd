"""The benchmark item programs and their synthetic inputs.

Each config gives: the item function (written against tallymap_amd's jax-shaped API, as a reference user writes
it against JAX), its `vmap` outputs / in_axes / max_steps, a seeded input generator, and the cotangent of the
gradient the config asks for.  Inputs are generated on the host with tallymap_amd.random (numpy threefry), so the
GPU and the oracle see the same arrays.

C1  the reference's quickstart walker (reference examples/quickstart.py:19-30).
C2  1-D random walk with absorbing walls: per step one occupancy emit at int32(x * 128), then
    x += drift + 0.02 * normal(fold_in(key, k)); after the loop one emit into the wall histogram.
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


CONFIGS = {"c1": C1, "c2": C2}
