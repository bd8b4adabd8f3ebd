"""Forward mode on the GPU (tm.jvp, tm.jacfwd: the fused tangent kernel, reference _api.py:305-345,
_primitive.py:419-436, 693-801) against closed forms, the oracle's forward-mode (dual number) gradients and the
product's own reverse mode (<ct, J t> = <J^T ct, t>); tangent tallies within 1e-4 relative (gradients, BASELINE
north_star), bitwise where the arithmetic fixes the bits (exact tallies, constant emits)."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs
from tallymap_amd import numpy as jnp

pytestmark = pytest.mark.gpu
GTOL = 1e-4


def _sync():
    import torch
    torch.cuda.synchronize()


def _np(x):
    return x.cpu().numpy()


def _mapped(cfg, outputs=None, **opts):
    return tm.vmap(cfg["item"], outputs=outputs or cfg["outputs"], in_axes=cfg["in_axes"],
                   max_steps=cfg["max_steps"], **opts)


def _rel(got, want):
    return abs(float(got) - float(want)) / max(abs(float(want)), 1e-30)


@pytest.mark.parametrize("opts", [dict(), dict(schedule="item")], ids=["step", "item"])
def test_c1_jvp_theta_exact_is_half_the_primal(opts):
    """theta = 2 multiplies every emit: the tangent emit (1 - x) is exactly half the primal's, so with exact
    tallies the tangent histogram is bitwise the primal / 2 (and the primal equals the plain forward's)."""
    print(f"case: C1 jvp theta exact {opts}", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 16)
    f = _mapped(configs.C1, {"hist": tm.Sum((16,), fixed_point=True)}, **opts)
    res, tan = tm.jvp(f, (xs, keys, theta), (None, None, np.float32(1.0)))
    ref = f(xs, keys, theta)
    _sync()
    h, ht = _np(res.outputs["hist"]), _np(tan.outputs["hist"])
    assert np.array_equal(h.view(np.uint32), _np(ref.outputs["hist"]).view(np.uint32))
    assert np.array_equal(ht.view(np.uint32), (h / np.float32(2)).view(np.uint32))
    assert np.array_equal(_np(res.per_item), _np(ref.per_item))


def test_c1_jvp_xs_against_oracle_and_vjp(oracle):
    """a random per-item tangent of xs: <ct, hist'> equals the oracle's sum_i v_i d(ct.hist)/d x_i and the product's
    reverse mode <vjp(ct), v>."""
    print("case: C1 jvp xs", flush=True)
    xs, keys, theta = configs.c1_inputs()
    ct = np.linspace(0.5, 2.0, 16).astype(np.float32)
    v = np.random.default_rng(3).standard_normal(xs.shape[0]).astype(np.float32)
    f = _mapped(configs.C1)
    _, tan = tm.jvp(f, (xs, keys, theta), (v, None, None))
    _sync()
    got = float(np.dot(_np(tan.outputs["hist"]).astype(np.float64), ct))
    _, want_x, ntr = oracle.c1_grad(xs, keys, theta, ct, per_item=True)
    want = float(np.dot(want_x.astype(np.float64), v))
    assert ntr == 0 and _rel(got, want) <= GTOL, (got, want)
    _, pull = tm.vjp(f, xs, keys, theta, argnums=0)
    gx = _np(pull({"hist": ct}))
    assert _rel(got, float(np.dot(gx.astype(np.float64), v))) <= GTOL


def test_c2_jvp_is_exactly_zero():
    """every C2 emit is the constant 1.0: the tangents w.r.t. drift and x0 are exactly zero."""
    print("case: C2 jvp N=65536", flush=True)
    x0, keys, drift = configs.c2_inputs(65_536)
    res, tan = tm.jvp(_mapped(configs.C2), (x0, keys, drift), (np.ones_like(x0), None, np.float32(1.0)))
    _sync()
    assert not _np(tan.outputs["occ"]).any() and not _np(tan.outputs["wall"]).any()
    assert float(_np(res.outputs["wall"]).sum()) == 65_536.0


@pytest.mark.parametrize("n", [65_536, 1_048_576])
def test_c3_jvp_mu_a_against_oracle_and_vjp(oracle, n):
    """d <ct, absorbed> / d mu_a through the loop-carried weight: forward mode vs the oracle's dual numbers and vs
    the replay adjoint."""
    print(f"case: C3 jvp mu_a N={n}", flush=True)
    keys, mu_a = configs.c3_inputs(n)
    ct = np.random.default_rng(5).uniform(0.5, 1.5, (64, 64)).astype(np.float32)
    f = _mapped(configs.C3)
    res, tan = tm.jvp(f, (keys, mu_a), (None, np.float32(1.0)))
    _sync()
    got = float(np.sum(_np(tan.outputs["absorbed"]).astype(np.float64) * ct))
    want, ntr = oracle.c3_grad(keys, mu_a, ct)
    assert ntr == 0 and _rel(got, want) <= GTOL, (got, float(want))
    _, pull = tm.vjp(f, keys, mu_a, argnums=1)
    assert _rel(got, float(_np(pull({"absorbed": ct})))) <= GTOL


def test_c4_jvp_amplitude_closed_form(oracle):
    """a multiplies every score: the tangent tallies are the primal tallies / a (within f32 rounding of a * s)."""
    print("case: C4 jvp a", flush=True)
    n = 65_536
    p0, keys, ids, a = configs.c4_inputs(n)
    res, tan = tm.jvp(_mapped(configs.c4_config(n)), (p0, keys, ids, a), (None, None, None, np.float32(1.0)))
    _sync()
    w, wt = _np(res.outputs["walker"]).astype(np.float64), _np(tan.outputs["walker"]).astype(np.float64)
    assert np.max(np.abs(wt - w / float(a))) <= 1e-6 * np.max(np.abs(w / float(a)))
    g, gt = _np(res.outputs["grid"]).astype(np.float64), _np(tan.outputs["grid"]).astype(np.float64)
    assert np.max(np.abs(gt - g / float(a))) <= 1e-5 * np.max(np.abs(g / float(a)))


@pytest.mark.parametrize("n", [16_384, 262_144])
def test_c5_jvp_amplitude_against_oracle(oracle, n):
    """d sum_i E(final_i) / d A in forward mode (tangent state tally, dotted with the energy cotangent) vs the
    oracle's dual-number gradient."""
    print(f"case: C5 jvp A N={n}", flush=True)
    th0, om0, ids, A = configs.c5_inputs(n)
    f = _mapped(configs.c5_config(n))
    res, tan = tm.jvp(f, (th0, om0, ids, A), (None, None, None, np.float32(1.0)))
    _sync()
    ct = configs.c5_energy_ct(_np(res.outputs["state"]))
    got = float(np.sum(_np(tan.outputs["state"]).astype(np.float64) * ct))
    want, ntr = oracle.c5_grad(th0, om0, ids, A, ct)
    assert ntr == 0 and _rel(got, want) <= GTOL, (got, float(want))


def _poly_item(t, x, w):
    b = jnp.clip((x * 8.0).astype(jnp.int32), 0, 7)
    v = w[0] + w[1] * x + w[2] * x * x
    for k in range(3, w.shape[0]):
        v = v + w[k] * tm.lax.sin(x * float(k))
    return t.add("h", b, v)


@pytest.mark.parametrize("m", [5, 20])
def test_jacfwd_dual_lanes_closed_form(m):
    """the Jacobian of 8 bins w.r.t. an m-vector parameter (5: one 5-lane kernel; 20: a 16-lane and a 4-lane
    kernel): d h[b] / d w[k] = sum over the items in bin b of the k-th feature, against float64 numpy; each lane
    equals the single-direction jvp bitwise (exact tallies)."""
    print(f"case: jacfwd m={m}", flush=True)
    x = np.random.default_rng(7).uniform(0, 1, 50_000).astype(np.float32)
    w = np.linspace(0.5, 1.5, m).astype(np.float32)
    f = tm.vmap(_poly_item, outputs={"h": tm.Sum((8,), fixed_point=True)}, in_axes=(0, None))
    J = _np(tm.jacfwd(f, argnums=1)(x, w)["h"][1])
    _sync()
    assert J.shape == (8, m)
    b = np.clip((x * np.float32(8.0)).astype(np.int32), 0, 7)
    x64 = x.astype(np.float64)
    feats = [np.ones_like(x64), x64, x64 * x64] + [np.sin(x64 * k) for k in range(3, m)]
    want = np.stack([np.bincount(b, fk, 8) for fk in feats], axis=1)
    assert np.max(np.abs(J - want) / np.maximum(np.abs(want), 1.0)) <= 1e-5
    for k in (0, m - 1):
        e = np.zeros(m, np.float32)
        e[k] = 1
        _, tan = tm.jvp(f, (x, w), (None, e))
        _sync()
        assert np.array_equal(_np(tan.outputs["h"]).view(np.uint32), J[:, k].astype(np.float32).view(np.uint32))


def test_jvp_truncation_poisons_tangents():
    print("case: C1 jvp max_steps=3", flush=True)
    xs, keys, theta = configs.c1_inputs()
    f = _mapped(dict(configs.C1, max_steps=3))
    res, tan = tm.jvp(f, (xs, keys, theta), (None, None, np.float32(1.0)))
    _sync()
    assert int(_np(res.stats["n_truncated"])) > 0
    assert np.isnan(_np(res.outputs["hist"])).all() and np.isnan(_np(tan.outputs["hist"])).all()


def _cond_loop_item(t, x, a):
    def body(i, c):
        y = tm.lax.cond(c > 0.5, lambda z: z * a, lambda z: z + a, c)
        return y * 0.5
    y = tm.lax.fori_loop(0, 3, body, x)
    return t.add("h", 0, y), y


def test_jvp_through_cond_inside_loop():
    """tangents through a cond inside a loop body: the per-item tangent equals a float32 emulation of the same
    derivative arithmetic bitwise (tangent of c * a: dc * a + c; of c + a: dc + 1; times 0.5)."""
    print("case: jvp through cond in a loop", flush=True)
    x = np.random.default_rng(11).uniform(0, 1.5, 100_000).astype(np.float32)
    a = np.float32(1.3)
    f = tm.vmap(_cond_loop_item, outputs={"h": tm.Sum((1,), fixed_point=True)}, in_axes=(0, None))
    res, tan = tm.jvp(f, (x, a), (None, np.float32(1.0)))
    _sync()
    c, dc = x.copy(), np.zeros_like(x)
    h = np.float32(0.5)
    for _ in range(3):
        big = c > np.float32(0.5)
        c2 = np.where(big, c * a, c + a).astype(np.float32)
        dc2 = np.where(big, dc * a + c, dc + np.float32(1.0)).astype(np.float32)
        c, dc = (c2 * h).astype(np.float32), (dc2 * h).astype(np.float32)
    assert np.array_equal(_np(res.per_item).view(np.uint32), c.view(np.uint32))
    assert np.array_equal(_np(tan.per_item).view(np.uint32), dc.view(np.uint32))
    from oracle import exact as X
    assert _np(tan.outputs["h"])[0].view(np.uint32) == X.exact_sum(dc)[0].view(np.uint32)


def test_jvp_and_jacfwd_under_n_active():
    """n_active = n composes with forward and reverse mode as with the call: tangent and primal tallies equal those
    of the call over the first n items (float32 sums in atomic order: 1e-5 relative), per-item cotangents and the
    exact broadcast cotangent bitwise, and the inactive items' per-item cotangents are zero."""
    print("case: jvp / jacfwd with n_active", flush=True)
    xs, keys, theta = configs.c1_inputs(4096)
    f = _mapped(configs.C1)
    n = 1234
    ra, ta = tm.jvp(f, (xs, keys, theta), (np.ones_like(xs), None, np.float32(1.0)), n_active=n)
    rb, tb = tm.jvp(f, (xs[:n], keys[:n], theta), (np.ones_like(xs[:n]), None, np.float32(1.0)))
    _sync()
    assert np.allclose(_np(ta.outputs["hist"]), _np(tb.outputs["hist"]), rtol=1e-5, atol=0)
    assert np.allclose(_np(ra.outputs["hist"]), _np(rb.outputs["hist"]), rtol=1e-5, atol=0)
    ja = _np(tm.jacfwd(f, argnums=2)(xs, keys, theta, n_active=n)["hist"][2])
    jb = _np(tm.jacfwd(f, argnums=2)(xs[:n], keys[:n], theta)["hist"][2])
    _sync()
    assert np.allclose(ja, jb, rtol=1e-5, atol=0)
    res, pull = tm.vjp(f, xs, keys, theta, argnums=(0, 2), n_active=n)
    gx, gt = pull({"hist": 1.0})
    _, pull_b = tm.vjp(f, xs[:n], keys[:n], theta, argnums=(0, 2))
    gxb, gtb = pull_b({"hist": 1.0})
    _sync()
    assert not _np(gx)[n:].any() and np.array_equal(_np(gx)[:n].view(np.uint32), _np(gxb).view(np.uint32))
    assert np.array_equal(np.atleast_1d(_np(gt)).view(np.uint32), np.atleast_1d(_np(gtb)).view(np.uint32))
