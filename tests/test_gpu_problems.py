"""The reference's own benchmark problems (tallymap_amd/problems.py; reference benchmarks/vs_jax/problems/) on the
GPU.  Two independent derivations of each loss gradient agree: the replay adjoint (vjp with the loss's cotangent of
the tally) against forward mode (jacfwd of the tally w.r.t. theta, contracted with the same cotangent) within
1e-4 -- the reference's own check of its gradients (tests/reverse.py:280).  The random walk, whose trip counts
are a closed form, is also checked against a numpy float32 emulation of the same walkers: trip counts bitwise,
the histogram within 1e-5 of the emits' float64 sum."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import problems as P
from tallymap_amd import random as R

pytestmark = pytest.mark.gpu
F32 = np.float32


def _np(x):
    return x.cpu().numpy()


@pytest.mark.parametrize("name", [k for k, p in P.PROBLEMS.items() if p["argnum"] is not None])
def test_problem_gradient_equals_forward_mode(name):
    import torch
    p = P.PROBLEMS[name]
    n = 1 << 10 if name in ("ode_ensemble", "shower") else 1 << 12
    print(f"case: problem {name} N={n}", flush=True)
    args, extra = p["inputs"](n)
    f = P.mapped(name)
    res, pull = tm.vjp(f, *args, argnums=p["argnum"])
    tal = {k: v for k, v in res.outputs.items()}
    ct = p["ct"](tal, n, extra)
    g = _np(pull(ct)).astype(np.float64)
    torch.cuda.synchronize()
    assert int(_np(res.stats["n_truncated"])) == 0
    jac, prim = tm.jacfwd(f, argnums=p["argnum"], with_primal=True)(*args)
    for k, v in prim.outputs.items():              # (the primal beside the lanes: the forward call's outputs)
        assert np.allclose(_np(v), _np(res.outputs[k]), rtol=1e-5, atol=1e-6), k
    fwd = np.zeros_like(g)
    for out, c in ct.items():
        J = _np(jac[out][p["argnum"]]).astype(np.float64)           # output.shape + theta.shape
        fwd += np.tensordot(_np(c).astype(np.float64), J, axes=(list(range(c.ndim)), list(range(c.ndim))))
    scale = np.abs(g).max()
    assert scale > 0 and np.all(np.abs(g - fwd) <= 1e-4 * scale), (g, fwd)


def test_random_walk_against_emulation():
    n = 1 << 14
    print(f"case: problem random_walk emulation N={n}", flush=True)
    (keys, decay, th), _ = P.rw_inputs(n)
    res = P.mapped("random_walk")(keys, decay, th)
    k_got, hist = _np(res.per_item), _np(res.outputs["hist"]).astype(np.float64)
    # numpy float32 emulation, all walkers in lockstep
    w = np.ones(n, F32)
    k = np.zeros(n, np.int32)
    acc = np.zeros(P.RW_NB, np.float64)
    alive = w > F32(P.RW_WMIN)
    step = 0
    while alive.any():
        idx = np.nonzero(alive)[0]
        u = R._host_uniform(R._host_fold_in(keys[idx], np.full(len(idx), step, np.uint32)), 0.0, 1.0)
        b = (u * F32(P.RW_NB)).astype(np.int32)
        wa = w[idx]
        v = ((wa * th[0] + th[1] * u) + (th[2] * wa) * wa).astype(F32)
        np.add.at(acc, b, v.astype(np.float64))
        w[idx] = (wa * decay[idx]).astype(F32)
        k[idx] += 1
        step += 1
        alive = w > F32(P.RW_WMIN)
    assert np.array_equal(k_got, k)
    assert np.all(np.abs(hist - acc) <= 1e-5 * np.abs(acc))
    # the reference's closed form of the trip count, ceil(log(0.01) / log(decay)), holds up to float32 rounding
    closed = np.ceil(np.log(0.01) / np.log(decay.astype(np.float64)))
    assert np.mean(k == closed) > 0.999


def test_problems_run_at_small_n():
    """every problem (the forward-only Gillespie one included) runs untruncated with finite outputs; every Gillespie
    realisation lands in one histogram bin; the shower spawns and drops no child."""
    for name, p in P.PROBLEMS.items():
        n = 1 << 10
        print(f"case: problem {name} forward N={n}", flush=True)
        args, _ = p["inputs"](n)
        r = P.mapped(name)(*args)
        assert int(_np(r.stats["n_truncated"])) == 0
        for k, v in r.outputs.items():
            assert np.all(np.isfinite(_np(v))), (name, k)
        if name == "gillespie":
            assert float(_np(r.outputs["hist"]).sum()) == n
        if name == "shower":
            assert int(_np(r.stats["spawned"])) > 0 and int(_np(r.stats["children_dropped"])) == 0
