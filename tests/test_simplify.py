"""Common-subexpression elimination before emission (backend/simplify.py; CPU only)."""
import numpy as np

import tallymap_amd as tm
from tallymap_amd import _core as C
from tallymap_amd import configs, lax
from tallymap_amd import numpy as jnp
from tallymap_amd._api import build_program
from tallymap_amd.backend import kernel as K, reverse as R, simplify as S


def _prims(eqns):
    return [e.prim for e in eqns]


def test_fused_value_and_grad_post_evaluates_once():
    """value_and_grad's fused C4 program runs POST (atan2, sin, two emits) and then POST's VJP, which re-evaluates
    the same primal values on the same loop results: after CSE each is computed once and every emit stays."""
    n = 1024
    cfg = configs.c4_config(n)
    f = tm.vmap(cfg["item"], outputs=cfg["outputs"], in_axes=cfg["in_axes"], max_steps=cfg["max_steps"])
    prog = f._prepare(configs.c4_inputs(n))[0]
    adj = R.adjoint_program(prog, ((), (0,)))
    q = R.forward_only_program(adj, R.plan(adj), keep=True)
    w = K._split(q.jaxpr)
    before = _prims(q.jaxpr.eqns[w + 1:])
    jx = S.cse(q.jaxpr, w)
    after = _prims(jx.eqns[w + 1:])
    assert before.count("atan2") == 2 and after.count("atan2") == 1
    assert after.count("tallymap_emit") == before.count("tallymap_emit") >= 3
    assert len(after) < len(before)
    # every variable an equation reads is defined before it (or is an invar)
    defined = {v.id for v in jx.invars}
    for e in jx.eqns:
        for v in e.invars:
            assert not isinstance(v, C.Var) or v.id in defined
        defined |= {o.id for o in e.outvars}
    for v in jx.outvars:
        assert not isinstance(v, C.Var) or v.id in defined


def test_scopes_and_effects():
    """PRE and POST are separate scopes (a POST value is never renamed to a PRE one, which would keep it live
    through the loop); repeated emits are effects and all stay; duplicates inside the loop body are removed."""
    def item(t, x, key):
        a = jnp.sin(x * 2.0)
        t = t.add("h", 0, a)
        t = t.add("h", 0, a)

        def body(c):
            k, y = c
            return k + 1, y + jnp.cos(y) * jnp.cos(y)
        k, y = lax.while_loop(lambda c: c[0] < 3, body, (0, x))
        b = jnp.sin(x * 2.0)
        return t.add("h", 1, b + y), k
    p = build_program(item, {"h": tm.Sum((2,))}, (0, 0), [C.AVal((), np.float32), C.AVal((2,), np.uint32)], [],
                      None)[0]
    w = K._split(p.jaxpr)
    jx = S.cse(p.jaxpr, w)
    pre, post = _prims(jx.eqns[:w]), _prims(jx.eqns[w + 1:])
    assert pre.count("sin") == 1 and post.count("sin") == 1
    assert pre.count("tallymap_emit") == 2 and post.count("tallymap_emit") == 1
    body = jx.eqns[w].params["body_jaxpr"]
    assert _prims(body.eqns).count("cos") == 1
    assert _prims(p.jaxpr.eqns[w].params["body_jaxpr"].eqns).count("cos") == 2


def test_unchanged_program_is_returned_as_is():
    p = build_program(configs.c1_item, configs.C1["outputs"], (0, 0, None),
                      [C.AVal((), np.float32), C.AVal((2,), np.uint32)], [C.AVal((), np.float32)], 100)[0]
    jx = S.cse(p.jaxpr, K._split(p.jaxpr))
    assert len(jx.eqns) <= len(p.jaxpr.eqns)
    assert S.cse(jx, K._split(jx)) is jx
