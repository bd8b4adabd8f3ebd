"""The tracer, the tally rules and the cap (CPU only)."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import _core as C
from tallymap_amd import configs, lax, random
from tallymap_amd import numpy as jnp
from tallymap_amd._api import build_program


def _prog(item, outputs, pav, bav, axes, max_steps=None):
    return build_program(item, outputs, axes, [C.AVal(*a) for a in pav], [C.AVal(*a) for a in bav], max_steps)[0]


def test_quickstart_traces_to_one_capped_loop():
    p = _prog(configs.c1_item, configs.C1["outputs"], [((), np.float32), ((2,), np.uint32)], [((), np.float32)],
              (0, 0, None), 100)
    prims = [e.prim for e in p.jaxpr.eqns]
    assert prims.count("while") == 1
    w = p.jaxpr.eqns[prims.index("while")]
    body = [e.prim for e in w.params["body_jaxpr"].eqns]
    assert body.count("threefry2x32") == 2 and "tallymap_emit" in body
    assert p.trunc == 1                                # per-item results: [k, truncated]
    assert [v.aval.dtype for v in p.jaxpr.outvars] == [np.float32, np.int32, np.bool_]


def test_weak_types_follow_jax():
    def item(t, x, key):
        y = x * 3            # f32 * weak int -> f32
        z = (x > 0.5)        # bool
        i = (y * 2).astype(jnp.int32) + 1
        return t.add("h", i, 1.0), i
    p = _prog(item, {"h": tm.Sum((4,))}, [((), np.float32), ((2,), np.uint32)], [], (0, 0))
    assert p.jaxpr.outvars[1].aval.dtype == np.int32
    assert all(e.outvars[0].aval.dtype in (np.float32, np.int32, np.bool_) for e in p.jaxpr.eqns)


def test_python_scalars_take_the_operand_dtype_at_full_precision():
    """a Python float meeting a float64 operand (or a Python int meeting an int64 one) becomes a constant of that
    dtype directly, not through float32 / int32 (JAX's weak typing)."""
    def item(t, x, n):
        t = t.add("f", 0, x * 4e18 + 0.1)
        return t.add("i", 0, n * 4_000_000_000_000_000_000)
    p = _prog(item, {"f": tm.Sum((1,), np.float64), "i": tm.Sum((1,), np.int64)},
              [((), np.float64), ((), np.int64)], [], (0, 0))
    lits = [v.val for e in p.jaxpr.eqns for v in e.invars if isinstance(v, C.Lit) and v.aval.shape == ()]
    assert any(x.dtype == np.float64 and x == 4e18 for x in lits)
    assert any(x.dtype == np.float64 and x == 0.1 for x in lits)
    assert any(x.dtype == np.int64 and x == 4_000_000_000_000_000_000 for x in lits)


def test_tally_read_fork_drop_raise():
    def forked(t, x):
        t1 = t.add("h", 0, x)
        t.add("h", 1, x)
        return t1

    def dropped(t, x):
        t.add("h", 0, x)
        return t

    with pytest.raises(tm.TallyError):
        _prog(forked, {"h": tm.Sum((2,))}, [((), np.float32)], [], (0,))
    with pytest.raises(tm.TallyError):
        _prog(dropped, {"h": tm.Sum((2,))}, [((), np.float32)], [], (0,))


def test_tuple_index_flattening():
    def item(t, i, j):
        return t.add("g", (i, j), 1.0)
    p = _prog(item, {"g": tm.Sum((3, 4))}, [((), np.int32), ((), np.int32)], [], (0, 0))
    prims = [e.prim for e in p.jaxpr.eqns]
    assert "select_n" in prims and "tallymap_emit" in prims


def test_cond_and_fori_trace():
    def item(t, x):
        y = lax.cond(x > 0.5, lambda a: a * 2.0, lambda a: a - 1.0, x)
        s = lax.fori_loop(0, 3, lambda i, a: a + y, 0.0)
        return t.add("h", 0, s)
    p = _prog(item, {"h": tm.Sum((1,))}, [((), np.float32)], [], (0,))
    assert [e.prim for e in p.jaxpr.eqns].count("cond") == 1


def test_uniform_normal_avals():
    def item(t, key):
        u = random.uniform(key, minval=0.2, maxval=0.8)
        n = random.normal(random.fold_in(key, 3))
        return t.add("h", 0, u + n)
    p = _prog(item, {"h": tm.Sum((1,))}, [((2,), np.uint32)], [], (0,))
    prims = [e.prim for e in p.jaxpr.eqns]
    assert prims.count("threefry2x32") == 3 and "erf_inv" in prims


def test_unknown_option_raises():
    with pytest.raises(ValueError):
        tm.vmap(configs.c1_item, outputs=configs.C1["outputs"], bogus=1)
