"""Records outputs on the GPU (tm.Records + t.append, reference _api.py:101-140, _tally.py:302-364, _records.py):
one pass (a raw slot per append from one atomic counter), then the canonical layout -- record k of item i at
offset[i] + k -- against a numpy emulation of the same walker (the host threefry of tallymap_amd.random, pinned by
the oracle tests) record for record, bitwise; overflow, empty outputs, several outputs, jvp tangents."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs, lax
from tallymap_amd import numpy as jnp
from tallymap_amd import random as R

pytestmark = pytest.mark.gpu
f32 = np.float32


def _sync():
    import torch
    torch.cuda.synchronize()


def _np(x):
    return x.cpu().numpy()


def _walker(t, x, key, theta):
    """the quickstart walker; every step with bin < 8 appends (bin, theta (1 - x)); one more record per item at the
    end (its step count and final x) into a second output."""
    def cond(c):
        return c[1] > 0.05

    def body(c):
        k, x, t = c
        u = R.uniform(R.fold_in(key, k))
        b = (x * 16.0).astype(jnp.int32)
        t = t.append("steps", {"bin": b, "w": theta * (1.0 - x)}, when=b < 8)
        return k + 1, x * (0.5 + 0.5 * u), t
    k, x, t = lax.while_loop(cond, body, (0, x, t))
    t = t.append("ends", {"k": k, "x": x})
    t = t.add("hist", jnp.clip((x * 40.0).astype(jnp.int32), 0, 1), 1.0)
    return t, k


def _emulate(xs, keys, theta, M=100):
    """numpy float32 emulation, all items in lockstep: (steps records (item, ordinal, bin, w), ends (k, x))."""
    n = len(xs)
    x = xs.astype(f32).copy()
    ks = np.zeros(n, np.int32)
    alive = x > f32(0.05)
    items, ords, bins, ws = [], [], [], []
    nord = np.zeros(n, np.int64)
    step = 0
    while alive.any() and step < M:
        idx = np.nonzero(alive)[0]
        xa = x[idx]
        u = R._host_uniform(R._host_fold_in(keys[idx], np.full(len(idx), step, np.uint32)), 0.0, 1.0)
        b = (xa * f32(16.0)).astype(np.int32)
        w = (f32(theta) * (f32(1.0) - xa)).astype(f32)
        app = b < 8
        items.append(idx[app])
        ords.append(nord[idx[app]].copy())
        nord[idx[app]] += 1
        bins.append(b[app])
        ws.append(w[app])
        x[idx] = (xa * (f32(0.5) + f32(0.5) * u)).astype(f32)
        ks[idx] += 1
        step += 1
        alive = alive & (x > f32(0.05))
    items, ords = np.concatenate(items), np.concatenate(ords)
    order = np.lexsort((ords, items))
    return (np.concatenate(bins)[order], np.concatenate(ws)[order], items[order]), (ks, x)


def _outputs(cap_steps, cap_ends):
    return {"steps": tm.Records({"bin": np.int32, "w": np.float32}, capacity=cap_steps),
            "ends": tm.Records({"k": np.int32, "x": np.float32}, capacity=cap_ends),
            "hist": tm.Sum((2,))}


def _bits(a):
    return np.asarray(a).view(np.uint32)


@pytest.mark.parametrize("opts", [dict(), dict(schedule="item"), dict(block=64), dict(refill=8),
                                  dict(post_batch=64)], ids=["step", "item", "block64", "refill8", "postbatch"])
def test_records_canonical_layout_bitwise(opts):
    print(f"case: records walker N=65536 {opts}", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 16)
    (bins, ws, items), (ks, xfin) = _emulate(xs, keys, theta)
    n_rec = len(bins)
    f = tm.vmap(_walker, outputs=_outputs(1 << 20, 1 << 17), in_axes=(0, 0, None), max_steps=100, **opts)
    res = f(xs, keys, theta)
    _sync()
    st, en = res.outputs["steps"], res.outputs["ends"]
    assert int(_np(res.stats["appended"]["steps"])) == n_rec
    assert int(_np(res.stats["records_dropped"]["steps"])) == 0
    assert np.array_equal(_np(st["bin"])[:n_rec], bins)
    assert np.array_equal(_bits(_np(st["w"])[:n_rec]), _bits(ws))
    assert not _np(st["bin"])[n_rec:].any() and not _np(st["w"])[n_rec:].any()
    # one end record per item, in item order
    assert int(_np(res.stats["appended"]["ends"])) == len(xs)
    assert np.array_equal(_np(en["k"])[:len(xs)], ks)
    assert np.array_equal(_bits(_np(en["x"])[:len(xs)]), _bits(xfin))
    assert np.array_equal(_np(res.per_item), ks)
    assert float(_np(res.outputs["hist"]).sum()) == len(xs)


def test_records_overflow_poisons():
    """more records than the capacity: every float output NaN (records and sums), every integer field -1, the exact
    number appended and the number dropped reported."""
    print("case: records overflow", flush=True)
    xs, keys, theta = configs.c1_inputs(4096)
    (bins, _, _), _ = _emulate(xs, keys, theta)
    f = tm.vmap(_walker, outputs=_outputs(1000, 1 << 13), in_axes=(0, 0, None), max_steps=100)
    res = f(xs, keys, theta)
    _sync()
    st = res.outputs["steps"]
    assert int(_np(res.stats["appended"]["steps"])) == len(bins) > 1000
    assert int(_np(res.stats["records_dropped"]["steps"])) == len(bins) - 1000
    assert (_np(st["bin"]) == -1).all() and np.isnan(_np(st["w"])).all()
    assert np.isnan(_np(res.outputs["hist"])).all()
    assert np.isnan(_np(res.outputs["ends"]["x"])).all()          # (every float output of the call)
    assert (_np(res.outputs["ends"]["k"]) == -1).all()              # (and every integer record field)
    assert int(_np(res.stats["appended"]["ends"])) == 4096


def test_records_empty_and_when_false():
    print("case: records none appended", flush=True)

    def item(t, x):
        t = t.append("r", {"v": x}, when=x > 2.0)
        return t.append("r", {"v": x}, when=False)
    x = np.linspace(0, 1, 5000).astype(f32)
    res = tm.vmap(item, outputs={"r": tm.Records({"v": np.float32}, capacity=64)}, in_axes=(0,))(x)
    _sync()
    assert int(_np(res.stats["appended"]["r"])) == 0
    assert not _np(res.outputs["r"]["v"]).any()


def test_records_jvp_tangents_at_the_same_slots():
    """d w / d theta = 1 - x: the tangent records sit at the primal's slots and equal w / 2 bitwise (theta = 2)."""
    print("case: records jvp", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    f = tm.vmap(_walker, outputs=_outputs(1 << 18, 1 << 15), in_axes=(0, 0, None), max_steps=100)
    res, tan = tm.jvp(f, (xs, keys, theta), (None, None, f32(1.0)))
    _sync()
    n = int(_np(res.stats["appended"]["steps"]))
    w, wt = _np(res.outputs["steps"]["w"]), _np(tan.outputs["steps"]["w"])
    assert n > 0 and np.array_equal(_bits(wt[:n]), _bits(w[:n] / f32(2.0))) and not wt[n:].any()
    assert not _np(tan.outputs["ends"]["x"]).any()             # (x does not depend on theta)
    ref = f(xs, keys, theta)
    _sync()
    assert np.array_equal(_np(ref.outputs["steps"]["bin"]), _np(res.outputs["steps"]["bin"]))


def test_records_reverse_mode_theta_closed_form():
    """reverse mode through Records (the fill twin): d <ct, steps.w> / d theta = sum over records of ct[slot]
    (1 - x) = sum ct[slot] w[slot] / theta (theta = 2: w / theta is exact), against float64 on the forward's own
    records, within 1e-5; a Sum cotangent adds its own term (the histogram does not depend on theta: 0)."""
    print("case: records vjp theta", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    f = tm.vmap(_walker, outputs=_outputs(1 << 18, 1 << 15), in_axes=(0, 0, None), max_steps=100)
    res, pull = tm.vjp(f, xs, keys, theta, argnums=2)
    ct = np.random.default_rng(9).uniform(0.5, 1.5, 1 << 18).astype(f32)
    g = float(_np(pull({"steps": {"w": ct}, "hist": 1.0})))
    n = int(_np(res.stats["appended"]["steps"]))
    w = _np(res.outputs["steps"]["w"]).astype(np.float64)
    want = float(np.sum(ct[:n].astype(np.float64) * w[:n]) / float(theta))
    assert n > 0 and abs(g - want) <= 1e-5 * abs(want), (g, want)


def test_records_reverse_mode_xs_against_jvp():
    """the per-item cotangent of xs through the record values (w = theta (1 - x_k), x_k a product of the item's
    draws) dotted with a direction v equals forward mode's <ct, tangent records> (two derivations), within 1e-4."""
    print("case: records vjp xs", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    f = tm.vmap(_walker, outputs=_outputs(1 << 18, 1 << 15), in_axes=(0, 0, None), max_steps=100)
    ct = np.random.default_rng(10).uniform(0.5, 1.5, 1 << 18).astype(f32)
    cte = np.random.default_rng(11).uniform(0.5, 1.5, 1 << 15).astype(f32)
    _, pull = tm.vjp(f, xs, keys, theta, argnums=0)
    gx = _np(pull({"steps": {"w": ct}, "ends": {"x": cte}})).astype(np.float64)
    v = np.random.default_rng(12).standard_normal(xs.shape[0]).astype(f32)
    _, tan = tm.jvp(f, (xs, keys, theta), (v, None, None))
    _sync()
    jv = float(np.dot(_np(tan.outputs["steps"]["w"]).astype(np.float64), ct)
               + np.dot(_np(tan.outputs["ends"]["x"]).astype(np.float64), cte))
    assert abs(float(np.dot(gx, v)) - jv) <= 1e-4 * abs(jv), (float(np.dot(gx, v)), jv)


def test_records_reverse_mode_overflow_is_nan():
    print("case: records vjp overflow", flush=True)
    xs, keys, theta = configs.c1_inputs(4096)
    f = tm.vmap(_walker, outputs=_outputs(1000, 1 << 13), in_axes=(0, 0, None), max_steps=100)
    _, pull = tm.vjp(f, xs, keys, theta, argnums=2)
    assert np.isnan(_np(pull({"steps": {"w": 1.0}}))).all()


def test_records_without_capacity_sized_by_count_pass():
    """Records without a capacity: a count pass sizes each output to the next power of two at or above its record
    count (reference _api.py:838-852); the records equal the explicit-capacity call's bitwise, and reverse mode
    sizes the same way."""
    print("case: records without capacity", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    outs = {"steps": tm.Records({"bin": np.int32, "w": np.float32}),
            "ends": tm.Records({"k": np.int32, "x": np.float32}), "hist": tm.Sum((2,))}
    f = tm.vmap(_walker, outputs=outs, in_axes=(0, 0, None), max_steps=100)
    res = f(xs, keys, theta)
    ref = tm.vmap(_walker, outputs=_outputs(1 << 18, 1 << 15), in_axes=(0, 0, None), max_steps=100)(xs, keys, theta)
    _sync()
    n = int(_np(ref.stats["appended"]["steps"]))
    cap = 1 << (n - 1).bit_length()
    assert _np(res.outputs["steps"]["w"]).shape == (cap,) and _np(res.outputs["ends"]["x"]).shape == (1 << 14,)
    assert np.array_equal(_np(res.outputs["steps"]["w"])[:n].view(np.uint32),
                          _np(ref.outputs["steps"]["w"])[:n].view(np.uint32))
    assert int(_np(res.stats["records_dropped"]["steps"])) == 0
    g = float(_np(tm.grad(f, weights={"steps": {"w": 1.0}}, argnums=2)(xs, keys, theta)))
    w = _np(ref.outputs["steps"]["w"]).astype(np.float64)[:n]
    assert abs(g - w.sum() / 2.0) <= 1e-5 * w.sum() / 2.0


@pytest.mark.parametrize("n", [0, 5, 9_999, 1 << 14])
def test_n_active_runs_only_the_first_items(n):
    """n_active = n: the call over 2^14 items equals the call over the first n items (exact Sum bitwise, Records
    bitwise, per-item results), and the skipped items' per-item results are zero (reference edge.py:617-627)."""
    print(f"case: n_active={n}", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    outs = dict(_outputs(1 << 18, 1 << 15), hist=tm.Sum((2,), fixed_point=True))
    f = tm.vmap(_walker, outputs=outs, in_axes=(0, 0, None), max_steps=100)
    # the allocator's cached small blocks hold all-ones bytes, so a pass that read scratch the launch never wrote
    # (the hole list when no item runs) would see garbage rather than the zeros of fresh memory
    import torch
    junk = [torch.full((1 << 18,), -1, dtype=torch.int32, device="cuda") for _ in range(64)]
    del junk
    a = f(xs, keys, theta, n_active=n)
    _sync()
    k = _np(a.per_item)
    assert not k[n:].any() and not _np(a.truncated)[n:].any()
    if n == 0:
        assert int(_np(a.stats["appended"]["steps"])) == 0 and not _np(a.outputs["hist"]).any()
        return
    b = f(xs[:n], keys[:n], theta)
    _sync()
    m = int(_np(b.stats["appended"]["steps"]))
    assert int(_np(a.stats["appended"]["steps"])) == m and np.array_equal(k[:n], _np(b.per_item))
    assert np.array_equal(_np(a.outputs["hist"]).view(np.uint32), _np(b.outputs["hist"]).view(np.uint32))
    assert np.array_equal(_np(a.outputs["steps"]["w"]).view(np.uint32), _np(b.outputs["steps"]["w"]).view(np.uint32))


def test_records_appended_from_both_branches_of_a_cond():
    """appends from both branches of a cond inside a loop (lanes of one wave in different branches, which run one
    after the other): every record lands once in its item's canonical place, against the numpy enumeration."""
    print("case: records from both cond branches", flush=True)
    n = 6000
    rng = np.random.default_rng(3)
    u = rng.integers(0, 1 << 20, n).astype(np.uint32)
    x = (rng.integers(0, 1 << 12, n) / 64.0).astype(f32)

    def item(t, u, x):
        def body(i, t):
            def even(t):
                return t.append("r", {"a": u * 2 + i, "w": x * 2.0})

            def odd(t):
                return t.append("r", {"a": u + i, "w": x * 0.5}, when=(u & 4) == 0)
            return lax.cond((u + i) % 2 == 0, even, odd, t)
        return lax.fori_loop(0, 3, body, t)
    f = tm.vmap(item, outputs={"r": tm.Records({"a": np.uint32, "w": np.float32}, capacity=1 << 16)},
                in_axes=(0, 0))
    res = f(u, x)
    _sync()
    want_a, want_w = [], []
    for ui, xi in zip(u.tolist(), x.tolist()):
        for i in range(3):
            if (ui + i) % 2 == 0:
                want_a.append((ui * 2 + i) & 0xFFFFFFFF)
                want_w.append(f32(xi) * f32(2.0))
            elif (ui & 4) == 0:
                want_a.append((ui + i) & 0xFFFFFFFF)
                want_w.append(f32(xi) * f32(0.5))
    m = len(want_a)
    assert int(_np(res.stats["appended"]["r"])) == m
    assert np.array_equal(_np(res.outputs["r"]["a"])[:m], np.array(want_a, np.uint32))
    assert np.array_equal(_np(res.outputs["r"]["w"])[:m].view(np.uint32), np.array(want_w, f32).view(np.uint32))


def test_records_without_capacity_under_n_active():
    """a capacity-less Records output under n_active = n is sized by a count pass over the first n items only (the
    reference appends n_active before its count, _api.py:838-852): the output shape and records equal the call over
    the first n items, and the inactive items' records (here ~6x more) neither size it nor raise; reverse mode
    through the same call agrees with the first-n call."""
    print("case: records without capacity, n_active", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 14)
    outs = {"steps": tm.Records({"bin": np.int32, "w": np.float32}),
            "ends": tm.Records({"k": np.int32, "x": np.float32}), "hist": tm.Sum((2,))}
    f = tm.vmap(_walker, outputs=outs, in_axes=(0, 0, None), max_steps=100)
    n = 2300
    a = f(xs, keys, theta, n_active=n)
    b = f(xs[:n], keys[:n], theta)
    _sync()
    for r, fld in (("steps", "w"), ("ends", "x")):
        wa, wb = _np(a.outputs[r][fld]), _np(b.outputs[r][fld])
        assert wa.shape == wb.shape, (r, wa.shape, wb.shape)
        assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
    ga = _np(tm.grad(f, weights={"steps": {"w": 1.0}}, argnums=2)(xs, keys, theta, n_active=n))
    gb = _np(tm.grad(f, weights={"steps": {"w": 1.0}}, argnums=2)(xs[:n], keys[:n], theta))
    _sync()
    assert np.array_equal(np.atleast_1d(ga).view(np.uint32), np.atleast_1d(gb).view(np.uint32))


@pytest.mark.parametrize("n", [0, 1, 257])
def test_small_and_empty_calls(n):
    """N = 0, 1 and one not a multiple of the block (reference edge.py:296-307): Sums, Records and per-item results
    of the right shapes; nothing emitted at N = 0; the same values as a larger call's first n items."""
    print(f"case: N={n}", flush=True)
    xs, keys, theta = configs.c1_inputs(512)
    f = tm.vmap(_walker, outputs=dict(_outputs(1 << 12, 1 << 10), hist=tm.Sum((2,), fixed_point=True)),
                in_axes=(0, 0, None), max_steps=100)
    a = f(xs[:n], keys[:n], theta)
    b = f(xs, keys, theta, n_active=n)
    _sync()
    assert _np(a.per_item).shape == (n,) and _np(a.outputs["hist"]).shape == (2,)
    assert np.array_equal(_np(a.outputs["hist"]).view(np.uint32), _np(b.outputs["hist"]).view(np.uint32))
    assert np.array_equal(_np(a.outputs["steps"]["w"]).view(np.uint32), _np(b.outputs["steps"]["w"]).view(np.uint32))
    assert np.array_equal(_np(a.per_item), _np(b.per_item)[:n])
    if n == 0:
        assert not _np(a.outputs["hist"]).any() and int(_np(a.stats["appended"]["steps"])) == 0


def _scan_switch_item(t, x):
    c, ys = lax.scan(lambda c, v: (c + v, c * 2.0), 0.0, jnp.stack([x, x + 1.0, x + 2.0]))
    n, _ = lax.scan(lambda c, _: (c + 1, None), 0, length=1000)
    s = lax.switch((x * 3.0).astype(jnp.int32), [lambda v: v, lambda v: v * 2.0, lambda v: v * 3.0], x)
    return t.add("h", 0, c + ys[2] + s), (n, s)


def test_scan_and_switch_items():
    """an item with an unrolled scan (ys stacked), a 1000-step scan run as a loop and a switch: per-item results
    and the exact tally against a float32 numpy restatement of the same arithmetic, bitwise."""
    print("case: scan and switch", flush=True)
    x = np.random.default_rng(2).uniform(0, 1, 10_000).astype(f32)
    res = tm.vmap(_scan_switch_item, outputs={"h": tm.Sum((1,), fixed_point=True)}, in_axes=(0,))(x)
    _sync()
    c0 = (f32(0.0) + x).astype(f32)
    c1 = (c0 + (x + f32(1.0))).astype(f32)
    c = (c1 + (x + f32(2.0))).astype(f32)
    ys2 = (c1 * f32(2.0)).astype(f32)
    k = np.clip((x * f32(3.0)).astype(np.int32), 0, 2)
    s = np.choose(k, [x, (x * f32(2.0)).astype(f32), (x * f32(3.0)).astype(f32)]).astype(f32)
    n, sg = res.per_item
    assert (_np(n) == 1000).all() and np.array_equal(_np(sg).view(np.uint32), s.view(np.uint32))
    from oracle import exact as X
    v = ((c + ys2).astype(f32) + s).astype(f32)
    assert _np(res.outputs["h"])[0].view(np.uint32) == X.exact_sum(v)[0].view(np.uint32)


def _table_item(t, x, k, tab, small):
    """the reference's basic edge item shape (edge.py:110-118): a bin picked by a traced index, a broadcast table
    read at it (64 entries: read in place) and a small one (4 entries: in registers), negative and large indices
    clamped as jnp does."""
    i = (x * 80.0).astype(jnp.int32) - 8          # in [-8, 72): negatives count from the end, then clamped
    w = tab[i] * small[k % 4] + small[k - 6]
    return t.add("Q", jnp.clip(i, 0, 63), w * x), w


def test_dynamic_index_forward_jvp_grad():
    """tab[i] with a traced i: values against numpy's take with jnp's normalisation and clamping, bitwise
    (exact tally); jvp w.r.t. the table against the closed form d w / d tab[j]; grad w.r.t. the small table against
    forward mode."""
    print("case: dynamic index", flush=True)
    rng = np.random.default_rng(21)
    n = 20_000
    x = rng.uniform(0, 1, n).astype(f32)
    k = rng.integers(0, 12, n).astype(np.int32)
    tab = rng.uniform(0.5, 1.5, 64).astype(f32)
    small = np.array([1.0, 2.0, 0.5, -1.0], f32)
    f = tm.vmap(_table_item, outputs={"Q": tm.Sum((64,), fixed_point=True)}, in_axes=(0, 0, None, None))
    res = f(x, k, tab, small)
    _sync()

    def take(a, j):
        j = np.where(j < 0, j + len(a), j)
        return a[np.clip(j, 0, len(a) - 1)]
    i = (x * f32(80.0)).astype(np.int32) - 8
    w = (take(tab, i) * take(small, k % 4) + take(small, k - 6)).astype(f32)
    assert np.array_equal(_np(res.per_item).view(np.uint32), w.view(np.uint32))
    from oracle import exact as X
    v = (w * x).astype(f32)
    b = np.clip(i, 0, 63)
    want = np.array([X.exact_sum(v[b == j])[0] if (b == j).any() else f32(0) for j in range(64)], f32)
    assert np.array_equal(_np(res.outputs["Q"]).view(np.uint32), want.view(np.uint32))
    dt = rng.standard_normal(64).astype(f32)
    _, tan = tm.jvp(f, (x, k, tab, small), (None, None, dt, None))
    _sync()
    tw = take(dt, i).astype(np.float64) * take(small, k % 4)
    assert np.allclose(_np(tan.per_item).astype(np.float64), tw, rtol=1e-6, atol=1e-7)
    ct = rng.uniform(0.5, 1.5, 64).astype(f32)
    g = _np(tm.grad(f, weights={"Q": ct}, argnums=3)(x, k, tab, small)).astype(np.float64)
    ds = np.eye(4, dtype=f32)
    J = [float(np.dot(_np(tm.jvp(f, (x, k, tab, small), (None, None, None, ds[j]))[1].outputs["Q"]).astype(
        np.float64), ct)) for j in range(4)]
    assert np.allclose(g, J, rtol=1e-4), (g, J)
