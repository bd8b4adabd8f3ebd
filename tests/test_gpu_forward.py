"""Forward parity on the GPU: the HIP path (tm.vmap -> libtallymap_rocm.so tm_launch -> gfx950 kernel) against the
oracle on the same seeded inputs.  Integer per-item results and stats bit-exact; f32 tallies within 1e-5 relative of
the oracle's float64 re-summation."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _sync():
    import torch
    torch.cuda.synchronize()


def _np(x):
    return x.cpu().numpy()


def _close(got, want64, rtol=RTOL):
    got = np.asarray(got, np.float64)
    scale = np.max(np.abs(want64)) if want64.size else 0.0
    ok = np.abs(got - want64) <= rtol * np.abs(want64) + 1e-6 * rtol * scale
    return bool(np.all(ok)), float(np.max(np.abs(got - want64) / np.maximum(np.abs(want64), 1e-30)))


def _mapped(cfg, **opts):
    return tm.vmap(cfg["item"], outputs=cfg["outputs"], in_axes=cfg["in_axes"], max_steps=cfg["max_steps"], **opts)


def test_c1_quickstart_parity(oracle):
    print("case: C1 N=10000 full config", flush=True)
    xs, keys, theta = configs.c1_inputs()
    res = _mapped(configs.C1)(xs, keys, theta)
    _sync()
    ref = oracle.c1_fwd(xs, keys, theta, max_steps=100)
    assert np.array_equal(_np(res.per_item), ref.per_item)
    assert np.array_equal(_np(res.truncated), ref.trunc)
    ok, err = _close(_np(res.outputs["hist"]), ref.tallies64["hist"])
    assert ok, err
    assert int(_np(res.stats["dropped_emits"])) == int(ref.stats[4])
    assert int(_np(res.stats["n_truncated"])) == int(ref.trunc.sum()) == 0


def test_c1_truncation_poisons_float_tallies(oracle):
    print("case: C1 N=10000 max_steps=3", flush=True)
    xs, keys, theta = configs.c1_inputs()
    cfg = dict(configs.C1, max_steps=3)
    res = _mapped(cfg)(xs, keys, theta)
    _sync()
    ref = oracle.c1_fwd(xs, keys, theta, max_steps=3)
    assert np.array_equal(_np(res.per_item), ref.per_item)
    assert np.array_equal(_np(res.truncated), ref.trunc)
    assert int(_np(res.stats["n_truncated"])) == int(ref.trunc.sum()) > 0
    assert np.all(np.isnan(_np(res.outputs["hist"])))


@pytest.mark.parametrize("opts", [dict(schedule="item"), dict(block=64), dict(refill=8), dict(post_batch=64),
                                  dict(post_batch=0)])
def test_c1_schedule_and_launch_shape_invariance(oracle, opts):
    """per-item results do not depend on the schedule, block size, refill threshold or POST deferral
    (post_batch=64: every finished item waits for a shared POST pass; 0: none does) (reference
    docs/float_semantics.md:11-13, tests/invariants.py:290)."""
    print(f"case: C1 N=10000 {opts}", flush=True)
    xs, keys, theta = configs.c1_inputs()
    base = _mapped(configs.C1)(xs, keys, theta)
    res = _mapped(configs.C1, **opts)(xs, keys, theta)
    _sync()
    assert np.array_equal(_np(res.per_item), _np(base.per_item))
    ref = oracle.c1_fwd(xs, keys, theta)
    assert _close(_np(res.outputs["hist"]), ref.tallies64["hist"])[0]


def test_c1_edge_sizes(oracle):
    """N = 1, a partial wave, a partial block, one more than a block."""
    xs, keys, theta = configs.c1_inputs(1000)
    f = _mapped(configs.C1)
    for n in (1, 37, 64, 255, 257, 1000):
        print(f"case: C1 N={n}", flush=True)
        res = f(xs[:n], keys[:n], theta)
        _sync()
        ref = oracle.c1_fwd(xs[:n], keys[:n], theta)
        assert np.array_equal(_np(res.per_item), ref.per_item)
        assert _close(_np(res.outputs["hist"]), ref.tallies64["hist"])[0]


def test_dropped_emits_counted(oracle):
    """C1 with x up to 1.5: int32(x * 16) reaches 16..23, which are dropped and counted."""
    print("case: C1 out-of-range bins", flush=True)
    xs, keys, theta = configs.c1_inputs(4096)
    xs = np.linspace(0.5, 1.5, 4096).astype(np.float32)
    res = _mapped(configs.C1)(xs, keys, theta)
    _sync()
    ref = oracle.c1_fwd(xs, keys, theta)
    assert int(ref.stats[4]) > 0
    assert int(_np(res.stats["dropped_emits"])) == int(ref.stats[4])
    assert np.array_equal(_np(res.per_item), ref.per_item)


def test_c2_random_walk_parity(oracle):
    print("case: C2 N=65536", flush=True)
    x0, keys, drift = configs.c2_inputs(65_536)
    res = _mapped(configs.C2)(x0, keys, drift)
    _sync()
    ref = oracle.c2_fwd(x0, keys, drift)
    assert np.array_equal(_np(res.per_item), ref.per_item)
    assert not _np(res.truncated).any()
    for n in ("occ", "wall"):
        ok, err = _close(_np(res.outputs[n]), ref.tallies64[n])
        assert ok, (n, err)
    assert int(_np(res.stats["dropped_emits"])) == int(ref.stats[4])


def test_c2_full_size_parity(oracle):
    """N = 4,194,304 (the benchmark size): every item's trip count bit-exact against the oracle, the tallies within
    tolerance; over all items, one occupancy emit per step (kept or dropped) and one wall emit per item."""
    print("case: C2 N=4194304", flush=True)
    x0, keys, drift = configs.c2_inputs()
    res = _mapped(configs.C2)(x0, keys, drift)
    _sync()
    k = _np(res.per_item).astype(np.int64)
    ref = oracle.c2_fwd(x0, keys, drift)
    assert np.array_equal(k, ref.per_item)
    for n in ("occ", "wall"):
        ok, err = _close(_np(res.outputs[n]), ref.tallies64[n])
        assert ok, (n, err)
    occ = _np(res.outputs["occ"]).astype(np.float64)
    wall = _np(res.outputs["wall"]).astype(np.float64)
    total = float(k.sum())
    dropped = float(_np(res.stats["dropped_emits"]))
    assert int(dropped) == int(ref.stats[4])
    assert abs(occ.sum() + dropped - total) <= RTOL * total
    assert abs(wall.sum() - x0.size) <= RTOL * x0.size
    assert int(_np(res.stats["n_truncated"])) == 0


def test_c1_many_chunks_per_wave(oracle):
    """N = 2^20: every wave claims many 64-item chunks, so lanes are still walking earlier items when the wave
    claims and stages the next chunk; every item's trip count bit-exact against the oracle."""
    print("case: C1 N=1048576", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 20)
    res = _mapped(configs.C1)(xs, keys, theta)
    _sync()
    ref = oracle.c1_fwd(xs, keys, theta)
    assert np.array_equal(_np(res.per_item), ref.per_item)
    ok, err = _close(_np(res.outputs["hist"]), ref.tallies64["hist"])
    assert ok, err
