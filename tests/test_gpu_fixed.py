"""Sum(fixed_point=True, scale) of non-float32 dtypes (the scaled fixed-point format) and plain float64 / int64 /
uint64 sums on the GPU.  A fixed-point bin is round(v * scale) summed in an int64 low word with a signed carry word,
so its total is exact and bitwise independent of the schedule; the output is total / scale in the dtype (reference
_api.py:55-84, kernel.py:633-665, 844-869).  Checked bitwise against the oracle's 128-bit totals (C1, C2) and
against numpy integer sums (integer emits, carries past 2^63)."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs

pytestmark = pytest.mark.gpu


def _sync():
    import torch
    torch.cuda.synchronize()


def _np(x):
    return x.cpu().numpy()


def _mapped(cfg, outputs, **opts):
    return tm.vmap(cfg["item"], outputs=outputs, in_axes=cfg["in_axes"], max_steps=cfg["max_steps"], **opts)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("scale", [2.0 ** 32, 16.0, 0.5])
@pytest.mark.parametrize("opts", [dict(), dict(schedule="item"), dict(block=64), dict(refill=8)],
                         ids=["step", "item", "block64", "refill8"])
def test_c1_fixed_point_f64_bitwise(oracle, scale, opts):
    """C1's histogram as float64 fixed point: bitwise the oracle's totals / scale (LDS accumulators)."""
    print(f"case: C1 f64 fixed scale={scale} {opts}", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 16)
    res = _mapped(configs.C1, {"hist": tm.Sum((16,), np.float64, fixed_point=True, scale=scale)}, **opts)(
        xs, keys, theta)
    _sync()
    ref, out, over = oracle.wide_tallies(lambda: oracle.c1_fwd(xs, keys, theta), [(16, scale, np.float64)])
    assert _same(_np(res.outputs["hist"]), out[0][0])
    assert np.array_equal(_np(res.per_item), ref.per_item)
    assert int(_np(res.stats["fixed_point_overflow"])) == over == 0


def test_c1_fixed_point_global_words_bitwise(oracle):
    """a tally too large for LDS (4096 bins x 12 B) keeps its words in global memory: same bits."""
    print("case: C1 f64 fixed 4096 bins (global)", flush=True)
    xs, keys, theta = configs.c1_inputs(1 << 16)
    res = _mapped(configs.C1, {"hist": tm.Sum((4096,), np.float64, fixed_point=True, scale=2.0 ** 20)})(
        xs, keys, theta)
    _sync()
    _, out, _ = oracle.wide_tallies(lambda: oracle.c1_fwd(xs, keys, theta), [(16, 2.0 ** 20, np.float64)])
    h = _np(res.outputs["hist"])
    assert _same(h[:16], out[0][0]) and not h[16:].any()


def test_c1_fixed_point_overflow_poisons_bins(oracle):
    """|v * scale| >= 9.2e18: every emit is dropped and counted, every bin that received one is NaN."""
    print("case: C1 f64 fixed scale=1e21 (overflow)", flush=True)
    xs, keys, theta = configs.c1_inputs(4096)
    res = _mapped(configs.C1, {"hist": tm.Sum((16,), np.float64, fixed_point=True, scale=1e21)})(xs, keys, theta)
    _sync()
    _, out, over = oracle.wide_tallies(lambda: oracle.c1_fwd(xs, keys, theta), [(16, 1e21, np.float64)])
    h = _np(res.outputs["hist"])
    assert over > 0 and int(_np(res.stats["fixed_point_overflow"])) == over
    assert np.array_equal(np.isnan(h), out[0][1]) and out[0][1].any()


def test_c2_fixed_point_f64_bitwise(oracle):
    print("case: C2 f64 fixed N=65536", flush=True)
    x0, keys, drift = configs.c2_inputs(65_536)
    outs = {"occ": tm.Sum((128,), np.float64, fixed_point=True, scale=2.0 ** 24),
            "wall": tm.Sum((2,), np.float64, fixed_point=True, scale=1.0)}
    res = _mapped(configs.C2, outs)(x0, keys, drift)
    _sync()
    _, out, over = oracle.wide_tallies(lambda: oracle.c2_fwd(x0, keys, drift),
                                       [(128, 2.0 ** 24, np.float64), (2, 1.0, np.float64)])
    assert _same(_np(res.outputs["occ"]), out[0][0])
    assert _same(_np(res.outputs["wall"]), out[1][0])
    assert out[1][0].sum() == 65_536.0


def _int_item(t, x):
    return t.add("h", x % 7, x * 3 + 5)


def _int_totals(x):
    return [int((x[x % 7 == b].astype(np.int64) * 3 + 5).sum()) for b in range(7)]


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.int64, np.uint64])
def test_integer_fixed_point_sums(dt):
    """integer emits into integer fixed-point outputs against Python integers: per emit round-half-even(v * scale),
    the total times 1/scale in double, truncated toward zero (scale 1 and 4: the plain sum; 0.25: emits rounded to
    multiples of 4)."""
    print(f"case: integer fixed point {np.dtype(dt).name}", flush=True)
    x = np.arange(20_000, dtype=np.int32)
    v = x.astype(np.int64) * 3 + 5
    for scale in (1.0, 4.0, 0.25):
        res = tm.vmap(_int_item, outputs={"h": tm.Sum((7,), dt, fixed_point=True, scale=scale)}, in_axes=(0,))(x)
        _sync()
        tot = [sum(round(float(e) * scale) for e in v[x % 7 == b]) for b in range(7)]
        want = np.array([int(float(t) * (1.0 / scale)) for t in tot], dt)
        assert _same(_np(res.outputs["h"]), want)
        assert int(_np(res.stats["fixed_point_overflow"])) == 0


def test_integer_fixed_point_saturates_and_counts():
    """an int32 output whose total (~2e11) does not fit saturates to INT32_MAX and counts one overflow."""
    print("case: int32 fixed point saturation", flush=True)
    x = np.arange(20_000, dtype=np.int32)
    res = tm.vmap(lambda t, x: t.add("h", 0, x * 1000), outputs={"h": tm.Sum((1,), np.int32, fixed_point=True,
                                                                            scale=1.0)}, in_axes=(0,))(x)
    _sync()
    assert int(_np(res.outputs["h"])[0]) == 2 ** 31 - 1
    assert int(_np(res.stats["fixed_point_overflow"])) == 1


def test_fixed_point_carry_past_int64():
    """totals past 2^63 keep their carry word: 16 items emit +-4e18 (scale 1) into one bin and 4e18 into another;
    the float64 readout is the exact total; an int64 output of a total past 2^63 saturates and is counted."""
    print("case: fixed point carry past 2^63", flush=True)

    def item(t, s):
        t = t.add("a", 0, s * 4e18)
        return t.add("b", 0, 4e18)
    s = np.array([1.0] * 12 + [-1.0] * 4)
    res = tm.vmap(item, outputs={"a": tm.Sum((1,), np.float64, fixed_point=True, scale=1.0),
                                 "b": tm.Sum((1,), np.float64, fixed_point=True, scale=1.0)}, in_axes=(0,))(s)
    _sync()
    assert float(_np(res.outputs["a"])[0]) == 8 * 4e18 and float(_np(res.outputs["b"])[0]) == 16 * 4e18
    assert int(_np(res.stats["fixed_point_overflow"])) == 0

    def item64(t, s, c):
        return t.add("a", 0, s * c)
    res = tm.vmap(item64, outputs={"a": tm.Sum((1,), np.int64, fixed_point=True, scale=1.0)}, in_axes=(0, None))(
        s.astype(np.int64), np.int64(4_000_000_000_000_000_000))
    _sync()
    assert int(_np(res.outputs["a"])[0]) == 2 ** 63 - 1
    assert int(_np(res.stats["fixed_point_overflow"])) == 1


@pytest.mark.parametrize("dt", [np.float64, np.int64, np.uint64])
def test_plain_64bit_sums(dt, oracle):
    """plain (non-fixed) float64 / int64 / uint64 sums: native 64-bit atomics, privatised in LDS."""
    print(f"case: plain {np.dtype(dt).name} sum", flush=True)
    if dt == np.float64:
        xs, keys, theta = configs.c1_inputs(1 << 16)
        res = _mapped(configs.C1, {"hist": tm.Sum((16,), np.float64)})(xs, keys, theta)
        _sync()
        ref = oracle.c1_fwd(xs, keys, theta)
        np.testing.assert_allclose(_np(res.outputs["hist"]), ref.tallies64["hist"], rtol=1e-12)
        return
    x = np.arange(20_000, dtype=np.int32)
    res = tm.vmap(_int_item, outputs={"h": tm.Sum((7,), dt)}, in_axes=(0,))(x)
    _sync()
    assert _same(_np(res.outputs["h"]), np.array(_int_totals(x), dt))


def test_reverse_mode_through_float64_output_raises():
    """the replay adjoint reads float32 cotangents only: a cotangent for a float64 output is refused, never
    dropped."""
    print("case: vjp through a float64 output", flush=True)
    xs, keys, theta = configs.c1_inputs(256)
    f = _mapped(configs.C1, {"hist": tm.Sum((16,), np.float64, fixed_point=True)})
    _, pullback = tm.vjp(f, xs, keys, theta, argnums=2)
    with pytest.raises(Exception, match="float64"):
        pullback({"hist": 1.0})
