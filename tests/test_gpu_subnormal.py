"""Subnormal and signed-zero emits on the GPU (reference tests/edge.py:3106-3210): a GPU's f32 atomic add may flush
subnormal inputs and results to zero, and the build must not.  Eight bins whose sums are exact in any order:
  0: 4 x 1.4e-44                1: two normals cancelling to a subnormal      2: a normal + a subnormal
  3: one subnormal (2^-140)     4: a negative subnormal total                 5: 1 + 2^-149 (rounds to 1)
  6: 3 x 2^-110 (small normals) 7: -0.0 alone (a zeroed bin plus -0.0 is +0.0)
Every output is compared bitwise with the exact sums (Python integers in units of 2^-149, rounded once), for
privatised (LDS) and global bins, plain and exact (fixed_point=True) float32 sums, a Records field, float64 sums of
the values x 2^-900 (float64 subnormals), and the jvp tangents and grad cotangents of the same emits -- so the
subnormal-safe branches of the f32 atomics run on hardware."""
import numpy as np
import pytest

import tallymap_amd as tm
from oracle import exact as X

pytestmark = pytest.mark.gpu

TN = 2.0 ** -126
SUBN = [(0, 1.4e-44)] * 4 + [(1, 1.5 * TN), (1, -TN), (2, TN), (2, 2.0 ** -140), (3, 2.0 ** -140), (4, -3e-44),
                             (4, 1e-45), (5, 1.0), (5, 1e-45)] + [(6, 2.0 ** -110)] * 3 + [(7, -0.0)]
IDX = np.array([i for i, _ in SUBN], np.int32)
VAL = np.array([v for _, v in SUBN], np.float32)
NB = 8
# bins: 8 (privatised in LDS), 2048 (LDS for a plain f32 sum, global words for an exact one), 16384 (global)
SIZES = (NB, 2048, 16384)


def _exact(vals, bins, nb):
    tot = [0] * nb
    for v, b in zip(vals, bins):
        tot[int(b)] += X.units(v)
    return np.array([X.round_units(t) for t in tot], np.float32)


WANT = _exact(VAL, IDX, NB)


def _np(x):
    import torch
    torch.cuda.synchronize()
    return x.cpu().numpy()


def _bitwise(a, b):
    a, b = np.atleast_1d(np.asarray(a)), np.atleast_1d(np.asarray(b))
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_exact_sums_are_what_the_cases_say():
    """the expected bins, independently of the integer reference: 4 x 1.4e-44 is 40 x 2^-149 (1.4e-44 rounds to
    10 units); 1.5 TN - TN = 2^-127; bin 7 is +0.0."""
    assert WANT[0] == np.float32(40 * 2.0 ** -149) and WANT[1] == np.float32(2.0 ** -127)
    assert WANT[3] == np.float32(2.0 ** -140) and WANT[5] == np.float32(1.0) and WANT[6] == np.float32(3 * 2.0 ** -110)
    assert WANT[4] < 0 and abs(WANT[4]) < TN
    assert WANT[7].view(np.uint32) == 0


@pytest.mark.parametrize("fp", [False, True], ids=["plain", "exact"])
@pytest.mark.parametrize("S", SIZES)
def test_subnormal_emits_sum(S, fp):
    print(f"case: subnormal emits, Sum(({S},), fixed_point={fp})", flush=True)
    f = tm.vmap(lambda t, x, i: t.add("s", i, x), outputs={"s": tm.Sum((S,), np.float32, fixed_point=fp)})
    res = f(VAL, IDX)
    got = _np(res.outputs["s"])
    assert _bitwise(got[:NB], WANT), (got[:NB], WANT)
    assert not got[NB:].view(np.uint32).any()
    assert int(_np(res.stats["fixed_point_overflow"])) == 0


def test_subnormal_emits_records_field():
    print("case: subnormal emits, Records field", flush=True)
    f = tm.vmap(lambda t, x: t.append("r", {"q": x}), outputs={"r": tm.Records({"q": np.float32}, capacity=32)})
    q = _np(f(VAL).outputs["r"]["q"])
    want = np.zeros(32, np.float32)
    want[:len(SUBN)] = np.where(VAL == 0, np.float32(0.0), VAL)          # -0.0 lands as +0.0
    assert _bitwise(q, want), q[:len(SUBN)]


@pytest.mark.parametrize("S", (NB, 2048))
def test_subnormal_emits_float64(S):
    """the values x 2^-900 as float64 (subnormal doubles): a plain float64 Sum keeps them (CAS below 2^-970)."""
    print(f"case: subnormal emits, float64 Sum(({S},))", flush=True)
    f = tm.vmap(lambda t, x, i: t.add("s", i, x.astype(np.float64) * 2.0 ** -900),
                outputs={"s": tm.Sum((S,), np.float64)})
    got = _np(f(VAL, IDX).outputs["s"])
    want = WANT.astype(np.float64) * 2.0 ** -900
    assert np.all(np.abs(want[[0, 3, 4]]) < 2.0 ** -1022)        # (these bins are float64 subnormals)
    assert _bitwise(got[:NB], want), (got[:NB], want)


@pytest.mark.parametrize("fp", [False, True], ids=["plain", "exact"])
@pytest.mark.parametrize("S", SIZES)
def test_subnormal_tangents_and_cotangents(S, fp):
    """t.add(i, x * th) at th = 1: the jvp tangent along th is the emitted values again (bitwise the exact sums);
    the gradient of <w, s> with w = 1 on the all-subnormal bins 0, 3, 4 is the exact sum of their values."""
    print(f"case: subnormal tangents and cotangents, Sum(({S},), fixed_point={fp})", flush=True)
    f = tm.vmap(lambda t, x, i, th: t.add("s", i, x * th), in_axes=(0, 0, None),
                outputs={"s": tm.Sum((S,), np.float32, fixed_point=fp)})
    th = np.float32(1.0)
    p, tg = tm.jvp(f, (VAL, IDX, th), (None, None, np.float32(1.0)))
    assert _bitwise(_np(p.outputs["s"])[:NB], WANT)
    assert _bitwise(_np(tg.outputs["s"])[:NB], WANT)
    w = np.zeros(S, np.float32)
    w[[0, 3, 4]] = 1.0
    g = _np(tm.grad(f, weights={"s": w}, argnums=2)(VAL, IDX, th))
    sel = np.isin(IDX, [0, 3, 4])
    gwant = _exact(VAL[sel], np.zeros(int(sel.sum()), int), 1)[0]
    assert _bitwise(np.float32(g), gwant), (g, gwant)


def test_subnormal_records_tangent_and_cotangent():
    print("case: subnormal Records tangent and cotangent", flush=True)
    f = tm.vmap(lambda t, x, th: t.append("r", {"q": x * th}), in_axes=(0, None),
                outputs={"r": tm.Records({"q": np.float32}, capacity=32)})
    th = np.float32(1.0)
    p, tg = tm.jvp(f, (VAL, th), (None, np.float32(1.0)))
    want = np.zeros(32, np.float32)
    want[:len(SUBN)] = np.where(VAL == 0, np.float32(0.0), VAL)
    assert _bitwise(_np(p.outputs["r"]["q"]), want)
    t = _np(tg.outputs["r"]["q"])
    assert _bitwise(np.where(t == 0, np.float32(0.0), t), want)
    sub = np.zeros(32, np.float32)
    sub[:len(SUBN)] = np.abs(VAL) < TN
    g = _np(tm.grad(f, weights={"r": {"q": sub}}, argnums=1)(VAL, th))
    sel = np.abs(VAL) < TN
    gwant = _exact(VAL[sel], np.zeros(int(sel.sum()), int), 1)[0]
    assert _bitwise(np.float32(g), gwant), (g, gwant)
