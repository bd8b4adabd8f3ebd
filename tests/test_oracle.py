"""Pins the oracle (oracle/libtmref.so) before it is trusted: known-answer vectors, published values, closed forms,
brute force on tiny inputs, and an independent implementation of the RNG layering."""
import numpy as np
import pytest

from oracle import exact as X


# Random123 threefry2x32 (20 rounds) known-answer vectors (Salmon et al. 2011, kat_vectors); reference
# kernel.py:137-150 implements the same function.
KAT = [((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6b200159, 0x99ba4efe)),
       ((0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff), (0x1cb996fc, 0xbb002be7)),
       ((0x13198a2e, 0x03707344), (0x243f6a88, 0x85a308d3), (0xc4923a9c, 0x483df7a0))]


@pytest.mark.parametrize("key,ctr,want", KAT)
def test_threefry_kat(oracle, key, ctr, want):
    assert oracle.threefry(key[0], key[1], ctr[0], ctr[1]) == want


def test_threefry_kat_host_rng():
    from tallymap_amd import random as R
    for key, ctr, want in KAT:
        o0, o1 = R._tf_np(np.uint32(key[0]), np.uint32(key[1]), np.uint32(ctr[0]), np.uint32(ctr[1]))
        assert (int(o0), int(o1)) == want


def test_erfinv_published(oracle):
    # reference tests/edge.py:2727: erfinv(0.5) = 0.4769362762044699, erfinv(0.9) = 1.1630871536766743
    for y, v in ((0.5, 0.4769362762044699), (0.9, 1.1630871536766743)):
        got = float(oracle.erfinvf(y))
        assert got == float(np.float32(v)) or abs(got - v) <= 2 * np.spacing(np.float32(v))


def test_erfinv_two_ulp_of_rounded(oracle):
    # reference tests/edge.py:2739-2746: the f32 erf_inv is within 2 ulp of the correctly rounded value; the
    # correctly rounded value is checked here through erf (math.erf is correctly rounded to ~1 ulp of double)
    import math
    rng = np.random.default_rng(1)
    ys = rng.uniform(-0.999, 0.999, 4000).astype(np.float32)
    for y in ys:
        g = float(oracle.erfinvf(y))
        # solve erf(x) = y in double by bisection
        lo, hi = -6.0, 6.0
        for _ in range(200):
            mid = 0.5 * (lo + hi)
            if math.erf(mid) < float(y):
                lo = mid
            else:
                hi = mid
        x = np.float32(0.5 * (lo + hi))
        assert abs(np.float32(g) - x) <= 2 * np.spacing(abs(x)) + 1e-45


def test_rng_layering_matches_host_rng(oracle):
    """fold_in / split / bits / uniform / normal's uniform: the oracle's C and tallymap_amd.random's numpy are two
    independent restatements of jax's partitionable threefry layering (JAX itself is not installed here: the
    layering is pinned only by this agreement and the threefry KAT)."""
    from tallymap_amd import random as R
    key = R.PRNGKey(0)
    assert key.tolist() == [0, 0]
    ks = R.split(key, 100)
    assert np.array_equal(ks, oracle.split(key, 100))
    for i in range(0, 100, 7):
        for d in (0, 1, 17, 0xFFFFFFFF):
            assert np.array_equal(R.fold_in(ks[i], d), oracle.fold_in(ks[i], d))
        assert int(R.bits(ks[i])) == oracle.bits32(ks[i])
        for lo, hi in ((0.0, 1.0), (0.2, 0.8), (np.nextafter(np.float32(-1), np.float32(0)), 1.0)):
            a = R.uniform(ks[i], (), np.float32, lo, hi)
            b = oracle.uniform(ks[i], lo, hi)
            assert a.view(np.uint32) == b.view(np.uint32)
    # split(PRNGKey(0), n)[i] = threefry((0, 0); (0, i))
    assert oracle.threefry(0, 0, 0, 5) == tuple(int(x) for x in ks[5])


def test_exact_sum_against_python_integers(oracle):
    rng = np.random.default_rng(7)
    cases = [rng.standard_normal(1000).astype(np.float32),
             (rng.standard_normal(500) * 1e30).astype(np.float32),
             np.concatenate([np.full(1000, 1e-45, np.float32), np.full(3, 1.0, np.float32)]),
             np.array([1.0, 2 ** -24, 2 ** -24], np.float32),           # a tie resolved by the exact sum
             np.array([3.4e38, 3.4e38, -3.4e38], np.float32),           # exact through an intermediate overflow
             np.array([1e-38, -1e-38, 2e-45], np.float32),
             np.array([np.float32(2 ** 24), 1.0, 1.0, 1.0], np.float32)]
    for v in cases:
        got, bad = oracle.exact_sum(v)
        want, wbad = X.exact_sum(v)
        assert bad == wbad
        assert got.view(np.uint32) == want.view(np.uint32), (v[:4], got, want)
    for v in (np.array([np.inf, 1.0], np.float32), np.array([3.4e38, 3.4e38], np.float32)):
        got, bad = oracle.exact_sum(v)
        assert bad and np.isnan(got)


def _c1_python(xs, keys, theta, M=100):
    """brute-force pure-Python restatement of the quickstart walker on numpy float32 scalars (tiny N)."""
    from tallymap_amd import random as R
    f32 = np.float32
    hist = np.zeros(16, np.float64)
    ks, trs = [], []
    for i in range(len(xs)):
        x, k = f32(xs[i]), 0
        while k < M and x > f32(0.05):
            u = R.uniform(R.fold_in(keys[i], k))
            idx = int(np.trunc(np.float32(x * f32(16.0))))
            if 0 <= idx < 16:
                hist[idx] += float(f32(theta * f32(f32(1.0) - x)))
            x = f32(x * f32(f32(0.5) + f32(f32(0.5) * u)))
            k += 1
        ks.append(k)
        trs.append(k >= M and x > f32(0.05))
    return hist, np.array(ks), np.array(trs)


def test_c1_oracle_brute_force(oracle):
    from tallymap_amd import configs
    xs, keys, theta = configs.c1_inputs(300)
    h, k, tr = _c1_python(xs, keys, theta)
    r = oracle.c1_fwd(xs, keys, theta)
    assert np.array_equal(r.per_item, k)
    assert np.array_equal(r.trunc, tr)
    assert np.allclose(r.tallies64["hist"], h, rtol=1e-12, atol=0)
    assert np.allclose(r.tallies["hist"], h, rtol=1e-5)


def test_c1_oracle_truncation_planted(oracle):
    """a tiny max_steps truncates items: trip counts hit the cap, truncation flags are set; a planted mistake in
    the cap (one step more) is visible in the counts."""
    from tallymap_amd import configs
    xs, keys, theta = configs.c1_inputs(300)
    r = oracle.c1_fwd(xs, keys, theta, max_steps=3)
    assert r.per_item.max() == 3 and r.trunc.sum() > 0
    h, k, tr = _c1_python(xs, keys, theta, M=3)
    assert np.array_equal(r.per_item, k) and np.array_equal(r.trunc, tr)
    _, k4, _ = _c1_python(xs, keys, theta, M=4)
    assert not np.array_equal(r.per_item, k4)


def test_c1_gradient_closed_form(oracle):
    """theta is linear and outside control flow: d(hist.sum())/d theta = hist.sum() / theta."""
    from tallymap_amd import configs
    xs, keys, theta = configs.c1_inputs(10_000)
    r = oracle.c1_fwd(xs, keys, theta)
    g, ntr = oracle.c1_grad(xs, keys, theta, np.ones(16, np.float32))
    assert ntr == 0
    want = r.tallies64["hist"].sum() / float(theta)
    assert abs(float(g) - want) <= 1e-6 * abs(want)


def test_c2_oracle_invariants(oracle):
    from tallymap_amd import configs
    x0, keys, drift = configs.c2_inputs(2000)
    assert np.array_equal(x0, oracle.c2_x0(keys))
    r = oracle.c2_fwd(x0, keys, drift)
    # one occupancy emit per step (kept or dropped), one wall emit per item
    assert r.tallies64["occ"].sum() + r.stats[4] == r.per_item.sum()
    assert r.tallies64["wall"].sum() == 2000
    assert 200 < r.per_item.mean() < 1500 and not r.trunc.any()
    g, ntr = oracle.c2_grad(x0, keys, drift, np.ones(128, np.float32), np.ones(2, np.float32))
    assert g == 0.0 and ntr == 0


def test_c1_per_item_tangent_pathwise(oracle):
    """the oracle's forward-mode d/d x0 of each item against the pathwise derivative evaluated in float64 along the
    item's own (frozen) integer path: x_k = x0 prod_{j<k} f_j with f_j = 0.5 + 0.5 u_j independent of x0, so
    d/d x0 sum_k ct[bin_k] theta (1 - x_k) = -theta sum_k ct[bin_k] prod_{j<k} f_j."""
    from tallymap_amd import configs
    from tallymap_amd import random as R
    xs, keys, theta = configs.c1_inputs(200)
    ct = np.linspace(0.5, 2.0, 16).astype(np.float32)
    _, dx, _ = oracle.c1_grad(xs, keys, theta, ct, per_item=True)
    f32 = np.float32
    for i in range(200):
        x, k, prod, want = f32(xs[i]), 0, 1.0, 0.0
        while k < 100 and x > f32(0.05):
            u = R.uniform(R.fold_in(keys[i], k))
            b = int(np.trunc(np.float32(x * f32(16.0))))
            f = f32(f32(0.5) + f32(f32(0.5) * u))
            if 0 <= b < 16:
                want += float(ct[b]) * -float(theta) * prod
            prod *= float(f)
            x = f32(x * f)
            k += 1
        assert abs(float(dx[i]) - want) <= 1e-5 * max(1.0, abs(want)), (i, dx[i], want)
