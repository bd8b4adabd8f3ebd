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


def _c1_python(xs, keys, theta, M=100, emits=None):
    """brute-force pure-Python restatement of the quickstart walker on numpy float32 scalars (tiny N); emits: a
    list of 16 lists that collects every in-range emitted f32 value per bin."""
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
                if emits is not None:
                    emits[idx].append(f32(theta * f32(f32(1.0) - x)))
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


def test_oracle_exact_tallies_against_python_integers(oracle):
    """the oracle's exact tally mode (Sum(fixed_point=True)): each bin equals the Python-integer exact sum of the
    brute-force walker's emitted f32 values, rounded once (reference tests/edge.py:2038-2065), for any team size."""
    from tallymap_amd import configs
    xs, keys, theta = configs.c1_inputs(300)
    emits = [[] for _ in range(16)]
    _c1_python(xs, keys, theta, emits=emits)
    want = np.array([X.exact_sum(np.array(e, np.float32))[0] if e else np.float32(0) for e in emits], np.float32)
    for nt in (1, 3):
        _, ex = oracle.exact_tallies(lambda: oracle.c1_fwd(xs, keys, theta, nthreads=nt), [16])
        got, bad = ex[0]
        assert not bad.any()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_oracle_fixed_point_tallies_against_python_integers(oracle):
    """the oracle's scaled fixed-point mode (Sum(fixed_point=True, scale) of a non-f32 dtype): each bin's integer
    total equals the Python sum of round-half-even(v * scale) over the brute-force walker's emits, for scales that
    keep every emit exact (2^32), round them (16, 2^-1: many emits round to 0 or ties) and overflow every emit
    (1e21: all bins NaN, one count per emit); the readout is total * (1/scale) for float64 and saturates integer
    dtypes."""
    from tallymap_amd import configs
    xs, keys, theta = configs.c1_inputs(300)
    emits = [[] for _ in range(16)]
    _c1_python(xs, keys, theta, emits=emits)
    n_emits = sum(len(e) for e in emits)
    for scale in (2.0 ** 32, 16.0, 0.5):
        want = [sum(round(float(v) * scale) for v in e) for e in emits]
        for nt in (1, 3):
            _, out, over = oracle.wide_tallies(lambda: oracle.c1_fwd(xs, keys, theta, nthreads=nt),
                                               [(16, scale, np.float64)])
            vals, bad, tot = out[0]
            assert tot == want and not bad.any() and over == 0
            assert np.array_equal(vals, np.array([float(t) * (1.0 / scale) for t in want]))
    _, out, over = oracle.wide_tallies(lambda: oracle.c1_fwd(xs, keys, theta), [(16, 1e21, np.float64)])
    vals, bad, tot = out[0]
    assert over == n_emits and all(bad == np.array([len(e) > 0 for e in emits])) and tot == [0] * 16
    assert np.isnan(vals[bad]).all()
    # the readout into integer dtypes: truncation toward zero, saturation counted
    assert oracle.wide_readout(7, False, 2.0, np.int32) == (3, False)
    assert oracle.wide_readout(-7, False, 2.0, np.int32) == (-3, False)
    assert oracle.wide_readout(2 ** 40, False, 1.0, np.int32) == (2 ** 31 - 1, True)
    assert oracle.wide_readout(-1, False, 1.0, np.uint32) == (0, True)
    assert oracle.wide_readout(2 ** 70, False, 1.0, np.uint64) == (2 ** 64 - 1, True)
    v, c = oracle.wide_readout(2 ** 100, False, 2.0 ** -1000, np.float64)
    assert np.isnan(v) and c


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


# ------------------------------------------------------------------------------------------- C3 pins
def test_c3_no_scattering_is_beer_lambert(oracle):
    """mu_s = 0: a photon deposits its whole weight once, at its first interaction depth z ~ Exp(mu_a) on the axis
    (radius bin 0), or escapes past z = 5.  The depth histogram follows Beer-Lambert, P(bin j) = exp(-mu_a z_j) -
    exp(-mu_a z_(j+1)), z_j = 5 j / 64, within 5 binomial standard deviations per bin; and the pathwise gradient
    w.r.t. mu_a is exactly 0 (the deposit w mu_a / mu_t is 1)."""
    from tallymap_amd import random as R
    n, mu_a = 400_000, np.float32(0.5)
    keys = R.split(R.PRNGKey(3), n)
    r = oracle.c3_fwd(keys, mu_a, mu_s=0.0)
    t = r.tallies64["absorbed"]
    assert np.all(t[:, 1:] == 0)
    assert r.per_item.max() == 1 and not r.trunc.any()
    z = 5.0 * np.arange(65) / 64
    p = np.exp(-0.5 * z[:-1]) - np.exp(-0.5 * z[1:])
    dev = np.abs(t[:, 0] - n * p)
    assert np.all(dev <= 5 * np.sqrt(n * p * (1 - p)) + 1), dev.max()
    assert abs(t.sum() - n * (1 - np.exp(-2.5))) <= 5 * np.sqrt(n * 0.08)
    g, ntr = oracle.c3_grad(keys, mu_a, np.ones((64, 64), np.float32), mu_s=0.0)
    assert ntr == 0 and g == 0.0


def test_c3_henyey_greenstein_and_rotation(oracle):
    """The deflection cosine drawn from uniforms on a fine midpoint grid has mean g (the Henyey-Greenstein
    anisotropy), for g = 0.8 and g = 0.3, and stays in [-1, 1].  The direction update keeps directions unit length
    and turns each by exactly the sampled angle (old . new = cos theta), including the near-vertical frame, and two
    azimuths phi1, phi2 at the same deflection end cos(phi1 - phi2) apart around the old direction."""
    u = ((np.arange(1 << 20) + 0.5) / (1 << 20)).astype(np.float32)
    for g in (0.8, 0.3):
        c = oracle.hg_cost(u, g).astype(np.float64)
        assert abs(c.mean() - g) < 2e-4, (g, c.mean())
        assert c.min() >= -1.0 - 1e-6 and c.max() <= 1.0 + 1e-6
    rng = np.random.default_rng(1)
    n = 20_000
    d = rng.standard_normal((n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    d[:4] = [[0, 0, 1], [0, 0, -1], [0, 0, 1], [1e-4, 0, -1.0]]
    d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
    cost = rng.uniform(-1, 1, n).astype(np.float32)
    phi1 = rng.uniform(0, 2 * np.pi, n).astype(np.float32)
    phi2 = rng.uniform(0, 2 * np.pi, n).astype(np.float32)
    a = oracle.hg_rotate(d, cost, phi1).astype(np.float64)
    b = oracle.hg_rotate(d, cost, phi2).astype(np.float64)
    dd = d.astype(np.float64)
    # f32 roundoff of the update grows like eps / (1 - uz^2) near the vertical (sqrt(1 - uz^2) cancels)
    tol = 2e-5 + 4e-8 / np.maximum(1.0 - dd[:, 2] ** 2, 1e-12)
    near = np.abs(dd[:, 2]) > 0.99999                # the fixed frame treats d as vertical: the angle is off by at
    tol[near] = 2e-5 + np.hypot(dd[near, 0], dd[near, 1])  # most the transverse component it ignores
    assert np.all(np.abs(np.linalg.norm(a, axis=1) - 1.0) <= tol)
    assert np.all(np.abs(np.sum(dd * a, axis=1) - cost) <= 2 * tol)
    va = a - cost[:, None] * dd
    vb = b - cost[:, None] * dd
    nrm = np.linalg.norm(va, axis=1) * np.linalg.norm(vb, axis=1)
    ok = nrm > 1e-3
    cosd = np.sum(va * vb, axis=1)[ok] / nrm[ok]
    assert np.allclose(cosd, np.cos(phi1[ok].astype(np.float64) - phi2[ok]), atol=2e-3)


# ------------------------------------------------------------------------------------------- C4 pins
def test_c4_walk_on_spheres_estimates_the_harmonic_extension(oracle):
    """Walk on spheres estimates the harmonic function with boundary values sin(3 theta), u(r, theta) = r^3
    sin(3 theta): from fixed start points the mean score / a of 200,000 walkers agrees within 5 standard errors plus
    the 1e-3 shell's bias.  d(sum of the walker tally) / d a = sum(scores) / a (a multiplies every score)."""
    from tallymap_amd import random as R
    n = 200_000
    keys = R.split(R.PRNGKey(11), n)
    ids = np.arange(n, dtype=np.int32)
    for x, y in ((0.5, 0.3), (-0.2, 0.6), (0.1, -0.85)):
        p0 = np.tile(np.array([x, y], np.float32), (n, 1))
        r = oracle.c4_fwd(p0, keys, ids, np.float32(1.0))
        s = r.tallies64["walker"][:, 0]
        exact = np.hypot(x, y) ** 3 * np.sin(3 * np.arctan2(y, x))
        assert abs(s.mean() - exact) <= 5 * s.std() / np.sqrt(n) + 3e-3, (x, y, s.mean(), exact)
        assert not r.trunc.any()
    a = np.float32(0.75)
    r = oracle.c4_fwd(p0, keys, ids, a)
    g, ntr = oracle.c4_grad(p0, keys, ids, a, np.zeros((256, 256), np.float32), np.ones((n, 1), np.float32))
    assert abs(float(g) - r.tallies64["walker"].sum() / 0.75) <= 1e-5 * np.abs(r.tallies64["walker"]).sum()


# ------------------------------------------------------------------------------------------- C5 pins
def test_c5_tableau_is_dormand_prince(oracle):
    """the oracle's and the item's coefficients are scipy's RK45 (Dormand-Prince 5(4)) tableau, as f32 (the error
    weights up to sign, which the error norm does not see)."""
    from scipy.integrate._ivp.rk import RK45

    from tallymap_amd import configs
    c, a, b, e = oracle.c5_tableau()
    assert np.array_equal(c, RK45.C[1:5].astype(np.float32))
    assert np.array_equal(a, np.concatenate([RK45.A[i, :i] for i in range(1, 6)]).astype(np.float32))
    assert np.array_equal(b, RK45.B[[0, 2, 3, 4, 5]].astype(np.float32))
    assert np.array_equal(e, (-RK45.E[[0, 2, 3, 4, 5, 6]]).astype(np.float32))
    assert np.array_equal(np.float32(configs.DP_C), c)
    assert np.array_equal(np.float32(np.concatenate(configs.DP_A)), a)
    assert np.array_equal(np.float32(configs.DP_B), b)
    assert np.array_equal(np.float32(configs.DP_E), e)


def _pendulum(A):
    def f(t, y):
        return [y[1], -0.1 * y[1] - np.sin(y[0]) + A * np.cos(2.0 / 3.0 * t)]
    return f


def test_c5_undriven_pendulum_matches_scipy(oracle):
    """A = 0 (no drive): the damped pendulum is not chaotic; the oracle's adaptive f32 DP5(4) final states at t = 50
    agree with scipy's solve_ivp (RK45, rtol 1e-11, float64) within 2e-4."""
    from scipy.integrate import solve_ivp
    rng = np.random.default_rng(5)
    th0 = rng.uniform(-3.0, 3.0, 12).astype(np.float32)
    om0 = rng.uniform(-2.0, 2.0, 12).astype(np.float32)
    ids = np.arange(12, dtype=np.int32)
    r = oracle.c5_fwd(th0, om0, ids, np.float32(0.0))
    assert not r.trunc.any()
    for i in range(12):
        s = solve_ivp(_pendulum(0.0), (0.0, 50.0), [float(th0[i]), float(om0[i])], rtol=1e-11, atol=1e-13)
        assert np.allclose(r.tallies64["state"][i], s.y[:, -1], atol=2e-4), (i, r.tallies64["state"][i], s.y[:, -1])


def test_c5_gradient_matches_finite_differences(oracle):
    """a weak drive (A = 0.1) from small initial states, where the motion is not chaotic: the oracle's forward-mode
    gradient of E(final) w.r.t. A for each item agrees with a central difference (h = 1e-3) of scipy's float64
    solution within 2e-3 relative."""
    from scipy.integrate import solve_ivp
    rng = np.random.default_rng(6)
    n = 6
    th0 = rng.uniform(-0.5, 0.5, n).astype(np.float32)
    om0 = rng.uniform(-0.5, 0.5, n).astype(np.float32)
    ids = np.arange(n, dtype=np.int32)
    A, h = 0.1, 1e-3
    r = oracle.c5_fwd(th0, om0, ids, np.float32(A))
    st = r.tallies["state"]
    ct_all = np.stack([np.sin(st[:, 0].astype(np.float64)), st[:, 1]], 1).astype(np.float32)
    for i in range(n):
        ct = np.zeros((n, 2), np.float32)
        ct[i] = ct_all[i]
        g, ntr = oracle.c5_grad(th0, om0, ids, np.float32(A), ct)
        y = [solve_ivp(_pendulum(a), (0.0, 50.0), [float(th0[i]), float(om0[i])], rtol=1e-12, atol=1e-14).y[:, -1]
             for a in (A + h, A - h)]
        dy = (y[0] - y[1]) / (2 * h)
        want = float(ct[i].astype(np.float64) @ dy)
        assert abs(float(g) - want) <= 2e-3 * abs(want), (i, float(g), want)
