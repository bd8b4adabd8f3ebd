"""The reference's published trip-count tables, reproduced on the GPU.

docs/performance_detail.md holds, for each of its benchmark problems at divergence `mid`, the mean, 99th percentile
and maximum of the per-item step counts at five sizes N (tables at :167, :274, :381, :488, :558, :758, :1119), measured by
benchmarks/vs_jax/harness.py:152-156 (`trip_stats`: numpy mean, np.percentile(k, 99), max) and printed with
make_tables.py:88-91 (`f"{x:.3g}"`).  The inputs are the problems' own (keys = jax.random.split(PRNGKey(s), N) as in
benchmarks/vs_jax/problems/*.py), so the per-item draws -- and with them the tail of the trip-count distribution --
are fixed by JAX's PRNG layering (split, fold_in, random_bits, uniform, normal over threefry2x32).  The maxima at
five sizes are extreme-value statistics of those particular draws: a layering that differed anywhere (a swapped
counter word, a different fold_in, another uniform mantissa construction) gives the same distribution but other
maxima.  The walker of random_walk draws nothing that decides its trip count (ceil(log wmin / log decay)), so its
rows check the inputs only.

ode_ensemble draws nothing either (numpy inputs): its trip count is the adaptive Bogacki-Shampine integrator's
number of trial steps, and a trial whose scaled error norm lies within an ulp or so of 1 is accepted or rejected
depending on the last bits of the arithmetic.  The published table was measured on plain XLA (harness `telemetry`,
ode_ensemble.py:94-101) with XLA's own GPU pow / sin and its own operation fusion, not the uncontracted float32 with
glibc's powf / sinf this build computes, so its p99 and maximum are compared within ODE_TAIL_STEPS trial steps and
its means exactly.
"""
import numpy as np
import pytest

from tallymap_amd import problems as P

pytestmark = pytest.mark.gpu

# (N, mean, p99, max) as printed, divergence `mid`
PUBLISHED = {
    "random_walk": ("docs/performance_detail.md:171-175",
                    [(4096, "25.2", "85", "90"), (16384, "25.5", "85", "90"), (65536, "25.4", "85", "90"),
                     (524288, "25.5", "84", "90"), (4194304, "25.5", "84", "90")]),
    "transport": ("docs/performance_detail.md:278-282",
                  [(4096, "16.1", "61", "84"), (16384, "16.1", "61", "94"), (65536, "16.2", "62", "99"),
                   (524288, "16.1", "62", "107"), (4194304, "16.1", "62", "110")]),
    "walk_on_spheres": ("docs/performance_detail.md:385-389",
                        [(4096, "8.88", "32", "48"), (16384, "8.75", "31", "59"), (65536, "8.78", "30", "76"),
                         (524288, "8.79", "31", "88"), (4194304, "8.8", "31", "90")]),
    "ode_ensemble": ("docs/performance_detail.md:492-496",
                     [(256, "226", "317", "319"), (16384, "228", "322", "337"), (65536, "227", "322", "336"),
                      (262144, "227", "323", "340"), (1048576, "227", "323", "342")]),
    "gillespie": ("docs/performance_detail.md:562-566",
                  [(1024, "1.99e+03", "4.64e+03", "5.15e+03"), (16384, "1.91e+03", "4.71e+03", "5.72e+03"),
                   (65536, "1.91e+03", "4.7e+03", "5.84e+03"), (262144, "1.92e+03", "4.71e+03", "6.3e+03"),
                   (1048576, "1.92e+03", "4.71e+03", "6.3e+03")]),
    "barrier": ("docs/performance_detail.md:762-766",
                [(4096, "222", "252", "252"), (16384, "222", "252", "252"), (65536, "221", "252", "252"),
                 (524288, "221", "252", "252"), (4194304, "221", "252", "252")]),
    # benchmarks/vs_jax/problems/small_n.py:31-43: the barrier item and keys at mid, down to N = 1; at small N the
    # mean trip count is a property of those few normal draws
    "small_n": ("docs/performance_detail.md:1123-1131",
                [(1, "252", "252", "252"), (4, "252", "252", "252"), (16, "228", "252", "252"),
                 (64, "222", "252", "252"), (256, "215", "252", "252"), (1024, "220", "252", "252"),
                 (4096, "222", "252", "252"), (16384, "222", "252", "252"), (65536, "221", "252", "252")]),
}
PROBLEM_OF = {"small_n": "barrier"}


ODE_TAIL_STEPS = 4


def _fmt(x):
    return f"{x:.3g}"


@pytest.mark.parametrize("name", list(PUBLISHED))
def test_trip_counts_equal_published_tables(name):
    import torch
    src, rows = PUBLISHED[name]
    prob = PROBLEM_OF.get(name, name)
    f = P.mapped(prob)
    got = []
    for n, mean, p99, mx in rows:
        print(f"case: published trips {name} N={n}", flush=True)
        args, _ = P.PROBLEMS[prob]["inputs"](n)
        r = f(*args)
        assert int(r.stats["n_truncated"].item()) == 0
        k = r.per_item[-1] if isinstance(r.per_item, (tuple, list)) else r.per_item
        k = k.cpu().numpy().astype(np.int64)
        torch.cuda.synchronize()
        got.append(((n, _fmt(float(k.mean())), _fmt(float(np.percentile(k, 99))), _fmt(int(k.max()))),
                    (n, mean, p99, mx)))
    if name == "ode_ensemble":
        bad = [(g, w) for g, w in got
               if g[1] != w[1] or any(abs(float(a) - float(b)) > ODE_TAIL_STEPS for a, b in zip(g[2:], w[2:]))]
    else:
        bad = [(g, w) for g, w in got if g != w]
    assert not bad, f"{name}: (measured, published {src}) differ: {bad}"


# transport's divergence levels differ only in theta (benchmarks/vs_jax/problems/transport.py:37-38, TH0)
TRANSPORT_LEVELS = {
    "high": ((0.05, 0.5), "docs/performance_detail.md:288-289", [(4096, "159", "309", "338"),
                                                                 (524288, "161", "307", "371")]),
    "low": ((0.5, 0.5), "docs/performance_detail.md:295-296", [(4096, "4.49", "16.1", "35"),
                                                               (524288, "4.51", "17", "45")]),
}


@pytest.mark.parametrize("level", list(TRANSPORT_LEVELS))
def test_transport_trip_counts_at_other_divergence_levels(level):
    import torch
    th, src, rows = TRANSPORT_LEVELS[level]
    f = P.mapped("transport")
    bad = []
    for n, mean, p99, mx in rows:
        print(f"case: published trips transport {level} N={n}", flush=True)
        (p0, keys, _, eff), _ = P.tr_inputs(n)
        r = f(p0, keys, np.array(th, np.float32), eff)
        assert int(r.stats["n_truncated"].item()) == 0
        k = r.per_item.cpu().numpy().astype(np.int64)
        torch.cuda.synchronize()
        got = (n, _fmt(float(k.mean())), _fmt(float(np.percentile(k, 99))), _fmt(int(k.max())))
        if got != (n, mean, p99, mx):
            bad.append((got, (n, mean, p99, mx)))
    assert not bad, f"transport {level}: (measured, published {src}) differ: {bad}"
