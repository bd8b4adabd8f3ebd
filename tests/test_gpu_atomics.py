"""The atomic-throughput microbenchmarks behind bench.py's emit roofline: every pattern's buffer holds exactly the
adds issued (the measured rate is of real, complete work)."""
import pytest

from tallymap_amd.backend import atomics

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pattern", atomics.PATTERNS)
def test_atomic_pattern_counts_exactly(pattern):
    print(f"case: atomics {pattern}", flush=True)
    r = atomics.run(pattern, reps=1)
    assert r["exact"], r
    assert r["adds_per_s"] > 0
