"""The spawn paths' device passes (backend/util.py): the exclusive scan against numpy's cumsum (sizes across the
1024-element blocks and the top scan's 1024-block chunks) and the canonical row scatter against its definition."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 1000, 1024, 1025, 70_001, 3_000_000])
def test_exclusive_scan(n):
    print(f"case: exclusive scan n={n}", flush=True)
    import torch

    from tallymap_amd.backend import util
    c = np.random.default_rng(n).integers(0, 1 << 20, n).astype(np.int32)
    got = util.exclusive_scan(torch.from_numpy(c).cuda()).cpu().numpy()
    want = np.cumsum(c.astype(np.int64)) - c
    assert got.dtype == np.int64 and np.array_equal(got, want)


@pytest.mark.parametrize("dtype,shape", [(np.float32, ()), (np.uint32, (2,)), (np.float64, ()), (np.bool_, ())])
def test_tree_scatter(dtype, shape):
    """children of 5,000 parents with 0..3 children each, in a shuffled (ticket) order, land at first-child + ordinal."""
    print(f"case: tree scatter {np.dtype(dtype).name} {shape}", flush=True)
    import torch

    from tallymap_amd.backend import util
    rng = np.random.default_rng(3)
    cnt = rng.integers(0, 4, 5000).astype(np.int32)
    par = np.repeat(np.arange(5000, dtype=np.int32), cnt)
    ordn = np.concatenate([np.arange(k, dtype=np.int32) for k in cnt])
    m = len(par)
    perm = rng.permutation(m)
    src = (rng.integers(0, 1 << 30, (m,) + shape) % 2).astype(dtype) if dtype == np.bool_ else \
        rng.integers(0, 1 << 30, (m,) + shape).astype(dtype)
    off = util.exclusive_scan(torch.from_numpy(cnt).cuda())
    dst = torch.empty((m,) + shape, dtype=getattr(torch, np.dtype(dtype).name if dtype != np.bool_ else "bool"),
                      device="cuda")
    util.tree_scatter(off, torch.from_numpy(par[perm]).cuda(), torch.from_numpy(ordn[perm]).cuda(),
                      torch.from_numpy(src[perm]).cuda(), dst, m)
    assert np.array_equal(dst.cpu().numpy(), src)
