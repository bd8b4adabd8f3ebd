"""Reverse mode on the GPU: the replay adjoint kernel against the oracle's forward-mode (dual number) gradients.
Gradients within 1e-4 relative; the per-item cotangents bitwise independent of the checkpoint
count C (reference tests/reverse.py:216); truncation makes every cotangent NaN (reference _primitive.py:586-594)."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs

pytestmark = pytest.mark.gpu
GTOL = 1e-4


def _sync():
    import torch
    torch.cuda.synchronize()


def _np(x):
    return x.cpu().numpy()


def _mapped(cfg, **opts):
    return tm.vmap(cfg["item"], outputs=cfg["outputs"], in_axes=cfg["in_axes"], max_steps=cfg["max_steps"], **opts)


def test_c1_grad_theta(oracle):
    """d(hist.sum())/d theta: one adjoint launch (tm.grad) against the oracle and the closed form hist.sum()/theta."""
    print("case: C1 grad theta N=10000", flush=True)
    xs, keys, theta = configs.c1_inputs()
    g = tm.grad(_mapped(configs.C1), argnums=2)(xs, keys, theta)
    _sync()
    got = float(_np(g))
    want, ntr = oracle.c1_grad(xs, keys, theta, np.ones(16, np.float32))
    assert ntr == 0
    assert abs(got - float(want)) <= GTOL * abs(float(want))
    ref = oracle.c1_fwd(xs, keys, theta)
    closed = ref.tallies64["hist"].sum() / float(theta)
    assert abs(got - closed) <= GTOL * abs(closed)


@pytest.mark.parametrize("C", [16, 4, 2, 1])
def test_c1_grad_xs_and_checkpoint_independence(oracle, C):
    """cotangents of xs (per item, through the loop state: the checkpointed replay) and of theta with weights ct;
    C = 1, 2, 4 force the replay and the K > C^2 branch; per-item results bitwise equal to C = 16."""
    print(f"case: C1 vjp (xs, theta) C={C}", flush=True)
    xs, keys, theta = configs.c1_inputs()
    ct = np.linspace(0.5, 2.0, 16).astype(np.float32)
    res, pull = tm.vjp(_mapped(configs.C1, rev_checkpoints=C), xs, keys, theta, argnums=(0, 2))
    gx, gth = pull({"hist": ct})
    _sync()
    want_th, want_x, ntr = oracle.c1_grad(xs, keys, theta, ct, per_item=True)
    gx = _np(gx)
    assert abs(float(_np(gth)) - float(want_th)) <= GTOL * abs(float(want_th))
    err = np.abs(gx - want_x) / np.maximum(np.abs(want_x), 1.0)
    assert err.max() <= GTOL, err.max()
    if C != 16:
        _, pull16 = tm.vjp(_mapped(configs.C1), xs, keys, theta, argnums=(0, 2))
        gx16, _ = pull16({"hist": ct})
        _sync()
        assert np.array_equal(gx.view(np.uint32), _np(gx16).view(np.uint32))


def test_c1_grad_truncation_is_nan(oracle):
    print("case: C1 grad max_steps=3", flush=True)
    xs, keys, theta = configs.c1_inputs()
    g = tm.grad(_mapped(dict(configs.C1, max_steps=3)), argnums=2)(xs, keys, theta)
    _sync()
    assert np.isnan(float(_np(g)))


def test_c2_grad_drift_is_exactly_zero(oracle):
    """the emitted values are constants: the pathwise gradient w.r.t. drift (and x0) is exactly 0."""
    print("case: C2 grad drift N=65536", flush=True)
    x0, keys, drift = configs.c2_inputs(65_536)
    f = _mapped(configs.C2)
    g = tm.grad(f, argnums=2)(x0, keys, drift)
    _sync()
    want, ntr = oracle.c2_grad(x0, keys, drift, np.ones(128, np.float32), np.ones(2, np.float32))
    assert float(_np(g)) == float(want) == 0.0
    res, pull = tm.vjp(f, x0, keys, drift, argnums=(0, 2))
    gx, gd = pull({"occ": 1.0, "wall": 1.0})
    _sync()
    assert float(_np(gd)) == 0.0 and not np.any(_np(gx))


def test_c2_grad_full_size():
    print("case: C2 grad drift N=4194304", flush=True)
    x0, keys, drift = configs.c2_inputs()
    g = tm.grad(_mapped(configs.C2), argnums=2)(x0, keys, drift)
    _sync()
    assert float(_np(g)) == 0.0


def test_no_stale_runtime_error_after_launches():
    """a forward launch and both adjoint kinds leave no pending runtime error for the framework's next call (the
    launch library clears the errors of its optional symbol lookups)."""
    import torch
    xs, keys, theta = configs.c1_inputs(512)
    f = _mapped(configs.C1)
    f(xs, keys, theta)
    tm.grad(f, argnums=2)(xs, keys, theta)                         # forward-only adjoint
    tm.vjp(f, xs, keys, theta, argnums=(0, 2))[1]({"hist": 1.0})   # checkpointed adjoint
    x = torch.full((8,), 2.0, device="cuda") * 3.0
    torch.cuda.synchronize()
    assert float(x.sum().item()) == 48.0
