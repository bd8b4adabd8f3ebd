"""Fill invariance (reference tests/reverse.py:1262): results do not depend on what the buffers the backend allocates
held before the call.  Every tensor the backend allocates (results, scratch, tapes, the spawn queues, the Records
buffers) is filled with 0x00 bytes in one run and with 0xFF bytes in another; forward, value_and_grad, the tape
adjoint (state and residual tapes), jvp, Records and a spawning call then give the same outputs: bitwise, but for
summed float32 outputs, whose atomic adds land in a different order in every run."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import configs

pytestmark = pytest.mark.gpu


def _fill(t, byte):
    import torch
    if t.is_cuda and t.numel() and t.is_contiguous():
        t.view(-1).view(torch.uint8).fill_(byte)
    return t


def _filled(orig, byte):
    """torch.empty / torch.empty_like whose new CUDA tensors are filled with `byte`"""
    return lambda *a, **k: _fill(orig(*a, **k), byte)


def _host(x):
    """every array of a nested result, on the host"""
    import torch
    if isinstance(x, torch.Tensor):
        return [x.detach().cpu().numpy().copy()]
    if isinstance(x, dict):
        return [b for k in sorted(x) for b in _host(x[k])]
    if isinstance(x, (list, tuple)):
        return [b for v in x for b in _host(v)]
    if x is None:
        return []
    return [np.atleast_1d(np.asarray(x)).copy()]


def _same(x, y):
    """bitwise, except float arrays: a summed float32 output is a sum of atomic adds whose order varies from run to
    run, so floats agree to 1e-6 relative (an uncleared buffer would show as NaN or garbage, far beyond it); the
    exact outputs, gradients (exact sums), per-item results and integers are bitwise"""
    if x.dtype != y.dtype or x.shape != y.shape:
        return False
    if x.dtype.kind == "f":
        return bool(np.allclose(x, y, rtol=1e-6, atol=1e-30, equal_nan=True))
    return bool(np.array_equal(x, y))


def _calls():
    from test_gpu_records import _outputs, _walker
    from test_gpu_spawn import NZ, TH, _particle, _roots
    c1 = configs.C1
    f1 = tm.vmap(c1["item"], outputs=c1["outputs"], in_axes=c1["in_axes"], max_steps=c1["max_steps"])
    xs, keys, theta = configs.c1_inputs(4096)
    c3 = configs.C3
    f3 = tm.vmap(c3["item"], outputs=c3["outputs"], in_axes=c3["in_axes"], max_steps=c3["max_steps"])
    k3, mu = configs.c3_inputs(1 << 14)
    fr = tm.vmap(_walker, outputs=_outputs(1 << 16, 1 << 13), in_axes=(0, 0, None), max_steps=100)
    fs = tm.vmap(_particle, outputs={"dep": tm.Sum((NZ,), fixed_point=True), "count": tm.Sum((NZ,), np.int32)},
                 in_axes=(0, None), spawn=tm.Queue(1 << 14))
    roots, th = _roots(512), np.array(TH, np.float32)
    ct = np.linspace(0.5, 2.0, 16).astype(np.float32)
    return [
        ("c1 forward", lambda: f1(xs, keys, theta)),
        ("c1 value_and_grad theta", lambda: tm.value_and_grad(f1, argnums=2)(xs, keys, theta)),
        ("c1 vjp xs (state tape)", lambda: tm.vjp(f1, xs, keys, theta, argnums=(0, 2))[1]({"hist": ct})),
        ("c1 vjp xs (residual tape)",
         lambda: tm.vjp(tm.vmap(c1["item"], outputs=c1["outputs"], in_axes=c1["in_axes"], max_steps=c1["max_steps"],
                                rev_residual=True), xs, keys, theta, argnums=(0, 2))[1]({"hist": ct})),
        ("c3 grad mu_a", lambda: tm.grad(f3, argnums=1)(k3, mu)),
        ("c1 jvp theta", lambda: tm.jvp(f1, (xs, keys, theta), (None, None, np.float32(1.0)))),
        ("records walker", lambda: fr(xs, keys, theta)),
        ("spawn shower", lambda: fs(roots, th)),
    ]


def test_results_do_not_depend_on_the_allocations_fill(monkeypatch):
    import torch
    runs = {}
    for byte in (0x00, 0xFF):
        print(f"case: fill 0x{byte:02x}", flush=True)
        with monkeypatch.context() as m:
            m.setattr(torch, "empty", _filled(torch.empty, byte))
            m.setattr(torch, "empty_like", _filled(torch.empty_like, byte))
            out = {}
            for name, call in _calls():
                print(f"case: fill 0x{byte:02x} {name}", flush=True)
                r = call()
                torch.cuda.synchronize()
                out[name] = _host(r)
        runs[byte] = out
    for name in runs[0x00]:
        a, b = runs[0x00][name], runs[0xFF][name]
        assert len(a) == len(b), name
        for i, (x, y) in enumerate(zip(a, b)):
            assert _same(x, y), (name, i)
