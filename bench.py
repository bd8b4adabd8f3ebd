"""Benchmark: items/s of the tallymap hot path (forward + replay gradient) on one MI355X.

Workload: BASELINE config 2, the 1-D random walk (C2) at N = 4,194,304 items, inputs resident in HBM.  One step is
one forward launch (occupancy and wall tallies, per-item trip counts) plus one replay-gradient launch (d sum(tallies)
/ d drift, exact float32), both queued on torch's current stream; `value` = N / (time per step).

roofline: the dominant kernel's algorithmic HBM bytes per launch (per item: x0 4 B + key 8 B read, trip count 4 B +
truncation flag 1 B written = 17 B; the gradient launch: 12 B read + 1 B written = 13 B) over its average launch
duration (HIP events on the launch stream), against MI355X's 8 TB/s.  The path is VALU-bound (threefry, erf_inv in
double), not HBM-bound: the fraction is reported as measured.  traffic: FETCH_SIZE + WRITE_SIZE per dispatch from
rocprofv3 counter runs, scaled by the same counters on a copy of known size (profiles/), when given with
--traffic-bytes; else null.
cpu_baseline: the oracle (the C/OpenMP restatement of the reference's CPU kernel backend) on the host's cores, on a
bounded sample of the same workload (the first items of the same inputs), forward + gradient, items/s.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FWD_BYTES_PER_ITEM = 17
GRAD_BYTES_PER_ITEM = 13


def cpu_baseline(x0, keys, drift, max_steps, target_s=10.0):
    """the oracle on a bounded sample: forward + forward-mode gradient, items/s."""
    import oracle as O
    O.build()
    threads = O.max_threads()
    n = 8192
    while True:
        t0 = time.perf_counter()
        O.c2_fwd(x0[:n], keys[:n], drift, max_steps=max_steps, shadow=False, per_item=True)
        O.c2_grad(x0[:n], keys[:n], drift, np.ones(128, np.float32), np.ones(2, np.float32), max_steps=max_steps)
        dt = time.perf_counter() - t0
        if dt * 4 > target_s or n * 2 > x0.size:
            break
        n = min(x0.size, max(n * 2, int(n * target_s / max(dt, 1e-3) / 2)))
    return dict(value=n / dt, unit="items/s", cores=threads, kind="port",
                sample=f"first {n} of the N=4,194,304 C2 items, forward + gradient (drift), {dt:.2f} s wall "
                       f"on {threads} OpenMP threads")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=4_194_304)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--traffic-bytes", type=float, default=None,
                    help="HBM bytes per dominant-kernel launch measured with rocprofv3 (profiles/)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {a.gpus}): items shard contiguously over "
              "GPUs with one all-reduce of the tallies, which is designed but not built", file=sys.stderr)
        sys.exit(2)
    import torch

    import tallymap_amd as tm
    from tallymap_amd import backend as B
    from tallymap_amd import configs
    cfg = configs.C2
    x0, keys, drift = configs.c2_inputs(a.n)
    dev = [torch.from_numpy(x0).cuda(), torch.from_numpy(keys).cuda(), torch.tensor(drift).cuda()]
    f = tm.vmap(cfg["item"], outputs=cfg["outputs"], in_axes=cfg["in_axes"], max_steps=cfg["max_steps"])
    g = tm.grad(f, argnums=2)
    stream = torch.cuda.current_stream()

    def step(ev=None):
        if ev:
            ev[0].record(stream)
        r = f(*dev)
        if ev:
            ev[1].record(stream)
        gr = g(*dev)
        if ev:
            ev[2].record(stream)
        return r, gr
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        r, gr = step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    grad_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    ms = wall * 1e3 / a.steps
    N = a.n
    # sanity: the step computed what it should (no truncation, every item absorbed once, zero gradient)
    assert int(r.stats["n_truncated"].item()) == 0
    assert abs(float(r.outputs["wall"].sum().item()) - N) <= 1e-5 * N
    assert float(gr.item()) == 0.0
    dom = "forward" if fwd_ms >= grad_ms else "gradient"
    dom_ms = max(fwd_ms, grad_ms)
    bpi = FWD_BYTES_PER_ITEM if dom == "forward" else GRAD_BYTES_PER_ITEM
    achieved = bpi * N / (dom_ms * 1e-3) / 1e9
    pi = B.compiled(f._prepare(dev)[0], f._opts)
    info = B.kernel_info(pi)
    out = {
        "metric": "items/s fwd+grad at N=4,194,304 (C2 random walk)",
        "value": N / (ms * 1e-3),
        "unit": "items/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded threefry keys, x0 ~ U(0.2, 0.8))",
        "config": {"workload": "C2: 1-D random walk, N=4,194,304, forward + replay gradient w.r.t. drift",
                   "n_items": N, "max_steps": cfg["max_steps"], "parallelism": "single GPU"},
        "fwd_items_per_s": N / (fwd_ms * 1e-3),
        "grad_items_per_s": N / (grad_ms * 1e-3),
        "fwd_ms": fwd_ms,
        "grad_ms": grad_ms,
        "mean_trip_count": float(r.per_item.double().mean().item()),
        "kernel": {"name": "tm_main (" + dom + ")", **info},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": a.traffic_bytes,
                     "algorithmic_bytes_per_launch": bpi * N},
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x0, keys, drift, cfg["max_steps"])
    print(json.dumps(out))


if __name__ == "__main__":
    main()
