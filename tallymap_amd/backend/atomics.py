"""Atomic-throughput microbenchmarks: the denominators of the emit rooflines (MI355X publishes no atomic peak).

Each pattern is a module with the kernel template's entry names (tm_zero, tm_main), registered and launched through
libtallymap_rocm.so like a program: a grid-stride loop where thread g performs `per` atomic adds, then (LDS
patterns) one flush of its block's bins.  The patterns are the ones the generated kernels issue:

  lds_f32_128     ds_add_f32 onto 128 LDS bins (a privatised f32 tally, C2's occupancy histogram)
  lds_u64_128     ds_add_u64 onto 128 LDS words (the exact accumulator's words)
  glb_f32_dist    global_atomic_add_f32, every add to its own address (per-item tallies: C4, C5)
  glb_f32_128     global_atomic_add_f32 onto 128 addresses (an unprivatised small tally)
  glb_f32_1       global_atomic_add_f32 onto 1 address (full contention)
  glb_claim_1     one returning u64 add per wave onto 1 address (tm_claim: the item, Records-batch and spawn-ticket
                  claims); its rate is claims (wave instructions) per second

The adds are of 1.0 (f32) or 1 (u64), so the totals are checkable: `run` returns adds per second and whether the
buffer holds exactly the number of adds issued.
"""
import numpy as np

from . import compile as Cm

PATTERNS = ("lds_f32_128", "lds_u64_128", "glb_f32_dist", "glb_f32_128", "glb_f32_1", "glb_claim_1")


def source(pattern, per):
    """HIP source of one pattern: P.p[0] = the bins (f32 or u64), P.p[1] = ctl (claim-free: unused)."""
    head = [Cm.prelude(), "struct TmParams { void* p[2]; };"]
    zero = ("extern \"C\" __global__ void tm_zero(const TmParams P, const i64 n_items) {\n"
            "  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, s = (i64)gridDim.x * blockDim.x;\n"
            "  const i64 nw = %s;\n"
            "  for (i64 i = g; i < nw; i += s) ((u32*)P.p[0])[i] = 0u;\n}")
    if pattern == "lds_f32_128":
        body = f"""
  __shared__ float sh[128];
  for (int i = threadIdx.x; i < 128; i += blockDim.x) sh[i] = 0.0f;
  __syncthreads();
  const u32 g = blockIdx.x * blockDim.x + threadIdx.x;
  for (u32 k = 0; k < {per}u; ++k) atomicAdd(&sh[(g + k * 7u) & 127u], 1.0f);
  __syncthreads();
  for (int i = threadIdx.x; i < 128; i += blockDim.x) atomicAdd(&((float*)P.p[0])[i], sh[i]);"""
        nw = "128"
    elif pattern == "lds_u64_128":
        body = f"""
  __shared__ u64 sh[128];
  for (int i = threadIdx.x; i < 128; i += blockDim.x) sh[i] = 0ull;
  __syncthreads();
  const u32 g = blockIdx.x * blockDim.x + threadIdx.x;
  for (u32 k = 0; k < {per}u; ++k) atomicAdd(&sh[(g + k * 7u) & 127u], 1ull);
  __syncthreads();
  for (int i = threadIdx.x; i < 128; i += blockDim.x) atomicAdd(&((u64*)P.p[0])[i], sh[i]);"""
        nw = "256"
    elif pattern == "glb_f32_dist":
        body = f"""
  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, s = (i64)gridDim.x * blockDim.x;
  for (u32 k = 0; k < {per}u; ++k) atomicAdd(&((float*)P.p[0])[g + (i64)k * s], 1.0f);"""
        nw = f"n_items * {per}"
    elif pattern == "glb_f32_128":
        body = f"""
  const u32 g = blockIdx.x * blockDim.x + threadIdx.x;
  for (u32 k = 0; k < {per}u; ++k) atomicAdd(&((float*)P.p[0])[(g + k * 7u) & 127u], 1.0f);"""
        nw = "128"
    elif pattern == "glb_f32_1":
        body = f"""
  for (u32 k = 0; k < {per}u; ++k) atomicAdd(&((float*)P.p[0])[0], 1.0f);"""
        nw = "128"                                  # the whole buffer (bins 1..127 stay 0)
    elif pattern == "glb_claim_1":
        body = f"""
  u64 acc = 0ull;
  for (u32 k = 0; k < {per}u; ++k) acc += tm_claim((u64*)P.p[0], 1u);
  if (acc == ~0ull) ((u64*)P.p[0])[1] = acc;        // (never: keeps the claims' results live)"""
        nw = "256"
    else:
        raise ValueError(pattern)
    main = ("extern \"C\" __global__ void __launch_bounds__(256) tm_main(const TmParams P, const i64 n_items) {"
            + body + "\n}")
    return "\n".join(head + [zero % nw, main])


PER = {"glb_f32_1": 16, "glb_claim_1": 256}       # one address: f32 counts stay exact below 2^24


def run(pattern, per=None, reps=5):
    """-> dict(adds_per_s, adds, exact): the pattern's atomic adds per second (median of reps launches, HIP events on
    torch's current stream) on a full persistent grid (256 threads x blocks per CU x CUs, per adds each, default
    1024; 16 onto a single address)."""
    per = int(per or PER.get(pattern, 1024))
    import ctypes

    import torch

    from . import Compiled, kernel_info
    src = source(pattern, per)
    img = Cm.code_object(src, name=f"tm_atomics_{pattern}.hip")
    kid = int(Cm._key(src)[:15], 16)
    Cm.check(Cm.lib().tm_register(kid, img, len(img), f"atomics {pattern}".encode()))
    c = Compiled(kid, None, 256, src, pattern)
    lanes = kernel_info(c)["resident_threads"]
    adds = (lanes // 64 if pattern == "glb_claim_1" else lanes) * per
    n_items = lanes                 # sizes the grid: ceil(lanes / 256) blocks, the persistent grid
    if pattern == "glb_f32_dist":
        buf = torch.empty(adds, dtype=torch.float32, device="cuda")
    elif pattern in ("lds_u64_128", "glb_claim_1"):
        buf = torch.empty(128, dtype=torch.int64, device="cuda")
    else:
        buf = torch.empty(128, dtype=torch.float32, device="cuda")
    ctl = torch.zeros(8, dtype=torch.int32, device="cuda")
    arr = (ctypes.c_void_p * 2)(buf.data_ptr(), ctl.data_ptr())
    s = torch.cuda.current_stream()

    def launch():
        Cm.check(Cm.lib().tm_launch(kid, ctypes.c_void_p(s.cuda_stream), arr, 2, 1, 0, n_items, 256))
    launch()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        launch()
        e1.record(s)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3)
    total = float(buf.double().sum().item())
    return dict(adds_per_s=adds / float(np.median(ts)), adds=adds, exact=total == adds, total=total)
