"""Device utility passes of the spawn paths: an exclusive prefix sum of int32 counts and the scatter of a
generation's rows into canonical (parent, ordinal) order.

One hipRTC module (`tm_util`), registered once, its entries launched through `tm_launch_aux` on torch's current
stream like a program's auxiliary passes (one by-value struct of buffer pointers, the element count as n_items):

  tm_xscan_local   block of 1024: exclusive prefix sums of counts[i] (int32) within the block -> out[i] (int64),
                   the block's total -> tot[b]
  tm_xscan_top     one block: exclusive prefix sums of the block totals, in place, 1024 at a time with a carry
  tm_xscan_add     out[i] += tot[i / 1024]
  tm_tree_scatter  row r of a generation's children goes to row off[par[r]] + ord[r] (the parent's first child plus
                   the child's ordinal); rows of u32 words, their count in a one-word buffer (tm_tree_scatter_b:
                   rows of bytes, for operands of 1- or 2-byte elements)

The reference computes the same order with jnp sorts in `_api._tree_order` (`_api.py:783-805`) and the offsets with
`_limits.offsets`; here they are linear passes because a generation's parents are already in canonical order.
"""
import threading

from . import compile as Cm

SCAN_BLOCK = 1024
_MOD = {}
_LOCK = threading.Lock()


def _source():
    return "\n".join([Cm.prelude(), "struct TmParams { void* p[6]; };", r'''
// (the loader requires a main entry; nothing launches it)
extern "C" __global__ void tm_main(const TmParams P, const i64 n_items) {}

extern "C" __global__ void __launch_bounds__(1024) tm_xscan_local(const TmParams P, const i64 n_items) {
  __shared__ i64 s[1024];
  const i64 i = (i64)blockIdx.x * 1024 + threadIdx.x;
  const i64 v = i < n_items ? (i64)((const i32*)P.p[0])[i] : 0;
  s[threadIdx.x] = v;
  __syncthreads();
  for (u32 d = 1; d < 1024u; d <<= 1) {
    const i64 a = threadIdx.x >= d ? s[threadIdx.x - d] : 0;
    __syncthreads();
    s[threadIdx.x] += a;
    __syncthreads();
  }
  if (i < n_items) ((i64*)P.p[1])[i] = s[threadIdx.x] - v;
  if (threadIdx.x == 1023u) ((i64*)P.p[2])[blockIdx.x] = s[1023];
}

extern "C" __global__ void __launch_bounds__(1024) tm_xscan_top(const TmParams P, const i64 n_items) {
  __shared__ i64 s[1024];
  __shared__ i64 carry;
  i64* const tot = (i64*)P.p[2];
  const i64 nb = (n_items + 1023) / 1024;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (i64 base = 0; base < nb; base += 1024) {
    const i64 i = base + threadIdx.x;
    const i64 v = i < nb ? tot[i] : 0;
    s[threadIdx.x] = v;
    __syncthreads();
    for (u32 d = 1; d < 1024u; d <<= 1) {
      const i64 a = threadIdx.x >= d ? s[threadIdx.x - d] : 0;
      __syncthreads();
      s[threadIdx.x] += a;
      __syncthreads();
    }
    const i64 c = carry;
    if (i < nb) tot[i] = c + s[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 1023u) carry = c + s[1023];
    __syncthreads();
  }
}

extern "C" __global__ void __launch_bounds__(1024) tm_xscan_add(const TmParams P, const i64 n_items) {
  const i64 i = (i64)blockIdx.x * 1024 + threadIdx.x;
  if (i < n_items) ((i64*)P.p[1])[i] += ((const i64*)P.p[2])[i / 1024];
}

extern "C" __global__ void __launch_bounds__(256) tm_tree_scatter(const TmParams P, const i64 n_items) {
  const i64* const off = (const i64*)P.p[0];
  const i32* const par = (const i32*)P.p[1];
  const i32* const ord = (const i32*)P.p[2];
  const u32* const src = (const u32*)P.p[3];
  u32* const dst = (u32*)P.p[4];
  const i64 w = ((const i64*)P.p[5])[0];
  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, st = (i64)gridDim.x * blockDim.x;
  for (i64 e = g; e < n_items * w; e += st) {
    const i64 r = e / w, k = e - r * w;
    const i64 d = off[par[r]] + (i64)ord[r];
    dst[d * w + k] = src[e];
  }
}

extern "C" __global__ void __launch_bounds__(256) tm_tree_scatter_b(const TmParams P, const i64 n_items) {
  const i64* const off = (const i64*)P.p[0];
  const i32* const par = (const i32*)P.p[1];
  const i32* const ord = (const i32*)P.p[2];
  const u8* const src = (const u8*)P.p[3];
  u8* const dst = (u8*)P.p[4];
  const i64 w = ((const i64*)P.p[5])[0];
  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, st = (i64)gridDim.x * blockDim.x;
  for (i64 e = g; e < n_items * w; e += st) {
    const i64 r = e / w, k = e - r * w;
    const i64 d = off[par[r]] + (i64)ord[r];
    dst[d * w + k] = src[e];
  }
}
'''])


def _module():
    """the registered module id (compiled once per process; the disk cache keeps the code object)."""
    with _LOCK:
        kid = _MOD.get("id")
        if kid is None:
            src = _source()
            img = Cm.code_object(src, name="tm_util.hip")
            kid = int(Cm._key(src)[:15], 16)
            Cm.check(Cm.lib().tm_register(kid, img, len(img), b"tm_util"))
            _MOD["id"] = kid
        return kid


def _aux(name, bufs, n, grid, block):
    import ctypes

    import torch
    ptrs = [b.data_ptr() for b in bufs] + [0] * (6 - len(bufs))
    arr = (ctypes.c_void_p * 6)(*ptrs)
    s = torch.cuda.current_stream().cuda_stream
    Cm.check(Cm.lib().tm_launch_aux(_module(), name.encode(), ctypes.c_void_p(s), arr, 6, int(n), int(grid), block))


def exclusive_scan(counts):
    """int32 counts [n] (device) -> their exclusive prefix sums as int64 [n], on torch's current stream."""
    import torch
    n = int(counts.shape[0])
    out = torch.empty((n,), dtype=torch.int64, device="cuda")
    if n == 0:
        return out
    nb = -(-n // SCAN_BLOCK)
    tot = torch.empty((nb,), dtype=torch.int64, device="cuda")
    c = counts.contiguous().view(torch.int32)
    _aux("tm_xscan_local", [c, out, tot], n, nb, SCAN_BLOCK)
    _aux("tm_xscan_top", [c, out, tot], n, 1, SCAN_BLOCK)
    _aux("tm_xscan_add", [c, out, tot], n, nb, SCAN_BLOCK)
    return out


def tree_scatter(off, par, ordn, src, dst, m):
    """dst rows [off[par[r]] + ordn[r]] = src rows [r] for r < m (rows: the trailing dims of src / dst, whole u32
    words; off int64 per parent, par / ordn int32 per child)."""
    import torch
    if m == 0:
        return
    rb = src[0].numel() * src.element_size()
    if dst.element_size() * dst[0].numel() != rb:
        raise Cm.BackendError(f"internal: tree_scatter of {rb}-byte rows into other rows")
    wd = rb // 4 if rb % 4 == 0 else rb
    w = torch.tensor([wd], dtype=torch.int64, device="cuda")
    grid = max(1, min(-(-m * wd // 256), 65536))
    _aux("tm_tree_scatter" if rb % 4 == 0 else "tm_tree_scatter_b", [off, par, ordn, src, dst, w], m, grid, 256)
