"""jax.random for item code and for the host: threefry2x32 keys (uint32[2]) with JAX's partitionable layering
(jax_threefry_partitionable=True, the default since JAX 0.5), which the reference delegates to JAX's own PRNGImpl
(reference tallymap/_compat.py:119-154, backends/kernel/op_table.py:1664-1761):

  fold_in(k, d)      = threefry2x32(k; (0, uint32(d)))           (threefry_fold_in: threefry_2x32(k, seed(d)))
  split(k, n)[i]     = threefry2x32(k; (hi(i), lo(i)))           (iota_2x32_shape counters)
  bits(k, (n,))[i]   = o0 ^ o1 of threefry2x32(k; (hi(i), lo(i)))  (32-bit random_bits; shape () is i = 0)
  uniform(k, lo, hi) = max(lo, (bitcast((bits >> 9) | 0x3f800000) - 1) * (hi - lo) + lo)
  normal(k)          = float32(sqrt 2) * erf_inv(uniform(k, nextafter(-1, 0), 1))

Inside a traced item these bind `threefry2x32` (four uint32 scalars -> two) and ordinary lax primitives.  On host
(numpy) arrays of keys they run vectorised in numpy: the benchmarks build their inputs with them.
"""
import numpy as np

from . import _core as C

_ROT = (13, 15, 26, 6, 17, 29, 16, 24)


# ------------------------------------------------------------------------------------------ host (numpy)
def _tf_np(k0, k1, c0, c1):
    """threefry2x32, 20 rounds (Salmon et al. 2011), vectorised over uint32 numpy arrays."""
    k0, k1, c0, c1 = (np.asarray(a, np.uint32) for a in (k0, k1, c0, c1))
    ks = (k0, k1, k0 ^ k1 ^ np.uint32(0x1BD11BDA))
    with np.errstate(over="ignore"):
        x0 = c0 + ks[0]
        x1 = c1 + ks[1]
        for blk in range(5):
            for r in range(4):
                x0 = x0 + x1
                d = _ROT[(blk & 1) * 4 + r]
                x1 = (x1 << np.uint32(d)) | (x1 >> np.uint32(32 - d))
                x1 = x1 ^ x0
            x0 = x0 + ks[(blk + 1) % 3]
            x1 = x1 + ks[(blk + 2) % 3] + np.uint32(blk + 1)
    return x0.astype(np.uint32), x1.astype(np.uint32)


def PRNGKey(seed):
    """jax.random.PRNGKey(seed) for a 32-bit seed: (seed >> 32, seed & 0xFFFFFFFF) = (0, seed)."""
    s = int(seed)
    return np.array([(s >> 32) & 0xFFFFFFFF if s >= 0 else 0xFFFFFFFF, s & 0xFFFFFFFF], np.uint32)


def _host_split(key, num):
    key = np.asarray(key, np.uint32)
    i = np.arange(num, dtype=np.uint64)
    o0, o1 = _tf_np(key[..., 0:1], key[..., 1:2], (i >> np.uint64(32)).astype(np.uint32),
                    i.astype(np.uint32))
    return np.stack([o0, o1], axis=-1)


def _host_fold_in(keys, d):
    keys = np.asarray(keys, np.uint32)
    d = np.asarray(d).astype(np.uint32)
    o0, o1 = _tf_np(keys[..., 0], keys[..., 1], np.zeros_like(d), d)
    return np.stack([o0, o1], axis=-1)


def _host_bits(keys, shape=()):
    keys = np.asarray(keys, np.uint32)
    n = _count(shape)
    if n is None:
        z = np.zeros(keys.shape[:-1], np.uint32)
        o0, o1 = _tf_np(keys[..., 0], keys[..., 1], z, z)
        return o0 ^ o1
    i = np.arange(n, dtype=np.uint64)
    o0, o1 = _tf_np(keys[..., 0:1], keys[..., 1:2], (i >> np.uint64(32)).astype(np.uint32), i.astype(np.uint32))
    return o0 ^ o1


def _count(shape):
    """None for shape (), n for shape (n,); other shapes are refused."""
    shape = tuple(int(d) for d in shape)
    if shape == ():
        return None
    if len(shape) != 1:
        raise C.TraceError(f"random draws of shape {shape}: only () and (n,) are supported by this backend")
    return shape[0]


def _host_uniform(keys, minval, maxval, shape=()):
    lo, hi = np.float32(minval), np.float32(maxval)
    f = ((_host_bits(keys, shape) >> np.uint32(9)) | np.uint32(0x3F800000)).view(np.float32) - np.float32(1.0)
    span = np.float32(hi - lo)
    r = (f * span).astype(np.float32) + lo
    return np.maximum(lo, r).astype(np.float32)


# ------------------------------------------------------------------------------------------- traced
def _words(key):
    if key.shape != (2,) or key.dtype != C.U32:
        raise C.TraceError(f"a PRNG key must be uint32[2], got {key.aval}")
    return key[0], key[1]


def threefry2x32(k0, k1, c0, c1):
    ins = []
    for x in (k0, k1, c0, c1):
        if C.is_traced(x):
            ins.append((x if x.dtype == C.U32 else C.convert(x, C.U32)).var)
        else:
            ins.append(C.literal(int(x) & 0xFFFFFFFF, C.U32, weak=False))
    o0, o1 = C.bind("threefry2x32", ins, [C.AVal((), C.U32), C.AVal((), C.U32)])
    return o0, o1


def _u32(d):
    if C.is_traced(d):
        return d if d.dtype == C.U32 else C.convert(d, C.U32)
    return int(d) & 0xFFFFFFFF


def fold_in(key, data):
    if not C.is_traced(key):
        if C.is_traced(data):
            key = C.literal(np.asarray(key, np.uint32), C.U32)
            raise C.TraceError("fold_in of a constant key with traced data: pass the key as an argument")
        return _host_fold_in(key, data)
    d = _u32(data)                # (converted before the key is read, in the order jax.random.fold_in binds them)
    k0, k1 = _words(key)
    o0, o1 = threefry2x32(k0, k1, 0, d)
    return C.stack([o0, o1])


def split(key, num=2):
    if not C.is_traced(key):
        return _host_split(key, num)
    k0, k1 = _words(key)
    rows = []
    for i in range(int(num)):
        o0, o1 = threefry2x32(k0, k1, (i >> 32) & 0xFFFFFFFF, i & 0xFFFFFFFF)
        rows.append(C.stack([o0, o1]))
    return C.stack(rows)


def bits(key, shape=()):
    if not C.is_traced(key):
        return _host_bits(key, shape)
    n = _count(shape)
    k0, k1 = _words(key)
    if n is None:
        o0, o1 = threefry2x32(k0, k1, 0, 0)
        return o0 ^ o1
    out = []
    for i in range(n):
        o0, o1 = threefry2x32(k0, k1, (i >> 32) & 0xFFFFFFFF, i & 0xFFFFFFFF)
        out.append(o0 ^ o1)
    return C.stack(out)


def _unit(b, lo, hi):
    """uniform's float32 arithmetic on one traced uint32 scalar of bits."""
    fb = (b >> 9) | np.uint32(0x3F800000)
    f = C.bind("bitcast_convert_type", [fb.var], [C.AVal((), C.F32)], new_dtype=C.F32)[0] - np.float32(1.0)
    span = np.float32(hi - lo)          # maxval - minval, in float32
    r = f * span + lo
    return C.binop("max", lo, r)


def uniform(key, shape=(), dtype=np.float32, minval=0.0, maxval=1.0):
    if np.dtype(dtype) != C.F32:
        raise C.TraceError("uniform: only float32 draws are supported by this backend")
    n = _count(shape)
    if not C.is_traced(key):
        return _host_uniform(key, minval, maxval, shape)
    lo, hi = np.float32(minval), np.float32(maxval)
    b = bits(key, shape)
    if n is None:
        return _unit(b, lo, hi)
    return C.stack([_unit(b[i], lo, hi) for i in range(n)])


def normal(key, shape=(), dtype=np.float32):
    if np.dtype(dtype) != C.F32:
        raise C.TraceError("normal: only float32 draws are supported by this backend")
    if not C.is_traced(key):
        raise C.TraceError("normal: host draws are not provided (erf_inv has no host restatement here)")
    n = _count(shape)
    lo = np.nextafter(np.float32(-1.0), np.float32(0.0))
    u = uniform(key, shape, np.float32, lo, np.float32(1.0))
    if n is None:
        return np.float32(np.sqrt(2)) * C.unop("erf_inv", u, float_only=True)
    return C.stack([np.float32(np.sqrt(2)) * C.unop("erf_inv", u[i], float_only=True) for i in range(n)])
