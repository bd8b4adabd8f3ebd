"""jax.numpy for item code: the subset the item programs use, with jax.numpy's semantics (ufuncs lower to the lax
primitives of the same name; jnp.where is lax.select_n; jnp.clip is maximum then minimum, as jax.numpy.clip)."""
import numpy as _np

from . import _core as C
from . import lax as _lax

float32, float64, int32, uint32, int64, uint32, bool_, uint8 = (_np.float32, _np.float64, _np.int32, _np.uint32,
                                                              _np.int64, _np.uint32, _np.bool_, _np.uint8)
pi = _np.pi
e = _np.e
inf = _np.inf
nan = _np.nan

exp, log, log1p, expm1 = _lax.exp, _lax.log, _lax.log1p, _lax.expm1
sin, cos, tan, tanh = _lax.sin, _lax.cos, _lax.tan, _lax.tanh
sqrt, floor, ceil = _lax.sqrt, _lax.floor, _lax.ceil
arctan2 = _lax.atan2
exp2, log2 = _lax.exp2, _lax.log2
arctan, arcsin, arccos = _lax.atan, _lax.asin, _lax.acos
sinh, cosh, arcsinh, arccosh, arctanh = _lax.sinh, _lax.cosh, _lax.asinh, _lax.acosh, _lax.atanh
cbrt, nextafter, isfinite = _lax.cbrt, _lax.nextafter, _lax.is_finite


def asarray(x, dtype=None):
    if C.is_traced(x):
        return x if dtype is None else C.convert(x, dtype)
    return _np.asarray(x, dtype)


def where(cond, x, y):
    return C.select(cond, x, y)


def maximum(a, b):
    return C.binop("max", a, b)


def minimum(a, b):
    return C.binop("min", a, b)


def abs(x):             # noqa: A001
    return C.unop("abs", x)


absolute = abs


def sign(x):
    return C.unop("sign", x)


def clip(x, a_min=None, a_max=None):
    if a_min is not None:
        x = maximum(a_min, x)
    if a_max is not None:
        x = minimum(a_max, x)
    return x


def square(x):
    return C.bind("integer_pow", [x.var], [x.aval], y=2)[0]


def power(a, b):
    return C.power(a, b)


def logical_and(a, b):
    return C.binop("and", a, b)


def logical_or(a, b):
    return C.binop("or", a, b)


def logical_not(a):
    return C.unop("not", a)


def stack(xs):
    return C.stack(xs)


def array(xs, dtype=None):
    if any(C.is_traced(x) for x in xs):
        r = C.stack(xs)
        return r if dtype is None else C.convert(r, dtype)
    return _np.array(xs, dtype)


def sum(x):             # noqa: A001
    return C.reduce_sum(x) if C.is_traced(x) else _np.sum(x)


def max(x):             # noqa: A001
    """the largest element of a small array: lax.max folded left to right (NaN-propagating, as XLA's reduce_max;
    its derivative goes through lax.max's rule, pairwise at ties)."""
    if not C.is_traced(x):
        return _np.max(x)
    if not x.shape:
        return x
    acc = x[0]
    for i in range(1, x.shape[0]):
        acc = C.binop("max", acc, x[i])
    return acc


def min(x):             # noqa: A001
    """the smallest element (lax.min folded left to right)."""
    if not C.is_traced(x):
        return _np.min(x)
    if not x.shape:
        return x
    acc = x[0]
    for i in range(1, x.shape[0]):
        acc = C.binop("min", acc, x[i])
    return acc


def _arg(x, better):
    best, idx = x[0], C.literal(0, C.I32, weak=False)
    for i in range(1, x.shape[0]):
        v = x[i]
        take = better(v, best)
        if _np.issubdtype(x.dtype, _np.floating):      # the first NaN wins, as jnp.argmin / argmax
            take = C.binop("or", take, C.binop("and", C.binop("ne", v, v), C.binop("eq", best, best)))
        best = C.select(take, v, best)
        idx = C.select(take, C.literal(i, C.I32, weak=False), idx)
    return idx


def argmin(x):
    """the index (int32) of the first smallest element of a small 1-d array; a NaN counts as the smallest."""
    if not C.is_traced(x):
        return _np.int32(_np.argmin(x))
    if len(x.shape) != 1:
        raise C.TraceError("argmin of an item value: 1-d arrays only")
    return _arg(x, lambda v, b: C.binop("lt", v, b))


def argmax(x):
    """the index (int32) of the first largest element of a small 1-d array; a NaN counts as the largest."""
    if not C.is_traced(x):
        return _np.int32(_np.argmax(x))
    if len(x.shape) != 1:
        raise C.TraceError("argmax of an item value: 1-d arrays only")
    return _arg(x, lambda v, b: C.binop("gt", v, b))


def arange(*a, dtype=None):
    """a constant range (numpy's): an index array for t.add, say."""
    return _np.arange(*a, dtype=dtype)


def cumsum(x):
    """the running sums of a small 1-d array, left to right."""
    if not C.is_traced(x):
        return _np.cumsum(x)
    if len(x.shape) != 1:
        raise C.TraceError("cumsum of an item value: 1-d arrays only")
    acc = [x[0]]
    for i in range(1, x.shape[0]):
        acc.append(acc[-1] + x[i])
    return C.stack(acc)


def dot(a, b):
    """the dot product of two small vectors: (a0 b0 + a1 b1) + ..., left to right."""
    acc = a[0] * b[0]
    for i in range(1, a.shape[0]):
        acc = acc + a[i] * b[i]
    return acc


def zeros_like(x):
    return x * 0


def int32_(x):
    return C.convert(x, C.I32)
