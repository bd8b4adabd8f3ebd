"""The item program IR and its tracer.

JAX is not a dependency of this backend, so an item function is traced by a small tracer of its own into a
jaxpr-shaped IR: equations named by JAX's primitive names ("add", "threefry2x32", "while", "cond", ...) with
JAX's parameter names, over typed variables.  The emitter (backend/codegen.py) lowers this IR to HIP; an adapter
for real JAX jaxprs maps a ClosedJaxpr onto the same classes.

Semantics follow jax.numpy / lax where the reference relies on them (reference tallymap/_api.py:626 traces the item
with jax.make_jaxpr; backends/kernel/op_table.py emits each primitive):
  * weak types: a Python scalar takes the dtype of the typed operand it meets (int + f32 -> f32; 0 -> int32);
  * bool < integer < floating promotion of two typed operands; two different integer types or two different
    float types raise (the configs never mix them);
  * values are scalars or small static arrays (a key is uint32[2]); elementwise ops broadcast a scalar against
    an array.
"""
import itertools

import numpy as np

_ids = itertools.count()

F32, F64 = np.dtype(np.float32), np.dtype(np.float64)
I32, U32, I64, U64 = np.dtype(np.int32), np.dtype(np.uint32), np.dtype(np.int64), np.dtype(np.uint64)
BOOL = np.dtype(np.bool_)
U8 = np.dtype(np.uint8)


class TraceError(TypeError):
    pass


class AVal:
    __slots__ = ("shape", "dtype", "weak")

    def __init__(self, shape, dtype, weak=False):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.weak = bool(weak)

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def strong(self):
        return AVal(self.shape, self.dtype, False)

    def __eq__(self, o):
        return isinstance(o, AVal) and self.shape == o.shape and self.dtype == o.dtype

    def __hash__(self):
        return hash((self.shape, self.dtype))

    def __repr__(self):
        return f"{self.dtype.name}{list(self.shape)}{'~' if self.weak else ''}"


class Var:
    __slots__ = ("id", "aval")

    def __init__(self, aval):
        self.id = next(_ids)
        self.aval = aval

    def __repr__(self):
        return f"v{self.id}:{self.aval}"


class Lit:
    __slots__ = ("val", "aval")

    def __init__(self, val, aval):
        self.aval = aval
        self.val = np.asarray(val, aval.dtype).reshape(aval.shape)

    def __repr__(self):
        return f"{self.val!r}"


class Eqn:
    __slots__ = ("prim", "invars", "outvars", "params")

    def __init__(self, prim, invars, outvars, params):
        self.prim, self.invars, self.outvars, self.params = prim, list(invars), list(outvars), dict(params)

    def __repr__(self):
        ps = {k: v for k, v in self.params.items() if not isinstance(v, Jaxpr)}
        return f"{self.outvars} = {self.prim}{ps} {self.invars}"


class Jaxpr:
    """invars -> outvars through eqns.  Sub-programs of while / cond are Jaxprs too (closed: captured outer values
    are explicit leading invars, as JAX's cond_nconsts / body_nconsts)."""
    __slots__ = ("invars", "outvars", "eqns")

    def __init__(self, invars, outvars, eqns):
        self.invars, self.outvars, self.eqns = list(invars), list(outvars), list(eqns)

    def pretty(self, ind=0):
        p = " " * ind
        out = [f"{p}{{ lambda {self.invars} ."]
        for e in self.eqns:
            out.append(f"{p}  {e}")
            for k, v in e.params.items():
                if isinstance(v, Jaxpr):
                    out.append(f"{p}    {k}:")
                    out.append(v.pretty(ind + 6))
                elif isinstance(v, (list, tuple)) and v and all(isinstance(x, Jaxpr) for x in v):
                    for i, x in enumerate(v):
                        out.append(f"{p}    {k}[{i}]:")
                        out.append(x.pretty(ind + 6))
        out.append(f"{p}  in {self.outvars} }}")
        return "\n".join(out)


# --------------------------------------------------------------------------------------------- tracing
class Builder:
    """collects the equations of one (sub-)program.  A value of an enclosing builder used here is captured: it
    becomes one of this program's leading invars (self.captured lists the outer vars, in order)."""

    def __init__(self, parent=None):
        self.parent = parent
        self.eqns = []
        self.invars = []
        self.captured = []          # outer Vars captured, in order (Vars of the parent builder)
        self.cap_local = []         # the local Var standing for each of them
        self.env = {}               # outer Var -> local Var
        self.owned = set()          # ids of Vars defined in this builder

    def new_invar(self, aval):
        v = Var(aval)
        self.invars.append(v)
        self.owned.add(v.id)
        return v

    def local(self, var):
        """the Var to use here for `var` (capturing it from an enclosing builder if needed)."""
        if isinstance(var, Lit) or var.id in self.owned:
            return var
        if var.id in self.env:
            return self.env[var.id]
        if self.parent is None:
            raise TraceError("a value from another trace leaked into this item program")
        outer = self.parent.local(var)
        v = Var(var.aval)
        self.owned.add(v.id)
        self.captured.append(outer)
        self.cap_local.append(v)
        self.env[var.id] = v
        return v


_STACK = []


def current():
    if not _STACK:
        raise TraceError("tallymap_amd ops are only usable while an item function is being traced")
    return _STACK[-1]


class Tracer:
    """a traced value.  Arithmetic follows jax.numpy (see the module docstring)."""
    __slots__ = ("var",)
    __array_priority__ = 1000
    __array_ufunc__ = None          # numpy scalars defer to the reflected operators (np.float32(2) * tracer)

    def __init__(self, var):
        self.var = var

    aval = property(lambda s: s.var.aval)
    shape = property(lambda s: s.var.aval.shape)
    dtype = property(lambda s: s.var.aval.dtype)
    ndim = property(lambda s: len(s.var.aval.shape))
    size = property(lambda s: s.var.aval.size)

    def __repr__(self):
        return f"Tracer<{self.var.aval}>"

    def __bool__(self):
        raise TraceError("a traced value has no concrete truth value: use lax.cond / lax.while_loop / "
                         "jnp.where instead of Python control flow on it")

    __index__ = __int__ = __float__ = lambda s: (_ for _ in ()).throw(
        TraceError("a traced value cannot be converted to a Python number"))

    # arithmetic
    def __add__(s, o): return binop("add", s, o)
    def __radd__(s, o): return binop("add", o, s)
    def __sub__(s, o): return binop("sub", s, o)
    def __rsub__(s, o): return binop("sub", o, s)
    def __mul__(s, o): return binop("mul", s, o)
    def __rmul__(s, o): return binop("mul", o, s)
    def __truediv__(s, o): return true_divide(s, o)
    def __rtruediv__(s, o): return true_divide(o, s)
    def __floordiv__(s, o): return floor_divide(s, o)
    def __mod__(s, o): return remainder(s, o)
    def __pow__(s, o): return power(s, o)
    def __rpow__(s, o): return power(o, s)
    def __neg__(s): return unop("neg", s)
    def __pos__(s): return s
    def __abs__(s): return unop("abs", s)
    def __lt__(s, o): return binop("lt", s, o)
    def __le__(s, o): return binop("le", s, o)
    def __gt__(s, o): return binop("gt", s, o)
    def __ge__(s, o): return binop("ge", s, o)
    def __eq__(s, o): return binop("eq", s, o)
    def __ne__(s, o): return binop("ne", s, o)
    def __and__(s, o): return binop("and", s, o)
    def __rand__(s, o): return binop("and", o, s)
    def __or__(s, o): return binop("or", s, o)
    def __ror__(s, o): return binop("or", o, s)
    def __xor__(s, o): return binop("xor", s, o)
    def __rxor__(s, o): return binop("xor", o, s)
    def __invert__(s): return unop("not", s)
    def __lshift__(s, o): return binop("shift_left", s, o)
    def __rshift__(s, o):
        return binop("shift_right_logical" if np.issubdtype(s.dtype, np.unsignedinteger)
                     else "shift_right_arithmetic", s, o)
    __hash__ = object.__hash__

    def astype(self, dtype):
        return convert(self, dtype)

    def __getitem__(self, i):
        return getitem(self, i)

    def __iter__(self):
        if not self.shape:
            raise TraceError("iteration over a 0-d traced value")
        return (self[i] for i in range(self.shape[0]))

    def __len__(self):
        if not self.shape:
            raise TraceError("len() of a 0-d traced value")
        return self.shape[0]

    def sum(self):
        return reduce_sum(self)


def is_traced(x):
    return isinstance(x, Tracer)


def _pyscalar(x):
    return isinstance(x, (bool, int, float, np.bool_)) and not isinstance(x, np.ndarray)


def _np_scalar(x):
    return isinstance(x, np.generic) or (isinstance(x, np.ndarray) and x.ndim == 0)


def literal(x, dtype=None, weak=None):
    """a constant operand -> Lit (a Python scalar is weakly typed)."""
    if isinstance(x, Lit):
        return x
    if _pyscalar(x):
        if dtype is None:
            dtype = BOOL if isinstance(x, (bool, np.bool_)) else (I32 if isinstance(x, int) else F32)
        return Lit(x, AVal((), dtype, weak=True if weak is None else weak))
    a = np.asarray(x)
    if dtype is not None:
        a = a.astype(dtype)
    if a.dtype == F64 and dtype is None:
        a = a.astype(F32)              # (without x64, as JAX: a float64 constant is float32)
    if a.dtype == I64 and dtype is None:
        a = a.astype(I32)
    return Lit(a, AVal(a.shape, a.dtype, weak=bool(weak)))


def as_var(x):
    if isinstance(x, Tracer):
        return current().local(x.var)
    return literal(x)


def bind(prim, invars, outavals, **params):
    """append one equation to the current program -> its output Tracers."""
    b = current()
    ins = [current().local(v) if isinstance(v, Var) else v for v in invars]
    outs = [Var(a) for a in outavals]
    for o in outs:
        b.owned.add(o.id)
    b.eqns.append(Eqn(prim, ins, outs, params))
    return [Tracer(o) for o in outs]


# ----------------------------------------------------------------------------------------- typing rules
def _kind(dt):
    if dt == BOOL:
        return 0
    if np.issubdtype(dt, np.integer):
        return 1
    return 2


def result_type(*avals):
    """JAX's promotion for the operands' avals: weak operands adopt the strong dtype of their kind or above."""
    strong = [a for a in avals if not a.weak]
    weak = [a for a in avals if a.weak]
    if strong:
        kinds = {_kind(a.dtype) for a in strong}
        dts = {a.dtype for a in strong}
        top = max(kinds)
        cand = {d for d in dts if _kind(d) == top}
        if len(cand) > 1:
            raise TraceError(f"mixed dtypes {sorted(d.name for d in cand)}: convert explicitly")
        dt = cand.pop()
        wk = max((_kind(a.dtype) for a in weak), default=-1)
        if wk > top:                   # an int tracer meets a Python float: float32 (weakly typed)
            return F32, True
        return dt, False
    top = max(_kind(a.dtype) for a in weak)
    return ({0: BOOL, 1: I32, 2: F32}[top]), True


def _shape_of(*avals):
    shapes = {a.shape for a in avals if a.shape != ()}
    if len(shapes) > 1:
        raise TraceError(f"incompatible shapes {sorted(shapes)}")
    return shapes.pop() if shapes else ()


def _coerce(x, dt, weak):
    """operand x as dtype dt (Lits are re-typed; Tracers converted when their dtype differs)."""
    if isinstance(x, Tracer):
        if x.dtype != dt:
            return convert(x, dt, weak=weak).var
        return x.var
    if _pyscalar(x):       # a Python scalar takes the operation's dtype at full precision (JAX's weak typing)
        return Lit(np.asarray(x).astype(dt), AVal((), dt, weak=True))
    v = literal(x)
    return Lit(v.val.astype(dt), AVal(v.aval.shape, dt, weak=v.aval.weak))


_CMP = ("lt", "le", "gt", "ge", "eq", "ne")
_LOGIC = ("and", "or", "xor")


def binop(prim, a, b):
    if not (is_traced(a) or is_traced(b)):
        raise TraceError(f"{prim} of two constants: use numpy")
    aa, ab = _aval(a), _aval(b)
    dt, weak = result_type(aa, ab)
    if prim in _LOGIC and _kind(dt) == 2:
        raise TraceError(f"{prim} of floats")
    if prim.startswith("shift") and _kind(dt) != 1:
        raise TraceError(f"{prim} needs integers")
    shape = _shape_of(aa, ab)
    va, vb = _coerce(a, dt, weak), _coerce(b, dt, weak)
    out = AVal(shape, BOOL if prim in _CMP else dt, weak=(weak and prim not in _CMP))
    return bind(prim, [va, vb], [out])[0]


def _aval(x):
    if isinstance(x, Tracer):
        return x.aval
    if _pyscalar(x):       # (its value is converted once, to the operation's dtype: _coerce)
        return AVal((), BOOL if isinstance(x, (bool, np.bool_)) else (I32 if isinstance(x, int) else F32), True)
    return literal(x).aval


def unop(prim, a, float_only=False):
    if not is_traced(a):
        raise TraceError(f"{prim} of a constant: use numpy")
    if float_only and _kind(a.dtype) != 2:
        raise TraceError(f"{prim} needs a float operand, got {a.dtype}")
    if prim == "not" and _kind(a.dtype) == 2:
        raise TraceError("~ of a float")
    return bind(prim, [a.var], [AVal(a.shape, a.dtype, a.aval.weak)])[0]


def convert(x, dtype, weak=False):
    dtype = np.dtype(dtype)
    if not is_traced(x):
        return literal(np.asarray(x).astype(dtype), dtype)
    if x.dtype == dtype and x.aval.weak == weak:
        return x
    return bind("convert_element_type", [x.var], [AVal(x.shape, dtype, weak)], new_dtype=dtype, weak_type=weak)[0]


def _float_of(x):
    """x as a float operand (true division, transcendentals): integers become float32."""
    if is_traced(x):
        return x if _kind(x.dtype) == 2 else convert(x, F32)
    return x


def true_divide(a, b):
    if is_traced(a) and _kind(a.dtype) != 2 and (not is_traced(b) or _kind(b.dtype) != 2) \
            and not (isinstance(b, float)):
        a = convert(a, F32)
    if is_traced(b) and _kind(b.dtype) != 2 and not (is_traced(a) and _kind(a.dtype) == 2) \
            and not isinstance(a, float):
        b = convert(b, F32)
    return binop("div", a, b)


def floor_divide(a, b):
    """jnp.floor_divide (`//`) as JAX defines it, primitive for primitive: unsigned -> div; signed -> div, minus 1
    where the signs differ and the remainder is nonzero; float -> CPython's float_divmod (rem, div of the
    difference, a correction, then round half away from zero)."""
    dt, weak = result_type(_aval(a), _aval(b))
    k = _kind(dt)
    if k == 1 and np.issubdtype(dt, np.unsignedinteger):
        return binop("div", a, b)
    if k == 1:
        a, b = _coerce_t(a, dt, weak), _coerce_t(b, dt, weak)
        q = binop("div", a, b)
        fix = binop("and", binop("ne", unop("sign", a), unop("sign", b)), binop("ne", binop("rem", a, b), 0))
        return select(fix, q - 1, q)
    if k == 2:
        a, b = _coerce_t(a, dt, weak), _coerce_t(b, dt, weak)
        mod = binop("rem", a, b)
        div = binop("div", binop("sub", a, mod), b)
        ind = binop("and", binop("ne", mod, 0), binop("ne", unop("sign", b), unop("sign", mod)))
        div = select(ind, div - 1, div)
        return bind("round", [div.var], [div.aval], rounding_method=0)[0]
    raise TraceError(f"floor division of {dt}")


def remainder(a, b):
    """jnp.remainder (`%`) as JAX defines it: an integer divisor of 0 is replaced by 1; the truncated remainder
    (lax.rem) takes the divisor's sign by one add where the two signs differ and it is nonzero."""
    dt, weak = result_type(_aval(a), _aval(b))
    if _kind(dt) not in (1, 2):
        raise TraceError(f"remainder of {dt}")
    a, b = _coerce_t(a, dt, weak), _coerce_t(b, dt, weak)
    if _kind(dt) == 1:
        b = select(b == 0, literal(1, dt, weak=weak), b)
    t = binop("rem", a, b)
    plus = binop("and", binop("ne", binop("lt", t, 0), binop("lt", b, 0)), binop("ne", t, 0))
    return select(plus, binop("add", t, b), t)


def _coerce_t(x, dt, weak):
    """x as a traced value of dtype dt (constants are materialised: the JAX definitions above apply primitives to
    both operands)."""
    if is_traced(x):
        return x if x.dtype == dt else convert(x, dt, weak)
    return Tracer(bind("copy", [literal(np.asarray(x, dt), dt)], [AVal((), dt, weak)])[0].var)


def power(a, b):
    if _pyscalar(b) and isinstance(b, int) and not isinstance(b, bool):
        x = a
        if not is_traced(x):
            raise TraceError("power of a constant")
        return bind("integer_pow", [x.var], [x.aval], y=int(b))[0]
    a = _float_of(a)
    b = _float_of(b)
    return binop("pow", a, b)


def select(pred, on_true, on_false):
    """lax.select / jnp.where(pred, on_true, on_false)."""
    pa = _aval(pred)
    if pa.dtype != BOOL:
        raise TraceError("where/select needs a boolean predicate")
    dt, weak = result_type(_aval(on_true), _aval(on_false))
    shape = _shape_of(pa, _aval(on_true), _aval(on_false))
    pv = pred.var if is_traced(pred) else literal(pred)
    if not (is_traced(pred) or is_traced(on_true) or is_traced(on_false)):
        raise TraceError("where of constants: use numpy")
    # lax.select_n(pred, on_false, on_true)
    return bind("select_n", [pv, _coerce(on_false, dt, weak), _coerce(on_true, dt, weak)],
                [AVal(shape, dt, weak)])[0]


def getitem(x, i):
    """x[i] along the leading axis: a constant index -> slice + squeeze, as jnp does; a traced integer index ->
    dynamic_index (normalised if negative, then clamped into range, as jnp's gather)."""
    if is_traced(i):
        return dynamic_index(x, i)
    if not isinstance(i, (int, np.integer)):
        raise TraceError("only integer indices are supported in item code")
    n = x.shape[0]
    i = int(i)
    if i < 0:
        i += n
    if not 0 <= i < n:
        raise IndexError(f"index {i} out of range for axis of size {n}")
    rest = x.shape[1:]
    s = bind("slice", [x.var], [AVal((1,) + rest, x.dtype, x.aval.weak)],
             start_indices=(i,) + (0,) * len(rest), limit_indices=(i + 1,) + rest, strides=None)[0]
    return bind("squeeze", [s.var], [AVal(rest, x.dtype, x.aval.weak)], dimensions=(0,))[0]


def dynamic_index(x, i):
    """row i of x (i traced, integer): i < 0 counts from the end, then i is clamped to [0, n - 1] (jnp indexing
    with a traced index; lax.dynamic_index_in_dim clamps the same way)."""
    if not is_traced(x):
        x = Tracer(bind("copy", [literal(np.asarray(x))], [literal(np.asarray(x)).aval.strong()])[0].var)
    if not x.shape:
        raise TraceError("indexing a 0-d value")
    if not np.issubdtype(i.dtype, np.integer) or i.shape != ():
        raise TraceError("a traced index must be an integer scalar")
    n = x.shape[0]
    i = convert(i, I32)
    i = select(i < 0, i + n, i)
    i = select(i < 0, literal(0, I32, weak=False), select(i > n - 1, literal(n - 1, I32, weak=False), i))
    return bind("dynamic_index", [x.var, i.var], [AVal(x.shape[1:], x.dtype, x.aval.weak)])[0]


def stack(xs):
    """jnp.stack of scalars / equal-shape arrays along a new leading axis (broadcast_in_dim + concatenate)."""
    xs = list(xs)
    avs = [_aval(x) for x in xs]
    dt, weak = result_type(*avs)
    shape = _shape_of(*avs)
    parts = []
    for x in xs:
        v = _coerce(x, dt, weak)
        if isinstance(v, Lit):
            parts.append(Lit(np.broadcast_to(v.val, shape).reshape((1,) + shape), AVal((1,) + shape, dt, weak)))
            continue
        if v.aval.shape != shape:
            raise TraceError("stack: operands of different shapes")
        t = bind("broadcast_in_dim", [v], [AVal((1,) + shape, dt, weak)], shape=(1,) + shape,
                 broadcast_dimensions=tuple(range(1, 1 + len(shape))))[0]
        parts.append(t.var)
    return bind("concatenate", parts, [AVal((len(xs),) + shape, dt, weak)], dimension=0)[0]


def reduce_sum(x):
    if not x.shape:
        return x
    acc = x[0]
    for i in range(1, x.shape[0]):
        acc = acc + x[i]
    return acc


def trace_fn(fn, in_avals, parent=None, wrap_in=None):
    """trace fn over fresh invars -> (Jaxpr, outputs as returned (Tracers / constants), builder).  wrap_in maps the
    list of input Tracers to fn's arguments (default: positional)."""
    b = Builder(parent)
    _STACK.append(b)
    try:
        ins = [Tracer(b.new_invar(a)) for a in in_avals]
        out = fn(*(wrap_in(ins) if wrap_in else ins))
    finally:
        _STACK.pop()
    return b, ins, out


def walk_eqns(jx):
    """every equation of jx, sub-programs included (depth first)."""
    for e in jx.eqns:
        yield e
        for sub in subjaxprs(e):
            yield from walk_eqns(sub)


def subjaxprs(e):
    out = []
    for v in e.params.values():
        if isinstance(v, Jaxpr):
            out.append(v)
        elif isinstance(v, (list, tuple)):
            out.extend(x for x in v if isinstance(x, Jaxpr))
    return out
