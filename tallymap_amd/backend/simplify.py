"""Common-subexpression elimination over item programs, before they are emitted.

The adjoint programs repeat work by construction: value_and_grad's fused program runs POST and then POST's VJP,
which re-evaluates POST's primal values on the same loop results; a forward-only adjoint's loop body runs the step
and the step's VJP, which recomputes the step's primal values.  Equations of a pure primitive with the same
operands (the same variables, or equal literals), the same parameters and the same result types compute the same
values, so the later one is dropped and its results renamed to the earlier one's.  The device compiler removes
some of these itself, but not where the duplicate sits after a global atomic or a loop whose memory effects it
cannot see through (a libm table load after a store is not provably the same load).

Scopes: every jaxpr (a while's cond and body, a cond's branches) is processed on its own, since the item IR's
sub-jaxprs are closed (their operands are passed in).  The top-level program is cut at its step loop: PRE and POST
are separate scopes, so a POST equation is never renamed to a PRE result, which would keep that value live in a
register through the whole loop.
"""
import numpy as np

from .. import _core as C
from .codegen import EW

# primitives whose results are functions of their operands and parameters alone (no tally, tape, queue or record
# effects, no per-launch state)
PURE = set(EW) | {"integer_pow", "round", "convert_element_type", "bitcast_convert_type", "select_n", "copy",
                  "stop_gradient", "tallymap_ct_read", "threefry2x32", "slice", "dynamic_index", "squeeze",
                  "reshape", "broadcast_in_dim", "concatenate"}


def _pkey(x):
    """a hashable key of a parameter value (None: not keyable, the equation is left alone)."""
    if isinstance(x, (bool, int, float, str, type(None), np.dtype)):
        return (type(x).__name__, x)
    if isinstance(x, np.generic):
        return ("np", x.dtype.str, x.tobytes())
    if isinstance(x, np.ndarray):
        return ("arr", x.dtype.str, x.shape, x.tobytes())
    if isinstance(x, (tuple, list)):
        ks = tuple(_pkey(y) for y in x)
        return None if any(k is None for k in ks) else ("seq", ks)
    if isinstance(x, type) and issubclass(x, np.generic):
        return ("npt", np.dtype(x).str)
    return None


def _vkey(v):
    if isinstance(v, C.Lit):
        a = np.asarray(v.val)
        return ("lit", v.aval.dtype.str if hasattr(v.aval.dtype, "str") else str(v.aval.dtype), a.shape,
                a.tobytes(), bool(getattr(v.aval, "weak", False)))
    return ("var", v.id)


def _akey(a):
    return (tuple(a.shape), str(a.dtype))


def cse(jx, cut=None):
    """-> jx with repeated pure equations removed (the same Jaxpr object when nothing changes).  cut: the index of
    an equation (the step loop) that separates two scopes; the equation itself is kept and processed."""
    sub = {}
    eqns = []
    seen = {}
    changed = False

    def r(v):
        return sub.get(v.id, v) if isinstance(v, C.Var) else v

    for i, e in enumerate(jx.eqns):
        if i == cut:
            seen = {}
        ins = [r(v) for v in e.invars]
        params = e.params
        if C.subjaxprs(e):
            new = {}
            for k, p in e.params.items():
                if isinstance(p, C.Jaxpr):
                    p2 = cse(p)
                elif isinstance(p, (list, tuple)) and any(isinstance(x, C.Jaxpr) for x in p):
                    xs = [cse(x) if isinstance(x, C.Jaxpr) else x for x in p]
                    p2 = p if all(a is b for a, b in zip(xs, p)) else type(p)(xs)
                else:
                    p2 = p
                new[k] = p2
            if any(new[k] is not p for k, p in e.params.items()):
                params = new
        if e.prim in PURE and params is e.params:
            pk = tuple(sorted((k, _pkey(p)) for k, p in params.items()))
            if all(k[1] is not None for k in pk):
                key = (e.prim, tuple(_vkey(v) for v in ins), pk, tuple(_akey(o.aval) for o in e.outvars))
                prev = seen.get(key)
                if prev is not None:
                    for o, p in zip(e.outvars, prev):
                        sub[o.id] = p
                    changed = True
                    continue
                seen[key] = e.outvars
        if i == cut:
            seen = {}
        if params is not e.params or any(a is not b for a, b in zip(ins, e.invars)):
            e = C.Eqn(e.prim, ins, e.outvars, params)
            changed = True
        eqns.append(e)
    if not changed:
        return jx
    return C.Jaxpr(jx.invars, [r(v) for v in jx.outvars], eqns)
