"""The Tally: a write-only, linearly threaded handle on an item's sum outputs (reference tallymap/_tally.py).

`t = t.add(name, index, value)` binds one `tallymap_emit` equation (reference _tally.py:29-99): invars
[tally, flat index (int32), value (the tally's dtype)], one result, the new tally.  A tuple index is flattened row
major with a per-dimension bounds test, and an out-of-range component makes the whole index -1 (reference
_tally.py:260-271); the backend drops every index outside [0, S) and counts it (stats['dropped_emits']).
"""
import numpy as np

from . import _core as C


class Tally:
    __slots__ = ("_a", "_shapes")

    def __init__(self, arrays, shapes):
        self._a = dict(arrays)
        self._shapes = dict(shapes)

    @classmethod
    def _from(cls, a, shapes):
        return cls(a, shapes)

    def _shapes_key(self):
        return tuple(sorted((n, tuple(s)) for n, s in self._shapes.items()))

    def _with(self, name, v):
        a = dict(self._a)
        a[name] = v
        return Tally(a, self._shapes)

    def add(self, name, index, value):
        """tally[name][index] += value.  index: an int (flat index of a 1-D output) or a tuple of ints, one per
        output dimension.  Out-of-range or negative indices are dropped and counted."""
        if name not in self._a:
            raise KeyError(f"tallymap: unknown output {name!r} (outputs: {sorted(self._a)})")
        shape = self._shapes[name]
        t = self._a[name]
        if isinstance(index, tuple):
            if len(index) != len(shape):
                raise IndexError(f"tallymap: output {name!r} has {len(shape)} dims, index has {len(index)}")
            flat, ok = None, None
            for i, n in zip(index, shape):
                _check_int(i)
                i = C.convert(i, C.I32) if C.is_traced(i) else int(i)
                okd = (i >= 0) & (i < n) if C.is_traced(i) else (0 <= i < n)
                ci = _clip(i, 0, n - 1)
                if flat is None:
                    flat, ok = ci, okd
                else:
                    flat = flat * n + ci
                    ok = ok & okd
            if not C.is_traced(flat):
                flat = flat if ok else -1
            else:
                from . import numpy as jnp
                flat = jnp.where(ok, flat, -1)
        else:
            if len(shape) > 1:
                raise IndexError(f"tallymap: output {name!r} has shape {shape}; index it with a tuple")
            _check_int(index)
            flat = C.convert(index, C.I32) if C.is_traced(index) else int(index)
        tdt = t.aval.dtype
        if not C.is_traced(flat):
            flat = C.literal(int(flat), C.I32, weak=False)
            fv = flat
        else:
            fv = flat.var
        if (not np.issubdtype(tdt, np.inexact) and C.is_traced(value)
                and np.issubdtype(value.dtype, np.inexact)):
            raise TypeError(f"tallymap: t.add({name!r}, ...): a float value added to an integer output")
        if C.is_traced(value):
            if value.shape != ():
                raise TypeError("tallymap: t.add(...): only scalar values are supported by this backend")
            vv = value.var if value.dtype == tdt else C.convert(value, tdt).var
        else:
            vv = C.literal(np.asarray(value).astype(tdt), tdt, weak=False)
        new = C.bind("tallymap_emit", [t.var, fv, vv], [t.aval])[0]
        return self._with(name, new)


def _check_int(i):
    if C.is_traced(i):
        if not np.issubdtype(i.dtype, np.integer):
            raise TypeError(f"tallymap: t.add(...): index dtype {i.dtype} is not an integer")
        if i.shape != ():
            raise TypeError("tallymap: t.add(...): only scalar indices are supported by this backend")
    elif not isinstance(i, (int, np.integer)):
        raise TypeError(f"tallymap: t.add(...): index {i!r} is not an integer")


def _clip(i, lo, hi):
    if not C.is_traced(i):
        return min(max(i, lo), hi)
    from . import numpy as jnp
    return jnp.clip(i, lo, hi)
