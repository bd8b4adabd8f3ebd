"""Python-integer exact sum of f32 values -- TEST INFRASTRUCTURE ONLY.

The reference's host integer reference for its exact sum (tests/edge.py:2038-2065): each finite f32 is an integer
number of units of 2^-149; the exact total is a Python int, rounded once to f32 (nearest, ties to even).  Used to
pin the oracle's and the product's exact accumulators on small inputs.
"""
import numpy as np


def units(v):
    """the f32 `v` as an integer count of 2^-149 units (None: not finite)."""
    b = int(np.float32(v).view(np.uint32))
    e = (b >> 23) & 255
    if e == 255:
        return None
    m = (b & 0x7FFFFF) | (0x800000 if e else 0)
    p = e - 1 if e else 0
    u = m << p
    return -u if b >> 31 else u


def round_units(total):
    """the integer `total` (units of 2^-149) rounded once to f32, nearest, ties to even (None: beyond f32)."""
    if total == 0:
        return np.float32(0.0)
    neg = total < 0
    a = -total if neg else total
    top = a.bit_length() - 1
    if top < 24:
        q, sh = a, 0
    else:
        sh = top - 23
        q = a >> sh
        rem = a - (q << sh)
        half = 1 << (sh - 1) if sh else 0
        if sh and (rem > half or (rem == half and (q & 1))):
            q += 1
    val = q * 2.0 ** (sh - 149)            # exact in double: q < 2^25
    if val > float(np.finfo(np.float32).max):
        return None
    r = np.float32(val)
    return -r if neg else r


def exact_sum(values):
    """(the exactly rounded f32 sum, bad): bad when a value is not finite or the total is beyond f32."""
    tot = 0
    for v in np.asarray(values, np.float32).ravel():
        u = units(v)
        if u is None:
            return np.float32(np.nan), True
        tot += u
    r = round_units(tot)
    if r is None:
        return np.float32(np.nan), True
    return r, False
