"""Per-operation edge semantics on the GPU (the classes of the reference's tests/ops.py:1-46, 'exact' rows): one
item per operand pair, every elementwise, conversion and shift rule the emitter lowers applied to NaN, +-0, +-inf,
subnormals, INT_MIN / -1, x / 0, shift counts >= the width and float -> integer values past the range, each result
compared BITWISE (NaN: any NaN) with a numpy restatement of lax's semantics (reference kernel.py:78-109: NaN-
propagating max / min with +0 / -0 ties, x / 0 = -1 and INT_MIN / -1 = INT_MIN, x rem 0 = x, shifts past the width
0 or the sign fill, saturating float -> integer conversion with NaN -> 0) and of jnp's `//` and `%`."""
import numpy as np
import pytest

import tallymap_amd as tm
from tallymap_amd import lax

pytestmark = pytest.mark.gpu

F32S = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 2.0 ** -126, -(2.0 ** -130), 1.0, -1.0, 0.5, -0.5,
                 1.5, 2.5, -2.5, 0.49999997, 3e38, -3e38, 3.4028235e38, 2147483520.0, 2147483648.0, -2147483648.0,
                 -2147483904.0, 4294967040.0, 4294967296.0, 9.223372e18, -9.223373e18, 1e10, -1e10, 7.0, -7.0, 3.0,
                 8388609.0, 0.1], np.float32)
I32S = np.array([0, 1, -1, 2, -2, 7, -7, 31, 32, 33, 63, 64, 100, -100, 2 ** 31 - 1, -2 ** 31, -2 ** 31 + 1,
                 16777217, -16777217, 123456789], np.int64)


def _pairs(spec, rnd, dt):
    a, b = np.meshgrid(spec, spec, indexing="ij")
    return np.concatenate([a.ravel(), rnd[0]]).astype(dt), np.concatenate([b.ravel(), rnd[1]]).astype(dt)


def _run(item, *ops):
    import torch
    f = tm.vmap(lambda t, *a: (t, item(*a)), outputs={})
    ys = f(*ops).per_item
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in (ys if isinstance(ys, (tuple, list)) else [ys])]


def _same(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.dtype == want.dtype and got.shape == want.shape, (name, got.dtype, want.dtype)
    if got.dtype.kind == "f":
        nan = np.isnan(want)
        ok = (np.isnan(got) == nan) & ((got.view(f"u{got.itemsize}") == want.view(f"u{want.itemsize}")) | nan)
    else:
        ok = got == want
    bad = np.flatnonzero(~ok)
    assert bad.size == 0, f"{name}: {bad.size} mismatches, first at {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


# ------------------------------------------------------------------------------------- numpy restatements
def _fmax(a, b):
    r = np.where(a > b, a, np.where(b > a, b, np.where(a == 0, a + b, a)))
    return np.where(np.isnan(a) | np.isnan(b), np.nan, r).astype(a.dtype)


def _fmin(a, b):
    r = np.where(a < b, a, np.where(b < a, b, np.where(a == 0, -(-a - b), a)))
    return np.where(np.isnan(a) | np.isnan(b), np.nan, r).astype(a.dtype)


def _fsign(a):
    return np.where(a > 0, 1, np.where(a < 0, -1, a)).astype(a.dtype)


def _round_away(a):
    x = a.astype(np.float64)
    return np.where(np.isfinite(x), np.trunc(x + np.copysign(0.5, x)), x).astype(a.dtype)


def _f2i(a, lo, hi):
    """saturating float -> integer toward zero, NaN -> 0 (lo, hi: the integer range as Python ints)."""
    out = []
    for v in np.asarray(a, np.float64):
        if v != v:
            out.append(0)
        elif v <= lo:
            out.append(lo)
        elif v >= hi:
            out.append(hi)
        else:
            out.append(int(v))
    return out


def _idiv(a, b, bits, signed=True):
    mn = -(1 << (bits - 1))
    q = []
    for x, y in zip(a.tolist(), b.tolist()):
        if y == 0:
            q.append(-1 if signed else (1 << bits) - 1)
        elif signed and y == -1 and x == mn:
            q.append(mn)
        else:
            q.append(abs(x) // abs(y) * (1 if (x < 0) == (y < 0) else -1))
    return np.array(q, a.dtype if signed else a.dtype)


def _irem(a, b, bits, signed=True):
    mn = -(1 << (bits - 1))
    r = []
    for x, y in zip(a.tolist(), b.tolist()):
        if y == 0:
            r.append(x)
        elif signed and y == -1 and x == mn:
            r.append(0)
        else:
            m = abs(x) % abs(y)
            r.append(-m if x < 0 else m)
    return np.array(r, a.dtype)


def _shl(a, s, bits):
    u = a.astype(f"u{bits // 8}")
    su = s.astype(f"u{bits // 8}")
    with np.errstate(over="ignore"):
        r = np.where(su >= bits, 0, u << np.minimum(su, bits - 1))
    return r.astype(f"u{bits // 8}").view(a.dtype) if a.dtype.kind == "i" else r.astype(a.dtype)


def _shrl(a, s, bits):
    u = a.astype(f"u{bits // 8}")
    su = s.astype(f"u{bits // 8}")
    r = np.where(su >= bits, 0, u >> np.minimum(su, bits - 1))
    return r.astype(f"u{bits // 8}").view(a.dtype) if a.dtype.kind == "i" else r.astype(a.dtype)


def _shra(a, s, bits):
    su = s.astype(f"u{bits // 8}")
    return np.where(su >= bits, np.where(a < 0, -1, 0), a >> np.minimum(su, bits - 1).astype(a.dtype)).astype(a.dtype)


def _jnp_floordiv_int(a, b, bits):
    q = _idiv(a, b, bits)
    r = _irem(a, b, bits)
    fix = (np.sign(a) != np.sign(b)) & (r != 0)
    with np.errstate(over="ignore"):
        return np.where(fix, q - a.dtype.type(1), q).astype(a.dtype)


def _jnp_mod_int(a, b, bits):
    b = np.where(b == 0, b.dtype.type(1), b)
    t = _irem(a, b, bits)
    plus = ((t < 0) != (b < 0)) & (t != 0)
    with np.errstate(over="ignore"):
        return np.where(plus, t + b, t).astype(a.dtype)


def _jnp_mod_f(a, b):
    t = np.fmod(a, b)
    plus = ((t < 0) != (b < 0)) & (t != 0)
    return np.where(plus, t + b, t).astype(a.dtype)


def _jnp_floordiv_f(a, b):
    mod = np.fmod(a, b)
    div = ((a - mod) / b).astype(a.dtype)
    ind = (mod != 0) & (_fsign(b) != _fsign(mod))
    div = np.where(ind, div - a.dtype.type(1), div).astype(a.dtype)
    return _round_away(div)


# ------------------------------------------------------------------------------------------------- tests
def test_f32_binary():
    print("case: f32 binary ops on specials x specials + random", flush=True)
    rng = np.random.default_rng(1)
    rnd = [(rng.standard_normal(4096) * np.exp(rng.uniform(-30, 30, 4096))).astype(np.float32) for _ in range(2)]
    a, b = _pairs(F32S, rnd, np.float32)
    got = _run(lambda x, y: (x + y, x - y, x * y, x / y, lax.rem(x, y), lax.max(x, y), lax.min(x, y), x < y, x <= y,
                             x == y, x != y, lax.select(x < y, x, y), x % y, x // y), a, b)
    with np.errstate(all="ignore"):
        want = [a + b, a - b, a * b, a / b, np.fmod(a, b), _fmax(a, b), _fmin(a, b), a < b, a <= b, a == b, a != b,
                np.where(a < b, a, b), _jnp_mod_f(a, b), _jnp_floordiv_f(a, b)]
    for n, g, w in zip(["add", "sub", "mul", "div", "rem", "max", "min", "lt", "le", "eq", "ne", "select", "mod",
                        "floordiv"], got, want):
        _same(n, g, w)


def test_f32_unary_and_conversions():
    print("case: f32 unary ops and conversions", flush=True)
    rng = np.random.default_rng(2)
    a = np.concatenate([F32S, (rng.standard_normal(8192) * np.exp(rng.uniform(-40, 45, 8192))),
                        rng.uniform(-4, 4, 4096)]).astype(np.float32)
    got = _run(lambda x: (-x, abs(x), lax.sign(x), lax.floor(x), lax.ceil(x), lax.round(x, 0), lax.round(x, 1),
                          lax.sqrt(x), x ** 3, x.astype(np.int32), x.astype(np.uint32), x.astype(np.int64),
                          x.astype(np.float64), lax.bitcast_convert_type(x, np.uint32)), a)
    with np.errstate(all="ignore"):
        want = [-a, np.abs(a), _fsign(a), np.floor(a), np.ceil(a), _round_away(a), np.rint(a), np.sqrt(a),
                a * (a * a), np.array(_f2i(a, -2 ** 31, 2 ** 31 - 1), np.int32),
                np.array(_f2i(a, 0, 2 ** 32 - 1), np.uint32), np.array(_f2i(a, -2 ** 63, 2 ** 63 - 1), np.int64),
                a.astype(np.float64), a.view(np.uint32)]
    for n, g, w in zip(["neg", "abs", "sign", "floor", "ceil", "round_away", "round_even", "sqrt", "pow3", "f2i32",
                        "f2u32", "f2i64", "f2f64", "bitcast"], got, want):
        _same(n, g, w)


def test_f64_ops_and_conversions():
    print("case: f64 ops and conversions", flush=True)
    rng = np.random.default_rng(3)
    spec = np.concatenate([F32S.astype(np.float64), [2.0 ** -1074, -(2.0 ** -1060), 1.7976931348623157e308,
                                                     2147483647.5, -2147483648.5, 3.4028235677973366e38,
                                                     1.401298464324817e-45 / 2, 0.1]])
    rnd = [rng.standard_normal(2048) * np.exp(rng.uniform(-700, 700, 2048)) for _ in range(2)]
    a, b = _pairs(spec, rnd, np.float64)
    got = _run(lambda x, y: (x + y, x * y, x / y, lax.max(x, y), lax.sqrt(x), x.astype(np.float32),
                             x.astype(np.int32), x.astype(np.uint32), x.astype(np.int64), lax.floor(x),
                             lax.rem(x, y), x % y), a, b)
    with np.errstate(all="ignore"):
        want = [a + b, a * b, a / b, _fmax(a, b), np.sqrt(a), a.astype(np.float32),
                np.array(_f2i(a, -2 ** 31, 2 ** 31 - 1), np.int32), np.array(_f2i(a, 0, 2 ** 32 - 1), np.uint32),
                np.array(_f2i(a, -2 ** 63, 2 ** 63 - 1), np.int64), np.floor(a), np.fmod(a, b), _jnp_mod_f(a, b)]
    for n, g, w in zip(["add", "mul", "div", "max", "sqrt", "f2f32", "d2i32", "d2u32", "d2i64", "floor", "rem", "mod"],
                       got, want):
        _same(n, g, w)


@pytest.mark.parametrize("dt,bits", [(np.int32, 32), (np.int64, 64)])
def test_signed_integer_ops(dt, bits):
    print(f"case: {np.dtype(dt).name} integer ops", flush=True)
    rng = np.random.default_rng(4)
    # (64-bit: the extremes, and ties and near-ties of the conversion to float32 at 2^40, where its ulp is 2^17)
    spec = I32S if bits == 32 else np.concatenate([I32S, [2 ** 63 - 1, -2 ** 63, 2 ** 40 + 7, -(2 ** 53) - 1,
                                                          2 ** 40 + 2 ** 16, 2 ** 40 + 2 ** 16 + 1, 2 ** 40 + 3 * 2 ** 16,
                                                          -(2 ** 40 + 3 * 2 ** 16), 2 ** 63 - 2 ** 38, 2 ** 32 - 1,
                                                          2 ** 32, 2 ** 32 + 1, 2 ** 56 + 2 ** 32 + 1]])
    rnd = [rng.integers(-2 ** (bits - 1), 2 ** (bits - 1), 2048, dtype=np.int64 if bits == 64 else np.int32)
           for _ in range(2)]
    rnd[1][:1024] = rng.integers(-3, bits + 3, 1024)
    a, b = _pairs(spec, rnd, dt)
    got = _run(lambda x, y: (lax.div(x, y), lax.rem(x, y), x // y, x % y, x << y, x >> y, lax.shift_right_logical(x, y),
                             lax.max(x, y), lax.min(x, y), x & y, x | y, x ^ y, -x, abs(x), lax.sign(x),
                             x.astype(np.float32), x.astype(np.float64), x < y), a, b)
    with np.errstate(over="ignore"):
        want = [_idiv(a, b, bits), _irem(a, b, bits), _jnp_floordiv_int(a, b, bits), _jnp_mod_int(a, b, bits),
                _shl(a, b, bits), _shra(a, b, bits), _shrl(a, b, bits), np.maximum(a, b), np.minimum(a, b), a & b,
                a | b, a ^ b, (0 - a.astype(f"u{bits // 8}")).view(dt), np.where(a < 0, (0 - a.astype(f"u{bits // 8}")).view(dt), a),
                np.sign(a).astype(dt), a.astype(np.float32), a.astype(np.float64), a < b]
    for n, g, w in zip(["div", "rem", "floordiv", "mod", "shl", "shra", "shrl", "max", "min", "and", "or", "xor", "neg",
                        "abs", "sign", "i2f32", "i2f64", "lt"], got, want):
        _same(n, g, w)


def test_unsigned_integer_ops():
    print("case: uint32 integer ops", flush=True)
    rng = np.random.default_rng(5)
    spec = np.array([0, 1, 2, 7, 31, 32, 33, 100, 2 ** 31, 2 ** 32 - 1, 2 ** 24 + 1, 3000000000], np.uint32)
    rnd = [rng.integers(0, 2 ** 32, 2048, dtype=np.uint32) for _ in range(2)]
    rnd[1][:1024] = rng.integers(0, 40, 1024)
    a, b = _pairs(spec, rnd, np.uint32)
    got = _run(lambda x, y: (lax.div(x, y), lax.rem(x, y), x // y, x % y, x << y, x >> y, lax.max(x, y),
                             x.astype(np.float32), x.astype(np.float64)), a, b)
    q = np.array([0xFFFFFFFF if y == 0 else x // y for x, y in zip(a.tolist(), b.tolist())], np.uint32)
    r = np.array([x if y == 0 else x % y for x, y in zip(a.tolist(), b.tolist())], np.uint32)
    m = np.array([x % (y if y else 1) for x, y in zip(a.tolist(), b.tolist())], np.uint32)
    want = [q, r, q, m, _shl(a, b, 32), _shrl(a, b, 32), np.maximum(a, b), a.astype(np.float32), a.astype(np.float64)]
    for n, g, w in zip(["div", "rem", "floordiv", "mod", "shl", "shrl", "max", "u2f32", "u2f64"], got, want):
        _same(n, g, w)


def test_static_loops_run_past_max_steps():
    """A 1000-step scan and a 300-step static fori_loop under max_steps=100 run to the end (JAX lowers both to
    scan, which the cap does not touch): no item truncated, the float tally finite and exact, beside a while_loop
    that the cap does stop."""
    import torch
    print("case: static loops past max_steps, N=4096", flush=True)

    def item(t, x):
        c, _ = lax.scan(lambda c, _: (c + x, None), np.float32(0.0), length=1000)
        k = lax.fori_loop(0, 300, lambda i, a: a + 1, 0)
        return t.add("h", 0, c), (c, k)
    x = np.full(4096, 0.5, np.float32)
    r = tm.vmap(item, outputs={"h": tm.Sum((1,))}, max_steps=100)(x)
    torch.cuda.synchronize()
    c, k = (v.cpu().numpy() for v in r.per_item)
    assert not r.truncated.cpu().numpy().any()
    assert (c == 500.0).all() and (k == 300).all()
    assert r.outputs["h"].cpu().numpy()[0] == 4096 * 500.0

    def item2(t, x):
        n = lax.while_loop(lambda a: a < 1000.0, lambda a: a + x, np.float32(0.0))
        return t.add("h", 0, n), n
    r2 = tm.vmap(item2, outputs={"h": tm.Sum((1,))}, max_steps=100)(x)
    torch.cuda.synchronize()
    assert r2.truncated.cpu().numpy().all() and (r2.per_item.cpu().numpy() == 50.0).all()
    assert np.isnan(r2.outputs["h"].cpu().numpy()[0])
