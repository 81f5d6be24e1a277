"""Pinning of the elementwise / reduction oracle (oracle/ops_ref.py) on the CPU.

The reference's own cases: broadcasting (exercises/a2-broadcasting/tests/
spec.rs:15-54), views (exercises/a3-strided-views/tests/spec.rs:17-68).  The
rest by what the mathematics fixes: involutions, identities, closed-form
sums, known bf16/f16 bit patterns, IEEE special values.
"""
import numpy as np
import pytest

from oracle import ops_ref as R
from oracle import oracle as O


# ---- broadcasting: A2 hand cases ------------------------------------------------

@pytest.mark.parametrize("a,b,out", [
    ((2, 3), (3,), (2, 3)), ((4, 1), (1, 5), (4, 5)), ((), (2, 2), (2, 2)), ((3, 1, 7), (4, 1), (3, 4, 7)),
    ((1,), (5,), (5,)), ((0, 3), (3,), (0, 3)),
])
def test_broadcast_shapes_a2(a, b, out):
    assert R.broadcast_shape(a, b) == out
    assert R.broadcast_shape(b, a) == out


@pytest.mark.parametrize("a,b", [((2, 3), (4,)), ((2, 3), (3, 2)), ((5,), (4,))])
def test_broadcast_refusals_a2(a, b):
    with pytest.raises(ValueError):
        R.broadcast_shape(a, b)


def test_views_a3():
    buf = np.arange(1, 7, dtype=np.float32)                    # [[1,2,3],[4,5,6]]
    assert R.view(buf, (3, 2), (1, 3)).tolist() == [[1, 4], [2, 5], [3, 6]]       # permute([1,0])
    assert R.view(buf, (2, 2), (3, 1), 1).tolist() == [[2, 3], [5, 6]]            # narrow(1, 1, 2)
    assert R.view(buf, (6,), (1,)).tolist() == [1, 2, 3, 4, 5, 6]                 # reshape


# ---- unary -----------------------------------------------------------------------

@pytest.mark.parametrize("dt", [R.F32, R.F64, R.BF16, R.F16])
def test_neg_abs_exact(dt):
    rng = np.random.default_rng(1)
    x = R.from_f32(rng.normal(0, 3, 257).astype(np.float32), dt)
    n = R.unary(x, R.UN_NEG, dt)
    assert np.array_equal(R.to_f32(R.unary(n, R.UN_NEG, dt), dt), R.to_f32(x, dt))   # involution
    assert np.array_equal(R.to_f32(R.unary(n, R.UN_ABS, dt), dt), np.abs(R.to_f32(x, dt)))
    assert np.all(R.to_f32(R.unary(x, R.UN_ABS, dt), dt) >= 0)


def test_exp_ln_special_values():
    x = np.array([0.0, 1.0, -1.0, np.inf, -np.inf], np.float32)
    e = R.unary(x, R.UN_EXP, R.F32)
    assert e[0] == 1 and abs(e[1] - np.float32(np.e)) == 0 and e[3] == np.inf and e[4] == 0
    l = R.unary(np.array([1.0, 0.0, -1.0, np.inf], np.float32), R.UN_LN, R.F32)
    assert l[0] == 0 and l[1] == -np.inf and np.isnan(l[2]) and l[3] == np.inf


def test_exp_ln_inverse():
    x = np.linspace(0.01, 50, 999).astype(np.float32)
    back = R.unary(R.unary(x, R.UN_LN, R.F32), R.UN_EXP, R.F32)
    assert np.max(np.abs(back - x) / x) < 4e-7


def test_rounding_points_bf16_f16():
    # 1 + 2^-8 is exactly halfway between bf16 1 and 1 + 2^-7: ties to even -> 1
    assert R.from_f32(np.array([1 + 2 ** -8], np.float32), R.BF16)[0] == 0x3F80
    assert R.from_f32(np.array([1 + 3 * 2 ** -8], np.float32), R.BF16)[0] == 0x3F82
    # a bf16 add is one f32 add then one rounding: 1 + 2^-9 stays 1
    one, tiny = R.from_f32(np.array([1.0], np.float32), R.BF16), R.from_f32(np.array([2 ** -9], np.float32), R.BF16)
    assert R.binary(one, tiny, R.BIN_ADD, R.BF16)[0] == 0x3F80
    assert R.from_f32(np.array([65520.0], np.float32), R.F16)[0] == np.float16(np.inf)


# ---- binary ----------------------------------------------------------------------

@pytest.mark.parametrize("dt", [R.F32, R.F64, R.BF16, R.F16])
def test_binary_identities(dt):
    rng = np.random.default_rng(2)
    a = R.from_f32(rng.normal(0, 2, (5, 7)).astype(np.float32), dt)
    b = R.from_f32(rng.normal(0, 2, (7,)).astype(np.float32), dt)
    A = R.to_f32(a, dt)
    zero = R.from_f32(np.zeros(7, np.float32), dt)
    ones = R.from_f32(np.ones(7, np.float32), dt)
    assert np.array_equal(R.to_f32(R.binary(a, zero, R.BIN_ADD, dt), dt), A)
    assert np.array_equal(R.to_f32(R.binary(a, ones, R.BIN_MUL, dt), dt), A)
    assert np.array_equal(R.to_f32(R.binary(a, a, R.BIN_SUB, dt), dt), np.zeros_like(A))
    # commutativity of add / mul (one rounding of an exact-commutative op)
    assert np.array_equal(R.binary(a, b, R.BIN_ADD, dt), R.binary(b, a, R.BIN_ADD, dt))
    assert np.array_equal(R.binary(a, b, R.BIN_MUL, dt), R.binary(b, a, R.BIN_MUL, dt))


def test_binary_broadcast_values():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([10, 20, 30], np.float32)
    assert R.binary(a, b, R.BIN_ADD, R.F32).tolist() == [[11, 22, 33], [14, 25, 36]]
    col = np.array([[2], [4]], np.float32)
    assert R.binary(a, col, R.BIN_DIV, R.F32).tolist() == [[0.5, 1, 1.5], [1, 1.25, 1.5]]


def test_float_division_ieee():
    r = R.binary(np.array([1, -1, 0], np.float32), np.array([0, 0, 0], np.float32), R.BIN_DIV, R.F32)
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2])


# ---- reductions --------------------------------------------------------------------

def test_sum_closed_forms():
    n = 1000
    x = np.arange(n, dtype=np.float32).reshape(10, 100)
    s, _ = R.reduce_sum_f64(x, [], R.F32)
    assert s == n * (n - 1) / 2
    s0, _ = R.reduce_sum_f64(x, [0], R.F32)
    assert s0.tolist() == [sum(r * 100 + c for r in range(10)) for c in range(100)]
    s1, _ = R.reduce_sum_f64(x, [1], R.F32)
    assert s1.tolist() == [sum(r * 100 + c for c in range(100)) for r in range(10)]
    assert R.reduced_shape((10, 100), [0]) == (100,) and R.reduced_shape((10, 100), []) == ()


def test_max_closed_forms_and_nan():
    x = np.random.default_rng(3).permutation(60).astype(np.float32).reshape(3, 4, 5)
    assert R.reduce_max(x, [], R.F32) == 59
    assert np.array_equal(R.reduce_max(x, [0, 2], R.F32), x.max(axis=(0, 2)))
    y = x.copy()
    y[1, 2, 3] = np.nan
    m = R.reduce_max(y, [2], R.F32)
    assert np.isnan(m[1, 2]) and np.isfinite(m[0, 0])
    with pytest.raises(ValueError):
        R.reduce_max(np.zeros((3, 0), np.float32), [1], R.F32)
    s, _ = R.reduce_sum_f64(np.zeros((3, 0), np.float32), [1], R.F32)
    assert s.tolist() == [0, 0, 0]


# ---- integer / boolean semantics (oracle/ops_ref.py int_*) ----------------------------
# Pinned by hand-worked cases and by the arithmetic identities that fix
# wrapping and truncating division, not by restating the oracle's formulas.

def test_int_hand_cases():
    i32 = lambda *v: np.array(v, np.int32)
    # truncation toward zero in every sign combination; MIN / -1 wraps
    np.testing.assert_array_equal(R.int_binary(i32(7, -7, 7, -7, -2 ** 31), i32(2, 2, -2, -2, -1), R.BIN_DIV, R.I32),
                                  i32(3, -3, -3, 3, -2 ** 31))
    np.testing.assert_array_equal(R.int_binary(i32(2 ** 31 - 1), i32(1), R.BIN_ADD, R.I32), i32(-2 ** 31))
    np.testing.assert_array_equal(R.int_binary(i32(-2 ** 31), i32(1), R.BIN_SUB, R.I32), i32(2 ** 31 - 1))
    np.testing.assert_array_equal(R.int_binary(i32(65536), i32(65536), R.BIN_MUL, R.I32), i32(0))
    np.testing.assert_array_equal(R.int_unary(i32(-2 ** 31, -5, 0, 5), R.UN_ABS, R.I32), i32(-2 ** 31, 5, 0, 5))
    np.testing.assert_array_equal(R.int_unary(i32(-2 ** 31, -5, 0), R.UN_NEG, R.I32), i32(-2 ** 31, 5, 0))
    u8 = lambda *v: np.array(v, np.uint8)
    np.testing.assert_array_equal(R.int_binary(u8(250, 3), u8(10, 5), R.BIN_ADD, R.U8), u8(4, 8))
    np.testing.assert_array_equal(R.int_binary(u8(3), u8(5), R.BIN_SUB, R.U8), u8(254))
    np.testing.assert_array_equal(R.int_unary(u8(0, 1, 255), R.UN_NEG, R.U8), u8(0, 255, 1))
    np.testing.assert_array_equal(R.int_binary(u8(255, 7), u8(16, 2), R.BIN_DIV, R.U8), u8(15, 3))
    i64 = lambda *v: np.array(v, np.int64)
    np.testing.assert_array_equal(R.int_binary(i64(2 ** 62), i64(4), R.BIN_MUL, R.I64), i64(0))
    np.testing.assert_array_equal(R.int_binary(i64(-2 ** 63), i64(-1), R.BIN_DIV, R.I64), i64(-2 ** 63))
    b = lambda *v: np.array(v, np.uint8)
    np.testing.assert_array_equal(R.int_binary(b(0, 0, 1, 1), b(0, 1, 0, 1), R.BIN_ADD, R.BOOL), b(0, 1, 1, 1))
    np.testing.assert_array_equal(R.int_binary(b(0, 0, 1, 1), b(0, 1, 0, 1), R.BIN_MUL, R.BOOL), b(0, 0, 0, 1))
    np.testing.assert_array_equal(R.int_binary(b(0, 0, 1, 1), b(0, 1, 0, 1), R.BIN_EQ, R.BOOL), b(1, 0, 0, 1))
    with pytest.raises(R.DivisionByZero):
        R.int_binary(i32(1, 2), i32(1, 0), R.BIN_DIV, R.I32)


@pytest.mark.parametrize("dt,np_t", [(R.I32, np.int32), (R.I64, np.int64), (R.U8, np.uint8)])
def test_int_identities(dt, np_t):
    rng = np.random.default_rng(dt)
    info = np.iinfo(np_t)
    a = rng.integers(info.min, info.max, 500, dtype=np_t, endpoint=True)
    b = rng.integers(info.min, info.max, 500, dtype=np_t, endpoint=True)
    b[b == 0] = 1
    mod = 1 << info.bits
    # wrapping = the exact result reduced modulo 2^bits
    for op, f in ((R.BIN_ADD, lambda x, y: x + y), (R.BIN_SUB, lambda x, y: x - y), (R.BIN_MUL, lambda x, y: x * y)):
        got = R.int_binary(a, b, op, dt)
        for x, y, g in zip(a.tolist(), b.tolist(), got.tolist()):
            assert (f(x, y) - g) % mod == 0
            assert info.min <= g <= info.max
    # a + neg(a) == 0; abs(a) == a or neg(a)
    z = R.int_binary(a, R.int_unary(a, R.UN_NEG, dt), R.BIN_ADD, dt)
    assert not z.any()
    ab = R.int_unary(a, R.UN_ABS, dt)
    assert np.all((ab == a) | (ab == R.int_unary(a, R.UN_NEG, dt)))
    # truncating division: a = q*b + r, |r| < |b|, r has a's sign (or is 0)
    q = R.int_binary(a, b, R.BIN_DIV, dt)
    for x, y, qq in zip(a.tolist(), b.tolist(), q.tolist()):
        if np_t != np.uint8 and x == info.min and y == -1:
            assert qq == info.min
            continue
        r = x - qq * y
        assert abs(r) < abs(y) and (r == 0 or (r > 0) == (x > 0))


def test_int_reductions_closed_forms():
    # sum of 0..n-1 = n(n-1)/2, wrapped into I32; order does not matter
    n = 100_000
    x = np.arange(n, dtype=np.int32).reshape(250, 400)
    want = (n * (n - 1) // 2) % (1 << 32)
    want = want - (1 << 32) if want >= (1 << 31) else want
    assert int(R.int_reduce(x, [], 0, R.I32)) == want
    perm = np.random.default_rng(0).permutation(n).astype(np.int32).reshape(250, 400)
    assert int(R.int_reduce(perm, [], 0, R.I32)) == want
    np.testing.assert_array_equal(R.int_reduce(x, [1], 0, R.I32),
                                  (400 * np.arange(250, dtype=np.int64) * 400 + 400 * 399 // 2).astype(np.int32))
    # max is the last of a sorted copy; Bool sum / max are any()
    y = np.random.default_rng(1).integers(-50, 50, (7, 9)).astype(np.int64)
    np.testing.assert_array_equal(R.int_reduce(y, [0], 1, R.I64), np.sort(y, axis=0)[-1])
    bb = np.array([[0, 0, 1], [0, 0, 0]], np.uint8)
    np.testing.assert_array_equal(R.int_reduce(bb, [1], 0, R.BOOL), [1, 0])
    np.testing.assert_array_equal(R.int_reduce(bb, [0], 1, R.BOOL), [0, 0, 1])
    # U8 sum wraps modulo 256
    assert int(R.int_reduce(np.full(300, 255, np.uint8), [], 0, R.U8)) == (300 * 255) % 256
