"""GPU parity of UnaryOps / BinaryOps / ReduceOps on I32, I64, U8 and Bool
against oracle/ops_ref.py's integer restatement, bit-exact, through the
C-ABI; the typed refusals (integer division by zero, ops a dtype does not
carry).  Semantics: crates/oxmera-ops/src/lib.rs:27-69 (div: :47-48),
crates/oxmera-core/src/dtype.rs:9-22."""
import numpy as np
import pytest

import oxmera_amd as ox
from oracle import ops_ref as R

pytestmark = pytest.mark.gpu

DEV = ox.Device.rocm(0)
DTS = [(ox.DType.I32, R.I32, np.int32), (ox.DType.I64, R.I64, np.int64), (ox.DType.U8, R.U8, np.uint8),
       (ox.DType.Bool, R.BOOL, np.uint8)]
IDS = ["i32", "i64", "u8", "bool"]


def rand(rng, npt, shape, bool_=False, nonzero=False):
    if bool_:
        return rng.integers(0, 2, shape).astype(np.uint8)
    info = np.iinfo(npt)
    v = rng.integers(info.min, info.max, shape, dtype=npt, endpoint=True)
    # mix in the extremes and small values
    flat = v.reshape(-1)
    flat[:: 7] = info.min
    flat[1:: 11] = info.max
    flat[2:: 5] = rng.integers(-3 if info.min < 0 else 0, 4, flat[2:: 5].shape)
    if nonzero:
        flat[flat == 0] = 1
    return v


def dev(arr, dtype):
    host = arr.astype(np.bool_) if dtype == ox.DType.Bool else arr
    return ox.Tensor.from_numpy(host, DEV, dtype)


def back(t):
    out = t.to_numpy()
    return out.astype(np.uint8) if t.dtype == ox.DType.Bool else out


def layouts(arr, dtype):
    """(name, device view, logical host values) for several layouts of arr (2-D)."""
    m, n = arr.shape
    out = [("contiguous", dev(arr, dtype), arr)]
    t = dev(np.ascontiguousarray(arr.T), dtype).permute([1, 0])
    out.append(("transposed", t, arr))
    pad = np.zeros((m, 2 * n + 3), arr.dtype)
    pad[:, 3:3 + 2 * n:2] = arr
    pv = dev(pad.reshape(-1), dtype).with_layout((m, n), (2 * n + 3, 2), 3)
    out.append(("strided", pv, arr))
    fl = dev(np.ascontiguousarray(arr[::-1]), dtype).with_layout((m, n), (-n, 1), (m - 1) * n)
    out.append(("flipped", fl, arr))
    return out


@pytest.mark.parametrize("dt,rdt,npt", DTS, ids=IDS)
def test_int_unary(hip, dt, rdt, npt):
    rng = np.random.default_rng(10 + rdt)
    x = rand(rng, npt, (37, 129), bool_=dt == ox.DType.Bool)
    ops = [("abs", hip.abs, R.UN_ABS)] + ([] if dt == ox.DType.Bool else [("neg", hip.neg, R.UN_NEG)])
    for lname, v, host in layouts(x, dt):
        for name, fn, op in ops:
            print(f"int unary {dt.name} {name} {lname}", flush=True)
            np.testing.assert_array_equal(back(fn(v)), R.int_unary(host, op, rdt), err_msg=f"{name} {lname}")


@pytest.mark.parametrize("dt,rdt,npt", DTS, ids=IDS)
def test_int_binary(hip, dt, rdt, npt):
    rng = np.random.default_rng(20 + rdt)
    is_bool = dt == ox.DType.Bool
    a = rand(rng, npt, (33, 200), bool_=is_bool)
    b = rand(rng, npt, (33, 200), bool_=is_bool, nonzero=True)
    ops = [("add", hip.add, R.BIN_ADD), ("mul", hip.mul, R.BIN_MUL), ("eq", hip.eq, R.BIN_EQ)]
    if not is_bool:
        ops += [("sub", hip.sub, R.BIN_SUB), ("div", hip.div, R.BIN_DIV)]
    la, lb = layouts(a, dt), layouts(b, dt)
    for (na, va, ha), (nb, vb, hb) in zip(la, lb[1:] + lb[:1]):
        for name, fn, op in ops:
            print(f"int binary {dt.name} {name} {na} x {nb}", flush=True)
            np.testing.assert_array_equal(back(fn(va, vb)), R.int_binary(ha, hb, op, rdt), err_msg=f"{name}")
    # broadcasts: a row, a column, a scalar
    row, col = b[0], b[:, :1]
    for bh in (row, col, b[:1, :1].reshape(())):
        bv = dev(np.ascontiguousarray(bh), dt)
        for name, fn, op in ops:
            np.testing.assert_array_equal(back(fn(la[0][1], bv)), R.int_binary(a, bh, op, rdt),
                                          err_msg=f"{name} broadcast {bh.shape}")


@pytest.mark.parametrize("dt,rdt,npt", DTS[:3], ids=IDS[:3])
def test_int_division_by_zero_is_typed(hip, dt, rdt, npt):
    a = dev(np.arange(1, 65, dtype=npt).reshape(8, 8), dt)
    z = np.ones((8, 8), npt)
    z[5, 3] = 0
    with pytest.raises(ox.DivisionByZero):
        hip.div(a, dev(z, dt))
    # a zero broadcast scalar too, and the backend still works afterwards
    with pytest.raises(ox.DivisionByZero):
        hip.div(a, dev(np.zeros((), npt), dt))
    np.testing.assert_array_equal(back(hip.div(a, dev(np.full((1, 8), 2, npt), dt))),
                                  R.int_binary(np.arange(1, 65, dtype=npt).reshape(8, 8), np.full((1, 8), 2, npt),
                                               R.BIN_DIV, rdt))


def test_int_refusals(hip):
    i = dev(np.arange(6, dtype=np.int32).reshape(2, 3), ox.DType.I32)
    bl = dev(np.array([[1, 0, 1]], np.uint8), ox.DType.Bool)
    for fn in (hip.exp, hip.ln, hip.sign):
        with pytest.raises(ox.UnsupportedDType):
            fn(i)
    with pytest.raises(ox.UnsupportedDType):
        hip.dgelu(i, i)
    with pytest.raises(ox.UnsupportedDType):
        hip.neg(bl)
    for fn in (hip.sub, hip.div):
        with pytest.raises(ox.UnsupportedDType):
            fn(bl, bl)
    with pytest.raises(ox.DTypeMismatch):
        hip.add(i, bl)


@pytest.mark.parametrize("dt,rdt,npt", DTS, ids=IDS)
def test_int_reductions(hip, dt, rdt, npt):
    rng = np.random.default_rng(30 + rdt)
    is_bool = dt == ox.DType.Bool
    # small and wide rows (the block-per-output schedule takes >= 1024 reduced elements)
    for shape in ((6, 7, 9), (4, 3000), (2, 4096, 3)):
        x = rand(rng, npt, shape, bool_=is_bool)
        v = dev(x, dt)
        for axes in ([], [0], [len(shape) - 1], [0, len(shape) - 1], list(range(len(shape)))):
            for name, fn, op in (("sum", hip.sum, 0), ("max", hip.max, 1)):
                print(f"int reduce {dt.name} {name} {shape} axes {axes}", flush=True)
                got = back(fn(v, axes))
                np.testing.assert_array_equal(got, R.int_reduce(x, axes, op, rdt), err_msg=f"{name} {axes}")
        # a transposed view reduced over its inner axis
        t = v.permute(list(reversed(range(len(shape)))))
        np.testing.assert_array_equal(back(hip.sum(t, [0])), R.int_reduce(np.transpose(x), [0], 0, rdt))
    with pytest.raises(ox.ShapeMismatch):
        hip.max(dev(np.zeros((3, 0), npt), dt), [1])
