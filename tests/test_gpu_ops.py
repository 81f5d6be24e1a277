"""GPU parity of the rest of the Backend (UnaryOps, BinaryOps, ReduceOps,
Tensor::contiguous) against oracle/ops_ref.py, through the C-ABI.

Bars: neg / abs / add / sub / mul / div and copies are bit-exact (one
operation, one rounding, as the oracle); exp / ln within 4 ulp for f32 and
f64 (device float functions against numpy's float64 ones), <= 1 ulp of a
16-bit output;
max bit-exact; sum within the f32 summation bound n * 2^-24 * sum |x| (plus
one rounding of the output dtype).
"""
import numpy as np
import pytest

import oxmera_amd as ox
from oracle import ops_ref as R

pytestmark = pytest.mark.gpu

DT = {ox.DType.F32: R.F32, ox.DType.F64: R.F64, ox.DType.BF16: R.BF16, ox.DType.F16: R.F16}
NPDT = {R.F32: np.float32, R.F64: np.float64, R.BF16: np.uint16, R.F16: np.float16}
DTYPES = [ox.DType.F32, ox.DType.F64, ox.DType.BF16, ox.DType.F16]
IDS = ["f32", "f64", "bf16", "f16"]


def log(msg):
    print(msg, flush=True)


def raw(values, dt):
    return R.from_f32(np.asarray(values, np.float64 if dt == R.F64 else np.float32), dt)


def dev_view(buf, dtype, shape, strides, offset=0):
    base = ox.Tensor.from_numpy(buf.reshape(-1), ox.Device.rocm(0), dtype)
    return base.with_layout(tuple(shape), tuple(strides), offset)


def layouts(rng, dtype, shape):
    """(name, device view, logical raw values) for several layouts of `shape`."""
    dt = DT[dtype]
    n = int(np.prod(shape))
    out = []
    buf = raw(rng.normal(0, 2, n), dt)
    out.append(("contiguous", dev_view(buf, dtype, shape, ox.contiguous_strides(shape)), buf.reshape(shape)))
    if len(shape) >= 2:
        tshape = tuple(reversed(shape))
        tbuf = raw(rng.normal(0, 2, n), dt)
        full = tbuf.reshape(tshape)
        st = ox.contiguous_strides(tshape)
        v = dev_view(tbuf, dtype, shape, tuple(reversed(st)))      # a transposed view
        out.append(("transposed", v, np.ascontiguousarray(full.T)))
    pbuf = raw(rng.normal(0, 2, 3 + 2 * n), dt)                     # every other element, offset 3
    st = tuple(2 * s for s in ox.contiguous_strides(shape))
    out.append(("strided", dev_view(pbuf, dtype, shape, st, 3), R.view(pbuf, shape, st, 3)))
    fbuf = raw(rng.normal(0, 2, n), dt)                             # first dim reversed
    st = list(ox.contiguous_strides(shape))
    off = (shape[0] - 1) * st[0]
    st[0] = -st[0]
    out.append(("flipped", dev_view(fbuf, dtype, shape, st, off), R.view(fbuf, shape, st, off)))
    return out


def got(t: ox.Tensor, dt):
    a = t.to_numpy()
    return R.from_f32(a, dt) if dt == R.BF16 else a.astype(NPDT[dt])


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("op", [R.UN_NEG, R.UN_ABS, R.UN_EXP, R.UN_LN], ids=["neg", "abs", "exp", "ln"])
def test_unary(hip, dtype, op):
    dt = DT[dtype]
    rng = np.random.default_rng(10 + op)
    for shape in [(37,), (64, 48), (3, 5, 129)]:
        for name, v, logical in layouts(rng, dtype, shape):
            if op == R.UN_LN:
                logical = R.unary(logical, R.UN_ABS, dt)            # ln of |x| (plus the NaN case below)
                v = v.abs()
            log(f"unary {op} {dtype.name} {shape} {name}")
            out = {R.UN_NEG: v.neg, R.UN_ABS: v.abs, R.UN_EXP: v.exp, R.UN_LN: v.ln}[op]()
            assert out.shape == shape and out.layout.is_contiguous()
            g, ref = R.to_f32(got(out, dt), dt), R.to_f32(R.unary(logical, op, dt), dt)
            if op in (R.UN_NEG, R.UN_ABS):
                assert np.array_equal(g, ref), name
            else:
                # f32 / f64: 4 ulp between the device's exp/log and numpy's
                # float64 result rounded to the dtype; 16-bit: one ulp
                ulp = {R.F32: 4 * 2.0 ** -23, R.F64: 4 * 2.0 ** -52, R.BF16: 2.0 ** -7, R.F16: 2.0 ** -10}[dt]
                tol = ulp * np.abs(ref) + (1e-300 if dt == R.F64 else 1e-38)
                fin = np.isfinite(ref)
                assert np.all(np.abs(g[fin] - ref[fin]) <= tol[fin]), name
                assert np.array_equal(np.isinf(g), np.isinf(ref)) and np.array_equal(np.isnan(g), np.isnan(ref))


@pytest.mark.parametrize("dtype", [ox.DType.F32, ox.DType.BF16], ids=["f32", "bf16"])
def test_unary_special_values(hip, dtype):
    dt = DT[dtype]
    x = ox.Tensor.from_numpy(raw([0.0, -1.0, 1.0, np.inf, -np.inf, 100.0], dt), ox.Device.rocm(0), dtype)
    l = R.to_f32(got(x.ln(), dt), dt)
    assert l[0] == -np.inf and np.isnan(l[1]) and l[2] == 0 and l[3] == np.inf
    e = R.to_f32(got(x.exp(), dt), dt)
    assert e[0] == 1 and e[3] == np.inf and e[4] == 0 and e[5] == np.inf


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("op", [R.BIN_ADD, R.BIN_SUB, R.BIN_MUL, R.BIN_DIV], ids=["add", "sub", "mul", "div"])
def test_binary_broadcasting(hip, dtype, op):
    dt = DT[dtype]
    rng = np.random.default_rng(20 + op)
    cases = [((64, 48), (64, 48)), ((64, 48), (48,)), ((5, 1, 33), (7, 1)), ((), (9, 4)), ((1, 8), (6, 1)),
             ((4, 130), (4, 130)), ((16, 40, 64), (40, 1)), ((256,), (5, 256)), ((3, 1, 96), (1, 7, 96))]
    for sa, sb in cases:
        for (na, va, la), (nb, vb, lb) in zip(layouts(rng, dtype, sa) if sa else [("scalar", dev_view(
                raw([1.5], dt), dtype, (), ()), raw([1.5], dt).reshape(()))], layouts(rng, dtype, sb)):
            log(f"binary {op} {dtype.name} {sa}x{sb} {na}/{nb}")
            out = {R.BIN_ADD: va.add, R.BIN_SUB: va.sub, R.BIN_MUL: va.mul, R.BIN_DIV: va.div}[op](vb)
            ref = R.binary(la, lb, op, dt)
            assert out.shape == ref.shape and out.layout.is_contiguous()
            g = got(out, dt)
            assert np.array_equal(R.to_f32(g, dt), R.to_f32(ref, dt), equal_nan=True), f"{na}/{nb}"


def test_binary_refusals(hip):
    d = ox.Device.rocm(0)
    with pytest.raises(ox.BroadcastIncompatible):
        ox.Tensor.empty((2, 3), ox.DType.F32, d).add(ox.Tensor.empty((4,), ox.DType.F32, d))
    with pytest.raises(ox.DTypeMismatch):
        ox.Tensor.empty((2, 3), ox.DType.F32, d).mul(ox.Tensor.empty((2, 3), ox.DType.BF16, d))
    # integer dtypes carry neg / abs and add / sub / mul / div / eq
    # (tests/test_gpu_int_ops.py); exp and ln are "float dtypes only"
    # (crates/oxmera-ops/src/lib.rs:31-34), Bool has no neg
    with pytest.raises(ox.UnsupportedDType):
        ox.Tensor.empty((2, 3), ox.DType.I32, d).exp()
    with pytest.raises(ox.UnsupportedDType):
        ox.Tensor.empty((2, 3), ox.DType.Bool, d).neg()


def test_division_ieee(hip):
    d = ox.Device.rocm(0)
    a = ox.Tensor.from_numpy(np.array([1, -1, 0], np.float32), d)
    z = ox.Tensor.from_numpy(np.zeros(3, np.float32), d)
    r = a.div(z).to_numpy()
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2])


REDUCE_CASES = [((64, 48), [0]), ((64, 48), [1]), ((64, 48), []), ((3, 5, 129), [0, 2]), ((3, 5, 129), [1]),
                ((7, 300, 9), [1]), ((2, 70000), [1]), ((40000, 3), [0]), ((1 << 21,), []),
                ((3000, 200), [0]), ((300, 1000), [1]), ((9, 40, 3, 100), [0, 2]),
                # one-pass column schedule (at least 256 groups of 128 bytes of outputs)
                ((300, 16384), [0]), ((3, 260, 8192), [1]),
                # a wave per row (at least 1024 rows of whole 16-byte vectors)
                ((1100, 264), [1]), ((3, 400, 520), [2])]


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_reduce_sum(hip, dtype):
    dt = DT[dtype]
    rng = np.random.default_rng(30)
    for shape, axes in REDUCE_CASES:
        for name, v, logical in layouts(rng, dtype, shape)[:2 if len(shape) > 1 else 1] + layouts(rng, dtype, shape)[2:3]:
            log(f"sum {dtype.name} {shape} axes {axes} {name}")
            out = v.sum(axes)
            exact, scale = R.reduce_sum_f64(logical, axes, dt)
            assert out.shape == R.reduced_shape(shape, axes)
            g = R.to_f32(got(out, dt), dt).astype(np.float64)
            n = int(np.prod([shape[a] for a in axes])) if axes else int(np.prod(shape))
            u = 2.0 ** -53 if dt == R.F64 else 2.0 ** -24
            out_ulp = {R.F32: 2.0 ** -24, R.F64: 2.0 ** -53, R.BF16: 2.0 ** -8, R.F16: 2.0 ** -11}[dt]
            bound = n * u * scale + out_ulp * np.abs(exact) + 1e-300
            assert np.all(np.abs(g - exact) <= bound), f"{shape} {axes} {name}"


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_reduce_max(hip, dtype):
    dt = DT[dtype]
    rng = np.random.default_rng(31)
    for shape, axes in REDUCE_CASES:
        for name, v, logical in layouts(rng, dtype, shape)[:2]:
            log(f"max {dtype.name} {shape} axes {axes} {name}")
            out = v.max(axes)
            assert np.array_equal(R.to_f32(got(out, dt), dt), R.to_f32(R.reduce_max(logical, axes, dt), dt))


def test_reduce_nan_empty_and_refusals(hip):
    d = ox.Device.rocm(0)
    x = np.arange(60, dtype=np.float32).reshape(3, 4, 5)
    x[1, 2, 3] = np.nan
    m = ox.Tensor.from_numpy(x, d).max([2]).to_numpy()
    assert np.isnan(m[1, 2]) and m[0, 0] == 4
    e = ox.Tensor.empty((3, 0), ox.DType.F32, d)
    assert e.sum([1]).to_numpy().tolist() == [0, 0, 0]
    with pytest.raises(ox.ShapeMismatch):
        e.max([1])
    with pytest.raises(ox.IndexOutOfBounds):
        ox.Tensor.empty((3, 4), ox.DType.F32, d).sum([2])


@pytest.mark.parametrize("dtype", DTYPES + [ox.DType.I32], ids=IDS + ["i32"])
def test_contiguous(hip, dtype):
    rng = np.random.default_rng(40)
    d = ox.Device.rocm(0)
    if dtype == ox.DType.I32:
        buf = rng.integers(-1000, 1000, 6 * 70 * 33).astype(np.int32)
    else:
        buf = raw(rng.normal(0, 1, 6 * 70 * 33), DT[dtype])
    base = ox.Tensor.from_numpy(buf, d, dtype).reshape((6, 70, 33))
    for name, v, perm in [("permuted", base.permute([2, 0, 1]), (2, 0, 1)), ("narrowed", base.narrow(1, 3, 50), None)]:
        c = v.contiguous()
        assert c.layout.is_contiguous() and c.shape == v.shape
        ref = buf.reshape(6, 70, 33)
        ref = np.transpose(ref, perm) if perm else ref[:, 3:53, :]
        gotv = c.to_numpy()
        if dtype == ox.DType.BF16:
            gotv = R.from_f32(gotv, R.BF16)
        elif dtype == ox.DType.F16:
            gotv = gotv.astype(np.float16)  # exact: the values are f16
        assert np.array_equal(np.ascontiguousarray(gotv).view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), name
    # tiled transposes: batch dims, tiles ragged on both sides
    if dtype == ox.DType.I32:
        buf2 = rng.integers(-1000, 1000, 3 * 100 * 130).astype(np.int32)
    else:
        buf2 = raw(rng.normal(0, 1, 3 * 100 * 130), DT[dtype])
    base2 = ox.Tensor.from_numpy(buf2, d, dtype).reshape((3, 100, 130))
    for perm in [(0, 2, 1), (2, 1, 0), (1, 2, 0)]:
        c = base2.permute(list(perm)).contiguous()
        ref = np.ascontiguousarray(np.transpose(buf2.reshape(3, 100, 130), perm))
        gotv = c.to_numpy()
        if dtype == ox.DType.BF16:
            gotv = R.from_f32(gotv, R.BF16)
        elif dtype == ox.DType.F16:
            gotv = gotv.astype(np.float16)
        assert np.array_equal(np.ascontiguousarray(gotv).view(np.uint8), ref.view(np.uint8)), perm
    # tiled transposes with 16-byte vectors on both sides (2- and 4-byte
    # elements: extents multiples of 8, tiles ragged, a batch dim); 8-byte
    # elements take the element-wise tile
    if dtype == ox.DType.I32:
        buf3 = rng.integers(-1000, 1000, 2 * 96 * 136).astype(np.int32)
    else:
        buf3 = raw(rng.normal(0, 1, 2 * 96 * 136), DT[dtype])
    base3 = ox.Tensor.from_numpy(buf3, d, dtype).reshape((2, 96, 136))
    for perm in [(0, 2, 1), (2, 1, 0), (1, 2, 0)]:
        c = base3.permute(list(perm)).contiguous()
        ref = np.ascontiguousarray(np.transpose(buf3.reshape(2, 96, 136), perm))
        gotv = c.to_numpy()
        if dtype == ox.DType.BF16:
            gotv = R.from_f32(gotv, R.BF16)
        elif dtype == ox.DType.F16:
            gotv = gotv.astype(np.float16)
        assert np.array_equal(np.ascontiguousarray(gotv).view(np.uint8), ref.view(np.uint8)), ("vec", perm)
    same = base.contiguous()
    assert same.data_ptr() == base.data_ptr()                         # a no-op clone when contiguous
