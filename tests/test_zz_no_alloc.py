"""oxm_reduce_noalloc (the reduction entry point that allocates nothing: its
split partials live in the library's static per-GPU scratch) against
oxm_reduce, through the C-ABI: two calls in a row, the second smaller, on
schedules that split (so the scratch is used), and the refusal of a
reduction whose partials do not fit.  No counterpart in the reference; the
bar is oxm_reduce's own result, bit for bit (same kernels, same split
counts)."""
import ctypes as C

import numpy as np
import pytest

import oxmera_amd as ox
from oxmera_amd import _lib
from tests.parity import host_buffer

pytestmark = pytest.mark.gpu

DEV = ox.Device.rocm(0)


def run(fn, op, x, axes):
    ax = (C.c_int32 * max(1, len(axes)))(*axes)
    vx = x.abi_view()
    nd = C.c_int32(0)
    shp = (C.c_int64 * _lib.MAX_DIMS)()
    ox.core.check(_lib.lib().oxm_reduce_infer(C.byref(vx), ax, len(axes), C.byref(nd), shp))
    out = ox.Tensor.empty(tuple(shp[i] for i in range(nd.value)), x.dtype, DEV)
    vo = out.abi_view()
    st = fn(op, C.byref(vx), ax, len(axes), C.byref(vo), None)
    return st, out


@pytest.mark.parametrize("dtype", [ox.DType.F32, ox.DType.BF16, ox.DType.F64], ids=["f32", "bf16", "f64"])
def test_noalloc_reduce_matches_oxm_reduce_twice(hip, dtype):
    rng = np.random.default_rng(71)
    L = _lib.lib()
    # (shape, axes): a column sum (split columns), a row sum (split rows), a max
    cases = [((4096, 4096), [0], _lib.RED_SUM), ((2048, 1024), [0], _lib.RED_SUM),
             ((64, 65536), [1], _lib.RED_SUM), ((16, 32768), [1], _lib.RED_SUM),
             ((3000, 2048), [0], _lib.RED_MAX), ((1000, 512), [0], _lib.RED_MAX)]
    for shape, axes, op in cases:   # each pair: the second call is smaller than the first
        print(f"noalloc {dtype.name} {shape} axes {axes} op {op}", flush=True)
        x = ox.Tensor.from_numpy(host_buffer(dtype, rng.normal(0, 1, shape).astype(np.float32))
                                 if dtype != ox.DType.F64 else rng.normal(0, 1, shape), DEV, dtype)
        st_a, ref = run(L.oxm_reduce, op, x, axes)
        st_b, got = run(L.oxm_reduce_noalloc, op, x, axes)
        assert st_a == _lib.OK and st_b == _lib.OK, _lib.last_error()
        np.testing.assert_array_equal(got.to_numpy(), ref.to_numpy())


def test_noalloc_reduce_refuses_what_does_not_fit(hip):
    # bf16 [8192, 16320] column sums: 255 groups of 64 outputs, one short of
    # the one-pass schedule, so 256 splits x 16320 f32 partials = 16 MiB > 8 MiB
    print("noalloc refusal", flush=True)
    x = ox.Tensor.empty((8192, 16320), ox.DType.BF16, DEV)
    st, _ = run(_lib.lib().oxm_reduce_noalloc, _lib.RED_SUM, x, [0])
    assert st == _lib.E_NOT_IMPLEMENTED
    assert "scratch" in _lib.last_error()
    # the plain entry point still does it, and the no-allocation one still
    # works afterwards
    st, _ = run(_lib.lib().oxm_reduce, _lib.RED_SUM, x, [0])
    assert st == _lib.OK
    y = ox.Tensor.from_numpy(np.arange(4096 * 64, dtype=np.float32).reshape(4096, 64), DEV)
    st_a, ref = run(_lib.lib().oxm_reduce, _lib.RED_SUM, y, [0])
    st_b, got = run(_lib.lib().oxm_reduce_noalloc, _lib.RED_SUM, y, [0])
    assert st_a == st_b == _lib.OK
    np.testing.assert_array_equal(got.to_numpy(), ref.to_numpy())
