"""Host-side tests of the product library that need no GPU.

  * liboxm.so loads and exports every entry point include/oxm.h declares;
  * the C++ host layer's broadcasting follows the A2 spec
    (exercises/a2-broadcasting/tests/spec.rs), refusals carry both operands
    (exercises/a5-error-taxonomy/tests/spec.rs:28-41);
  * matmul's shape rules and typed refusals (exercises/a4-reference-matmul/
    tests/spec.rs:68-83, crates/oxmera-ops/src/lib.rs:9-19) via oxm_gemm_infer
    and oxm_gemm's validation, which runs before any device work;
  * the Python mirror of Layout/DType/views (A1, A3 specs);
  * the registry refuses unregistered devices (crates/oxmera-runtime/tests/harness.rs:9-17).
"""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import oxmera_amd as ox
from oxmera_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "oxm.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_]+\s*\*?\s*(oxm_[a-z0-9_]+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 13
    for n in names:
        assert hasattr(L, n), n
    assert sorted(names) == sorted(_lib.exported_symbols())


def test_version_and_name():
    assert "gfx950" in _lib.lib().oxm_version().decode()
    assert ox.HipBackend(0).name() == "hip-gfx950"


# ---- broadcasting (A2) -----------------------------------------------------------

OK_CASES = [([2, 3], [3], [2, 3]), ([3], [2, 3], [2, 3]), ([2, 1], [1, 3], [2, 3]), ([], [2, 3], [2, 3]),
            ([2, 3], [], [2, 3]), ([], [], []), ([4, 1, 5], [3, 1], [4, 3, 5]), ([1], [1], [1]),
            ([5], [1], [5]), ([0], [1], [0]), ([2, 0], [1, 1], [2, 0])]
REFUSE = [([2], [3]), ([2, 3], [2, 4]), ([4, 3], [2, 1, 2]), ([0], [2])]


@pytest.mark.parametrize("lhs,rhs,expected", OK_CASES)
def test_broadcast_hand_cases(lhs, rhs, expected):
    assert ox.broadcast_shapes(lhs, rhs) == tuple(expected)


@pytest.mark.parametrize("lhs,rhs", REFUSE)
def test_broadcast_refusals_carry_operands(lhs, rhs):
    with pytest.raises(ox.BroadcastIncompatible) as e:
        ox.broadcast_shapes(lhs, rhs)
    assert (e.value.lhs, e.value.rhs) == (tuple(lhs), tuple(rhs))
    assert str(list(lhs)).replace(" ", "") in str(e.value).replace(" ", "")


@pytest.mark.parametrize("seed", range(50))
def test_broadcast_laws(seed):
    rng = np.random.default_rng(seed)
    a = list(rng.integers(0, 4, rng.integers(0, 4)))
    b = list(rng.integers(0, 4, rng.integers(0, 4)))
    try:
        ab = ox.broadcast_shapes(a, b)
    except ox.BroadcastIncompatible:
        ab = None
    try:
        ba = ox.broadcast_shapes(b, a)
    except ox.BroadcastIncompatible:
        ba = None
    assert ab == ba  # commutative, in result and refusal
    assert ox.broadcast_shapes(a, a) == tuple(a)  # idempotent
    assert ox.broadcast_shapes(a, []) == tuple(a)  # scalar identity
    if ab is not None:
        assert len(ab) == max(len(a), len(b))
        for op in (a, b):
            for i, d in enumerate(reversed(op)):
                assert ab[len(ab) - 1 - i] == d or d == 1


# ---- matmul shape rules and typed refusals (no device work) -----------------------

def host_tensor(shape, dtype=ox.DType.F32):
    return ox.Tensor.empty(shape, dtype, ox.Device.cpu())


def infer(a, b):
    nd = C.c_int32(0)
    out = (C.c_int64 * _lib.MAX_DIMS)()
    va, vb = a.abi_view(), b.abi_view()
    ox.core.check(_lib.lib().oxm_gemm_infer(C.byref(va), C.byref(vb), C.byref(nd), out))
    return tuple(out[i] for i in range(nd.value))


def test_infer_rank2_and_batched():
    assert infer(host_tensor([2, 3]), host_tensor([3, 5])) == (2, 5)
    assert infer(host_tensor([32, 512, 1024]), host_tensor([1, 1024, 768])) == (32, 512, 768)
    assert infer(host_tensor([4, 1, 6, 7]), host_tensor([3, 7, 2])) == (4, 3, 6, 2)
    assert infer(host_tensor([6, 7]), host_tensor([5, 7, 2])) == (5, 6, 2)


def test_inner_dimension_mismatch_is_shape_mismatch():
    with pytest.raises(ox.ShapeMismatch) as e:
        infer(host_tensor([2, 3]), host_tensor([4, 2]))
    assert "matmul" in str(e.value)


def test_rank1_operands_are_refused():
    with pytest.raises(ox.RankMismatch):
        infer(host_tensor([6]), host_tensor([6]))


def test_dtype_mismatch():
    with pytest.raises(ox.DTypeMismatch):
        infer(host_tensor([2, 3]), host_tensor([3, 2], ox.DType.BF16))


def test_batch_broadcast_refusal():
    with pytest.raises(ox.BroadcastIncompatible):
        infer(host_tensor([2, 3, 4]), host_tensor([3, 4, 5]))


def gemm_status(a, b, c, ep=None):
    va, vb, vc = a.abi_view(), b.abi_view(), c.abi_view()
    return _lib.lib().oxm_gemm(C.byref(va), C.byref(vb), C.byref(vc), C.byref(ep) if ep else None, None)


def test_host_views_are_refused_before_any_launch():
    st = gemm_status(host_tensor([2, 3]), host_tensor([3, 2]), host_tensor([2, 2]))
    assert st == _lib.E_DEVICE_MISMATCH
    assert "matmul" in _lib.last_error()


def test_unsupported_dtype():
    st = gemm_status(host_tensor([2, 3], ox.DType.I32), host_tensor([3, 2], ox.DType.I32), host_tensor([2, 2]))
    assert st == _lib.E_UNSUPPORTED_DTYPE


def test_output_shape_and_dtype_checked():
    assert gemm_status(host_tensor([2, 3]), host_tensor([3, 2]), host_tensor([2, 3])) == _lib.E_SHAPE_MISMATCH
    assert gemm_status(host_tensor([2, 3]), host_tensor([3, 2]),
                       host_tensor([2, 2], ox.DType.BF16)) == _lib.E_DTYPE_MISMATCH


def test_non_contiguous_output_refused():
    c = host_tensor([2, 2]).transpose_last()
    assert gemm_status(host_tensor([2, 3]), host_tensor([3, 2]), c) == _lib.E_NOT_IMPLEMENTED


def test_bad_epilogue_refused():
    a, b, c = host_tensor([2, 3]), host_tensor([3, 2]), host_tensor([2, 2])
    ep = _lib.OxmEpilogue(None, 0, 7, None)
    assert gemm_status(a, b, c, ep) in (_lib.E_INVALID_ARGUMENT, _lib.E_DEVICE_MISMATCH)
    # MUL_AUX without its factor
    ep = _lib.OxmEpilogue(None, 0, _lib.ACT_MUL_AUX, None)
    assert gemm_status(a, b, c, ep) in (_lib.E_INVALID_ARGUMENT, _lib.E_DEVICE_MISMATCH)


def test_null_view_is_invalid_argument():
    nd = C.c_int32(0)
    out = (C.c_int64 * _lib.MAX_DIMS)()
    assert _lib.lib().oxm_gemm_infer(None, None, C.byref(nd), out) == _lib.E_INVALID_ARGUMENT


def test_alloc_on_host_device_refused():
    p = C.c_void_p()
    assert _lib.lib().oxm_alloc(-1, 16, C.byref(p)) == _lib.E_DEVICE_MISMATCH


# ---- Python mirror: Layout / DType (A1) and views (A3) ---------------------------------

def test_dtype_sizes_and_classes():
    sizes = {ox.DType.F32: 4, ox.DType.F64: 8, ox.DType.I32: 4, ox.DType.I64: 8, ox.DType.U8: 1,
             ox.DType.Bool: 1, ox.DType.BF16: 2, ox.DType.F16: 2}
    for dt, n in sizes.items():
        assert dt.size_in_bytes() == n
    assert [dt.is_float() for dt in sizes] == [True, True, False, False, False, False, True, True]


def test_contiguous_strides_hand_cases():
    assert ox.contiguous_strides([]) == ()
    assert ox.contiguous_strides([4]) == (1,)
    assert ox.contiguous_strides([2, 3]) == (3, 1)
    assert ox.contiguous_strides([2, 1, 3]) == (3, 3, 1)
    assert ox.contiguous_strides([4, 2, 3]) == (6, 3, 1)


def test_offset_of_hand_cases_and_errors():
    L = ox.Layout.contiguous([2, 3])
    assert [L.offset_of(i) for i in ([0, 0], [0, 2], [1, 0], [1, 2])] == [0, 2, 3, 5]
    assert ox.Layout.contiguous([]).offset_of([]) == 0
    with pytest.raises(ox.RankMismatch) as e:
        L.offset_of([0])
    assert (e.value.index_rank, e.value.shape_rank) == (1, 2)
    with pytest.raises(ox.IndexOutOfBounds) as e:
        L.offset_of([0, 3])
    assert "[0, 3]" in str(e.value)


def test_contiguity_hand_cases():
    assert ox.Layout.contiguous([2, 3]).is_contiguous()
    assert ox.Layout.contiguous([]).is_contiguous()
    assert ox.Layout.contiguous([0, 3]).is_contiguous()
    assert not ox.Layout((2, 3), (1, 2), 0).is_contiguous()


def t23():
    return ox.Tensor.from_vec_f32([1, 2, 3, 4, 5, 6], [2, 3])


def test_views_share_storage_and_read_through():
    t = t23()
    tt = t.permute([1, 0])
    assert tt.shape == (3, 2) and tt.storage is t.storage
    assert [tt.get_f32(i) for i in ([0, 0], [0, 1], [1, 0], [2, 1])] == [1, 4, 2, 6]
    n = t.narrow(1, 1, 2)
    assert n.storage is t.storage and n.to_numpy().tolist() == [[2, 3], [5, 6]]
    r = t.reshape([3, 2])
    assert r.storage is t.storage and r.to_numpy().tolist() == [[1, 2], [3, 4], [5, 6]]


def test_view_errors_are_typed():
    t = t23()
    with pytest.raises(ox.OxmError):
        t.permute([0, 0])
    with pytest.raises(ox.OxmError):
        t.permute([0])
    with pytest.raises(ox.OxmError):
        t.narrow(1, 2, 2)
    with pytest.raises(ox.OxmError):
        t.narrow(2, 0, 1)
    with pytest.raises(ox.ShapeMismatch):
        t.reshape([4, 2])
    with pytest.raises(ox.ShapeMismatch):
        ox.Tensor.from_vec_f32([1.0] * 5, [2, 3])


def test_from_storage_rejects_out_of_range_layouts():
    t = t23()
    with pytest.raises(ox.IndexOutOfBounds):
        ox.Tensor.from_storage(t.storage, ox.Layout((2, 3), (3, 1), 1))
    with pytest.raises(ox.IndexOutOfBounds):
        ox.Tensor.from_storage(t.storage, ox.Layout((2, 3), (-3, 1), 0))
    flipped = ox.Tensor.from_storage(t.storage, ox.Layout((2, 3), (-3, 1), 3))
    assert flipped.to_numpy().tolist() == [[4, 5, 6], [1, 2, 3]]


def test_unregistered_device_is_backend_unavailable():
    with pytest.raises(ox.BackendUnavailable):
        ox.backend_for(ox.Device.rocm(7))
    with pytest.raises(ox.BackendUnavailable):
        ox.backend_for(ox.Device.cpu())


def test_bf16_host_rounding_matches_oracle(oracle):
    rng = np.random.default_rng(1)
    x = rng.normal(size=10000).astype(np.float32)
    assert np.array_equal(ox.f32_to_bf16_bits(x), oracle.bf16_round(x))


def test_from_numpy_keeps_rank_zero():
    import oxmera_amd as ox
    t = ox.Tensor.from_numpy(np.array(2.5, np.float32), ox.Device.cpu())
    assert t.shape == () and t.to_numpy().shape == () and float(t.to_numpy()) == 2.5


# ---- view byte ranges: overflow-checked (Tensor::from_storage's rule) ----------------

def raw_view(shape, strides, offset=0, dtype=ox.DType.F32):
    shp, st = _lib.i64_array(shape), _lib.i64_array(strides)
    v = _lib.OxmView(C.c_void_p(0x1000), int(dtype), len(shape), C.cast(shp, C.POINTER(C.c_int64)),
                     C.cast(st, C.POINTER(C.c_int64)), int(offset), 0)
    v._keep = (shp, st)
    return v


def byte_range(v):
    lo, hi = C.c_int64(0), C.c_int64(0)
    st = _lib.lib().oxm_view_byte_range(C.byref(v), C.byref(lo), C.byref(hi))
    return st, lo.value, hi.value


def brute_range(shape, strides, offset, es):
    """Every element's byte offset, enumerated (tiny views only)."""
    offs = [offset]
    for d, s in zip(shape, strides):
        offs = [o + i * s for o in offs for i in range(d)]
    return (min(offs) * es, (max(offs) + 1) * es) if offs and all(shape) else (0, 0)


@pytest.mark.parametrize("shape,strides,offset,dtype", [
    ([2, 3], [3, 1], 0, ox.DType.F32), ([2, 3], [1, 2], 5, ox.DType.BF16), ([3, 4], [-4, 1], 8, ox.DType.F32),
    ([2, 2, 2], [0, -1, 7], 3, ox.DType.F64), ([5], [-2], 9, ox.DType.U8), ([0, 4], [4, 1], 0, ox.DType.F32),
    ([], [], 6, ox.DType.I64), ([1, 1], [99, -99], 2, ox.DType.F16)])
def test_view_byte_range_matches_enumeration(shape, strides, offset, dtype):
    st, lo, hi = byte_range(raw_view(shape, strides, offset, dtype))
    assert st == _lib.OK
    assert (lo, hi) == brute_range(shape, strides, offset, dtype.size_in_bytes())


@pytest.mark.parametrize("shape,strides,offset", [
    ([2], [2 ** 61], 0),                  # (hi + 1) * 4 wraps to a negative byte count
    ([3], [2 ** 62], 0),                  # the span itself overflows
    ([2, 2], [-(2 ** 62), -(2 ** 62)], 0),  # the low end underflows
    ([2], [1], 2 ** 63 - 1),              # offset + span overflows
])
def test_view_byte_range_refuses_overflow(shape, strides, offset):
    st, _, _ = byte_range(raw_view(shape, strides, offset))
    assert st == _lib.E_INDEX_OUT_OF_BOUNDS
    assert "overflow" in _lib.last_error()


def test_element_count_overflow_is_refused():
    # 2^32 * 2^32 elements wraps int64 to 0: a view that would otherwise look empty
    v = raw_view([2 ** 32, 2 ** 32], [1, 1])
    st, _, _ = byte_range(v)
    assert st == _lib.E_INDEX_OUT_OF_BOUNDS
    a = raw_view([2 ** 32, 2 ** 32], [1, 1])
    b = raw_view([2 ** 32, 2], [2, 1])
    nd = C.c_int32(0)
    out = (C.c_int64 * _lib.MAX_DIMS)()
    assert _lib.lib().oxm_gemm_infer(C.byref(a), C.byref(b), C.byref(nd), out) == _lib.E_INDEX_OUT_OF_BOUNDS


def test_epilogue_buffers_are_checked_on_the_host():
    """bias / aux / colsum travel as raw pointers: Backend.matmul checks their
    dtype, shape and layout before the call (typed errors, no device work)."""
    be = ox.HipBackend(0)
    a, b = host_tensor([4, 3]), host_tensor([3, 8])
    with pytest.raises(ox.ShapeMismatch):
        be.matmul(a, b, bias=host_tensor([4]))
    with pytest.raises(ox.DTypeMismatch):
        be.matmul(a, b, bias=host_tensor([8], ox.DType.I32))
    with pytest.raises(ox.DTypeMismatch):
        be.matmul(a, b, act=_lib.ACT_GELU, aux=host_tensor([4, 8], ox.DType.F16))
    with pytest.raises(ox.NotImplementedOp):
        be.matmul(a, b, act=_lib.ACT_GELU, aux=host_tensor([8, 4]).transpose_last())
    with pytest.raises(ox.ShapeMismatch):
        be.matmul(a, b, colsum=host_tensor([4]))


# ---- the Rust binding crates (rust/, source only: no cargo in this image) -------------

def test_rust_sys_crate_declares_every_entry_point():
    """rust/oxmera-hip-sys binds exactly the functions include/oxm.h declares."""
    src = (ROOT / "rust" / "oxmera-hip-sys" / "src" / "lib.rs").read_text()
    declared = sorted(set(re.findall(r"pub fn (oxm_[a-z0-9_]+)\s*\(", src)))
    assert declared == header_functions()
    # the status codes agree with the header's enum
    hdr = (ROOT / "include" / "oxm.h").read_text()
    for name, val in re.findall(r"(OXM_E_[A-Z_]+) = (\d+)", hdr):
        assert re.search(rf"pub const {name}: oxm_status = {val};", src), name


def test_rust_safe_crate_maps_every_status():
    """oxmera-hip's check() names each Error variant (error.rs:14-102) for its
    status code."""
    src = (ROOT / "rust" / "oxmera-hip" / "src" / "lib.rs").read_text()
    body = src[src.index("fn check("):src.index("// ---- device storage")]
    for code, variant in [("OXM_E_SHAPE_MISMATCH", "ShapeMismatch"), ("OXM_E_BROADCAST_INCOMPATIBLE",
                          "BroadcastIncompatible"), ("OXM_E_DTYPE_MISMATCH", "DTypeMismatch"),
                          ("OXM_E_UNSUPPORTED_DTYPE", "UnsupportedDType"), ("OXM_E_DEVICE_MISMATCH", "DeviceMismatch"),
                          ("OXM_E_INDEX_OUT_OF_BOUNDS", "IndexOutOfBounds"), ("OXM_E_RANK_MISMATCH", "RankMismatch"),
                          ("OXM_E_BACKEND_UNAVAILABLE", "BackendUnavailable"),
                          ("OXM_E_NOT_IMPLEMENTED", "NotImplemented")]:
        assert re.search(rf"sys::{code} => Err\(Error::{variant}\b", body), code
    for trait in ("UnaryOps", "BinaryOps", "MatmulOps", "ReduceOps", "Backend"):
        assert f"impl {trait} for HipBackend" in src, trait
