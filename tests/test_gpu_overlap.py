"""Outputs that share memory with inputs are refused before any launch
(crates/oxmera-ops/src/lib.rs:16-17: every output is a fresh tensor), except
an elementwise input that is the output element for element (in place);
host copies run in the order of the backend's stream.  Through the C-ABI on
the GPU (the refusals need device allocations to get past the memory checks).
"""
import ctypes as C

import numpy as np
import pytest

import oxmera_amd as ox
from oxmera_amd import _lib

pytestmark = pytest.mark.gpu

DEV = ox.Device.rocm(0)


def dev(arr, dtype=ox.DType.F32):
    return ox.Tensor.from_numpy(np.asarray(arr, np.float32), DEV, dtype)


def st_gemm(a, b, c, ep=None):
    va, vb, vc = a.abi_view(), b.abi_view(), c.abi_view()
    return _lib.lib().oxm_gemm(C.byref(va), C.byref(vb), C.byref(vc), C.byref(ep) if ep else None, None)


def test_gemm_output_overlapping_an_operand_is_refused(hip):
    print("overlap: gemm", flush=True)
    rng = np.random.default_rng(1)
    buf = dev(rng.normal(0, 1, 64 * 64))
    a = buf.with_layout((16, 16), (16, 1), 0)
    b = dev(rng.normal(0, 1, (16, 16)))
    c_over_a = buf.with_layout((16, 16), (16, 1), 128)   # rows 8..23 of the buffer, overlapping a
    assert st_gemm(a, b, c_over_a) == _lib.E_INVALID_ARGUMENT
    assert "overlaps" in _lib.last_error()
    c_over_b = b
    assert st_gemm(a, b, c_over_b) == _lib.E_INVALID_ARGUMENT
    # disjoint parts of one buffer are fine
    c_ok = buf.with_layout((16, 16), (16, 1), 1024)
    assert st_gemm(a, b, c_ok) == _lib.OK
    np.testing.assert_allclose(c_ok.to_numpy(), a.to_numpy() @ b.to_numpy(), rtol=1e-5, atol=1e-5)


def test_gemm_aux_overlapping_the_output_is_refused(hip):
    print("overlap: gemm aux", flush=True)
    rng = np.random.default_rng(2)
    a, b = dev(rng.normal(0, 1, (8, 8))), dev(rng.normal(0, 1, (8, 8)))
    c = dev(np.zeros((8, 8)))
    ep = _lib.OxmEpilogue(None, 0, _lib.ACT_GELU, C.c_void_p(c.data_ptr()), None)
    assert st_gemm(a, b, c, ep) == _lib.E_INVALID_ARGUMENT
    ep = _lib.OxmEpilogue(None, 0, _lib.ACT_GELU, C.c_void_p(a.data_ptr()), None)   # pre-activation over lhs
    assert st_gemm(a, b, c, ep) == _lib.E_INVALID_ARGUMENT


def test_elementwise_in_place_is_allowed_partial_overlap_is_not(hip):
    print("overlap: elementwise", flush=True)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (32, 32)).astype(np.float32)
    y = rng.normal(0, 1, (32, 32)).astype(np.float32)
    a, b = dev(x), dev(y)
    va, vb = a.abi_view(), b.abi_view()
    # a = a + b in place: same elements, same strides
    assert _lib.lib().oxm_binary(_lib.BIN_ADD, C.byref(va), C.byref(vb), C.byref(va), None) == _lib.OK
    np.testing.assert_array_equal(a.to_numpy(), x + y)
    # neg in place
    assert _lib.lib().oxm_unary(_lib.UN_NEG, C.byref(vb), C.byref(vb), None) == _lib.OK
    np.testing.assert_array_equal(b.to_numpy(), -y)
    # output shifted by one element over the input: refused
    buf = dev(rng.normal(0, 1, 1025))
    src = buf.with_layout((32, 32), (32, 1), 0)
    dst = buf.with_layout((32, 32), (32, 1), 1)
    vs, vd = src.abi_view(), dst.abi_view()
    assert _lib.lib().oxm_unary(_lib.UN_ABS, C.byref(vs), C.byref(vd), None) == _lib.E_INVALID_ARGUMENT
    # a transposed view of the output as the input: refused
    vt = src.transpose_last().abi_view()
    assert _lib.lib().oxm_binary(_lib.BIN_MUL, C.byref(vt), C.byref(vs), C.byref(vs), None) == _lib.E_INVALID_ARGUMENT
    # a broadcast row that lives inside the output: refused
    row = buf.with_layout((32,), (1,), 0)
    vr = row.abi_view()
    assert _lib.lib().oxm_binary(_lib.BIN_ADD, C.byref(vs), C.byref(vr), C.byref(vs), None) == _lib.E_INVALID_ARGUMENT


def test_reduce_convert_copy_and_sgd_refuse_overlap(hip):
    print("overlap: reduce/convert/copy/sgd", flush=True)
    rng = np.random.default_rng(4)
    buf = dev(rng.normal(0, 1, 64 * 64))
    x = buf.with_layout((64, 63), (64, 1), 0)
    out = buf.with_layout((64,), (1,), 64 * 63)   # the last row: inside x's byte range
    ax = (C.c_int32 * 1)(1)
    vx, vo = x.abi_view(), out.abi_view()
    assert _lib.lib().oxm_reduce(_lib.RED_SUM, C.byref(vx), ax, 1, C.byref(vo), None) == _lib.E_INVALID_ARGUMENT
    # copy: identical views are a no-op, shifted ones refused
    s = buf.with_layout((32, 32), (32, 1), 0)
    d = buf.with_layout((32, 32), (32, 1), 16)
    vs, vd = s.abi_view(), d.abi_view()
    assert _lib.lib().oxm_copy_view(C.byref(vs), C.byref(vs), None) == _lib.OK
    assert _lib.lib().oxm_copy_view(C.byref(vs), C.byref(vd), None) == _lib.E_INVALID_ARGUMENT
    assert _lib.lib().oxm_convert(C.byref(vs), C.byref(vd), None) == _lib.E_INVALID_ARGUMENT
    # sgd: gradient inside the parameter
    p = buf.with_layout((32, 32), (32, 1), 0)
    g = buf.with_layout((32, 32), (32, 1), 512)
    vp, vg = p.abi_view(), g.abi_view()
    assert _lib.lib().oxm_sgd_step(C.byref(vp), C.byref(vg), None, 0.1, 0.0, 0.0, 0, None) == _lib.E_INVALID_ARGUMENT
    # raw device copy between overlapping ranges
    base = buf.data_ptr()
    assert _lib.lib().oxm_copy(C.c_void_p(base + 16), 0, C.c_void_p(base), 0, 1024, None) == _lib.E_INVALID_ARGUMENT


def _hip_runtime():
    """The HIP runtime library liboxm.so itself uses (already mapped into the
    process), for creating a plain non-blocking stream without torch."""
    for line in open("/proc/self/maps"):
        path = line.split()[-1]
        if "libamdhip64.so" in path and "/torch/" not in path:
            return C.CDLL(path)
    raise RuntimeError("libamdhip64 is not mapped: liboxm.so was not loaded")


def test_host_copies_follow_the_backend_stream(hip):
    """With a non-default backend stream, from_numpy / to_numpy are ordered
    after the kernels queued on it (a recycled block is not overwritten under
    a pending kernel; a read-back sees the finished result)."""
    print("host copies on the backend stream", flush=True)
    rng = np.random.default_rng(5)
    rt = _hip_runtime()
    stream = C.c_void_p()
    assert rt.hipStreamCreateWithFlags(C.byref(stream), 1) == 0  # hipStreamNonBlocking, default priority
    hip.set_stream(stream.value)
    try:
        x = rng.normal(0, 1, (2048, 2048)).astype(np.float32)
        a = dev(x)
        acc = a
        for _ in range(8):                     # queue work that reads a
            acc = hip.add(acc, a)
        got = acc.to_numpy()                   # ordered after the adds
        np.testing.assert_allclose(got, 9 * x, rtol=1e-6, atol=1e-5)
        del a
        b = dev(np.ones((2048, 2048)))         # may reuse a's block: written after the queued reads
        np.testing.assert_array_equal(b.to_numpy(), np.ones((2048, 2048), np.float32))
    finally:
        hip.set_stream(None)
        assert rt.hipStreamSynchronize(stream) == 0
        assert rt.hipStreamDestroy(stream) == 0
