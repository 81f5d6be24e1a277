"""Shared helpers of the GPU parity tests: device views of seeded host
buffers, the north-star tolerance, and size-independent checksums."""
from __future__ import annotations

import numpy as np

import oxmera_amd as ox
from oracle import oracle as O

DT_ORACLE = {ox.DType.F32: O.F32, ox.DType.BF16: O.BF16, ox.DType.F16: O.F16}


def splitmix_uniform(seed: int, n: int) -> np.ndarray:
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def host_buffer(dtype: ox.DType, values: np.ndarray) -> np.ndarray:
    """The raw host buffer for dtype: f32 array, bf16 bits (RNE) or f16 array."""
    if dtype == ox.DType.F32:
        return np.ascontiguousarray(values, dtype=np.float32)
    if dtype == ox.DType.BF16:
        return O.bf16_round(values)
    return np.ascontiguousarray(values, dtype=np.float16)


def widen(dtype: ox.DType, buf: np.ndarray) -> np.ndarray:
    if dtype == ox.DType.BF16:
        return O.bf16_to_f32(buf)
    return buf.astype(np.float32)


class Operand:
    """The same bytes seen as a device view (product) and an oracle view."""

    def __init__(self, dtype: ox.DType, buf: np.ndarray, shape, strides, offset=0, device=None):
        self.dtype = dtype
        self.buf = buf
        self.shape, self.strides, self.offset = tuple(shape), tuple(strides), int(offset)
        dev = device or ox.Device.rocm(0)
        base = ox.Tensor.from_numpy(buf, dev, dtype)
        self.dev = base.with_layout(self.shape, self.strides, self.offset)
        self.ora = O.StridedView(buf, DT_ORACLE[dtype], self.shape, self.strides, self.offset)

    def logical(self) -> np.ndarray:
        """float64 logical values (host), read through the view."""
        es = self.buf.itemsize
        v = np.lib.stride_tricks.as_strided(self.buf[self.offset:], shape=self.shape,
                                            strides=[s * es for s in self.strides])
        return widen(self.dtype, np.ascontiguousarray(v)).astype(np.float64)


def _materialize(v: O.StridedView) -> np.ndarray:
    """The view's elements (storage dtype) in logical order."""
    es = v.buf.itemsize
    return np.ascontiguousarray(np.lib.stride_tricks.as_strided(v.buf[v.offset:], shape=v.shape,
                                                                strides=[s * es for s in v.strides]))


def k_major(a: O.StridedView, b: O.StridedView) -> tuple[O.StridedView, O.StridedView]:
    """The same logical operands with K contiguous on both sides (A row-major,
    B the transpose of a row-major [.., N, K] copy).  The oracle sums each
    output in ascending k whatever the layout, so its results are bit-for-bit
    those of the original views; only its memory access pattern (and so its
    speed on full-size checks) changes."""
    am = _materialize(a)
    bt = np.ascontiguousarray(np.swapaxes(_materialize(b), -1, -2))
    av = O.StridedView.contiguous(am, a.dtype)
    bv = O.StridedView.contiguous(bt, b.dtype)
    perm = list(range(len(b.shape) - 2)) + [len(b.shape) - 1, len(b.shape) - 2]
    return av, bv.permute(perm)


def contiguous_operand(dtype, values, device=None):
    values = np.asarray(values, dtype=np.float32)
    shape = values.shape
    strides = ox.contiguous_strides(shape)
    return Operand(dtype, host_buffer(dtype, values.reshape(-1)), shape, strides, 0, device)


def to_f32(t: ox.Tensor) -> np.ndarray:
    return t.to_numpy().astype(np.float32)


def spec_tolerance(dtype: ox.DType, k: int, out_dtype: ox.DType = ox.DType.F32) -> float:
    """The north-star tolerance: f32 1e-5*sqrt(K); bf16/f16 inputs 1e-2."""
    if dtype == ox.DType.F32:
        return 1e-5 * np.sqrt(max(k, 1))
    return 1e-2


def assert_close(got: np.ndarray, ref: np.ndarray, tol: float, what: str = "") -> float:
    """|c - r| <= tol * max(|r|, rms(r)) elementwise; returns the worst ratio."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(ref * ref))) or 1e-30
    scale = np.maximum(np.abs(ref), rms)
    ratio = np.abs(got - ref) / (tol * scale)
    worst = float(np.max(ratio))
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert worst <= 1.0, f"{what}: max |c-r|/(tol*max(|r|,rms)) = {worst:.3g} at {np.unravel_index(np.argmax(ratio), ratio.shape)}"
    return worst


def sample_rows(total_rows: int, n: int, seed: int, tile: int = 256) -> np.ndarray:
    """Seeded rows plus the first/last rows and rows at tile boundaries."""
    rng = np.random.default_rng(seed)
    edges = [0, 1, total_rows - 1, total_rows - 2]
    for t in range(tile, total_rows, tile * 7):
        edges += [t - 1, t]
    picks = rng.choice(total_rows, size=min(n, total_rows), replace=False)
    rows = np.unique(np.clip(np.concatenate([picks, edges]), 0, total_rows - 1))
    return rows.astype(np.int64)


def checksum_residuals(a_logical: np.ndarray, b_logical: np.ndarray, c: np.ndarray):
    """Row sums C.1 vs A.(B.1) and column sums 1^T.C vs (1^T.A).B, float64,
    per batch.  Every output element enters one row sum and one column sum.
    Returns (row_err, row_scale, col_err, col_scale)."""
    b1 = b_logical.sum(axis=-1, keepdims=True)                 # [..., K, 1]
    rows_ref = np.matmul(a_logical, b1)[..., 0]                # [..., M]
    a1 = a_logical.sum(axis=-2, keepdims=True)                 # [..., 1, K]
    cols_ref = np.matmul(a1, b_logical)[..., 0, :]             # [..., N]
    rows_got = c.astype(np.float64).sum(axis=-1)
    cols_got = c.astype(np.float64).sum(axis=-2)
    rscale = np.matmul(np.abs(a_logical), np.abs(b_logical).sum(axis=-1, keepdims=True))[..., 0]
    cscale = np.matmul(np.abs(a_logical).sum(axis=-2, keepdims=True), np.abs(b_logical))[..., 0, :]
    return np.abs(rows_got - rows_ref), rscale, np.abs(cols_got - cols_ref), cscale
