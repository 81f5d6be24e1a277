"""GPU parity of the gfx950 GEMM against the CPU oracle, through the C-ABI.

Configurations from the north star (BASELINE.json "configs"):
  C1  f32 256^3 contiguous, U[-1,1)                 -> checked in full
  C2  f32 4096^3 N(0,1); odd 4097 x 4095 x 4093     -> checked in full + checksums
  C3  bf16 8192^3, B a transposed view [1, 8192]    -> >= 256 seeded rows x all 8192
                                                       columns + full checksums
      (and the same shape and layout with f16 operands)
  C4  f32 batched: A every other row of [32,1024,1024], B [1,1024,768] broadcast
                                                    -> checked in full + per-batch checksums
plus every operand layout the loaders distinguish (K-contiguous, M/N-contiguous,
generic strided, negative strides, offsets) for f32/bf16/f16 at odd sizes in
full, the A4 hand-computed cases, the fused epilogues, and the refusals that
need device memory.  Tolerance (north star): |c-r| <= tol * max(|r|, rms(r)),
tol = 1e-5*sqrt(K) for f32, 1e-2 for bf16/f16 inputs.
"""
import numpy as np
import pytest

import oxmera_amd as ox
from oracle import oracle as O
from tests.parity import (Operand, assert_close, checksum_residuals, contiguous_operand, host_buffer, k_major,
                          sample_rows, spec_tolerance, to_f32)

pytestmark = pytest.mark.gpu

F32, BF16, F16 = ox.DType.F32, ox.DType.BF16, ox.DType.F16


def log(msg):
    print(msg, flush=True)


# ---- A4 spec cases on the GPU (exact) -------------------------------------------

def test_a4_hand_computed_cases(hip):
    d = ox.Device.rocm(0)
    t = lambda v, s: ox.Tensor.from_numpy(np.array(v, np.float32).reshape(s), d)
    assert hip.matmul(t([1, 2, 3, 4], (2, 2)), t([5, 6, 7, 8], (2, 2))).to_numpy().tolist() == [[19, 22], [43, 50]]
    assert hip.matmul(t([1, 2, 3, 4, 5, 6], (2, 3)), t([1, 10, 100], (3, 1))).to_numpy().tolist() == [[321], [654]]
    a = [[1.5, -2.0], [0.25, 4.0]]
    assert hip.matmul(t(a, (2, 2)), t([1, 0, 0, 1], (2, 2))).to_numpy().tolist() == a
    assert hip.matmul(t([3, -1, 2, 7, .5, -4], (2, 3)), t([0] * 6, (3, 2))).to_numpy().tolist() == [[0, 0], [0, 0]]
    bt = t([5, 7, 6, 8], (2, 2)).permute([1, 0])  # transposed view, never copied
    assert hip.matmul(t([1, 2, 3, 4], (2, 2)), bt).to_numpy().tolist() == [[19, 22], [43, 50]]
    # TensorOps route through the registry
    assert t([1, 2, 3, 4], (2, 2)).matmul(t([5, 6, 7, 8], (2, 2))).to_numpy().tolist() == [[19, 22], [43, 50]]


def test_a4_refusals_on_device(hip):
    d = ox.Device.rocm(0)
    with pytest.raises(ox.ShapeMismatch):
        hip.matmul(ox.Tensor.empty((2, 3), F32, d), ox.Tensor.empty((4, 2), F32, d))
    with pytest.raises(ox.RankMismatch):
        hip.matmul(ox.Tensor.empty((6,), F32, d), ox.Tensor.empty((6,), F32, d))
    with pytest.raises(ox.DTypeMismatch):
        hip.matmul(ox.Tensor.empty((2, 3), F32, d), ox.Tensor.empty((3, 2), BF16, d))


@pytest.mark.parametrize("seed", range(8))
def test_transpose_law_and_column_independence(hip, seed):
    rng = np.random.default_rng(seed)
    d = ox.Device.rocm(0)
    a = ox.Tensor.from_numpy(rng.uniform(-8, 8, (2, 3)).astype(np.float32), d)
    b = ox.Tensor.from_numpy(rng.uniform(-8, 8, (3, 2)).astype(np.float32), d)
    x = hip.matmul(a, b).to_numpy().T
    y = hip.matmul(b.permute([1, 0]), a.permute([1, 0])).to_numpy()
    assert np.all(np.abs(x - y) <= 1e-4 * (1 + np.maximum(np.abs(x), np.abs(y))))
    full = hip.matmul(a, b).to_numpy()
    col = hip.matmul(a, b.narrow(1, seed % 2, 1)).to_numpy()
    assert np.all(np.abs(full[:, seed % 2] - col[:, 0]) <= 1e-4 * (1 + np.abs(full[:, seed % 2])))


# ---- every loader layout, full comparison at odd sizes ---------------------------

def make_operand(dtype, kind, rows, cols, seed, which):
    """An operand of logical shape [rows, cols] laid out per `kind`."""
    rng = np.random.default_rng(seed)
    if kind == "row":        # contiguous, last dim unit
        buf = host_buffer(dtype, rng.uniform(-1, 1, rows * cols).astype(np.float32))
        return Operand(dtype, buf, (rows, cols), (cols, 1), 0)
    if kind == "col":        # transposed view: first dim unit
        buf = host_buffer(dtype, rng.uniform(-1, 1, rows * cols).astype(np.float32))
        return Operand(dtype, buf, (rows, cols), (1, rows), 0)
    if kind == "gather":     # every other row of a bigger buffer, with an offset
        buf = host_buffer(dtype, rng.uniform(-1, 1, 5 + 2 * rows * (cols + 3)).astype(np.float32))
        return Operand(dtype, buf, (rows, cols), (2 * (cols + 3), 1), 5)
    if kind == "flip":       # rows reversed (negative stride)
        buf = host_buffer(dtype, rng.uniform(-1, 1, rows * cols).astype(np.float32))
        return Operand(dtype, buf, (rows, cols), (-cols, 1), (rows - 1) * cols)
    if kind == "colgap":     # column-major with a padded leading dim (MN-contiguous, aligned)
        ld = rows + 8
        buf = host_buffer(dtype, rng.uniform(-1, 1, ld * cols).astype(np.float32))
        return Operand(dtype, buf, (rows, cols), (1, ld), 0)
    raise ValueError(kind)


LAYOUTS = ["row", "col", "gather", "flip", "colgap"]
# (64,200,72) and (136,72,200): every extent a multiple of 8 with K not a
# multiple of 64, so the M/N-major direct-to-LDS path runs with a K tail.
SHAPES = [(64, 128, 64), (70, 136, 90), (300, 64, 260), (33, 200, 17), (257, 96, 129), (64, 200, 72),
          (136, 72, 200)]


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("la", LAYOUTS)
@pytest.mark.parametrize("lb", LAYOUTS)
def test_layouts_full(hip, dtype, la, lb):
    for si, (m, k, n) in enumerate(SHAPES):
        a = make_operand(dtype, la, m, k, 1000 + si, "a")
        b = make_operand(dtype, lb, k, n, 2000 + si, "b")
        log(f"layouts {dtype.name} {la}x{lb} M={m} K={k} N={n}")
        c = hip.matmul(a.dev, b.dev)
        ref = O.matmul(a.ora, b.ora)
        assert_close(to_f32(c), ref, spec_tolerance(dtype, k), f"{dtype.name} {la}x{lb} {m}x{k}x{n}")


# ---- every 16-bit tile configuration on edge shapes ---------------------------------
# The dispatcher gives 256x256 tiles only to problems of >= ~256 tiles, so at
# the sizes above every 16-bit GEMM runs 128x128 tiles.  OXM_GEMM_CFG (read by
# the library at each call) forces each configuration onto small shapes with
# ragged edge tiles in M and N and a K tail: 1 = 256x256 direct-to-LDS, 2x4
# waves (the default for large problems); 3 = the same with 2x2 waves; 4 =
# 256x256 register-staged; 6 = 256x256 direct-to-LDS with one wave per SIMD
# and a hand-placed instruction stream; 7 = the same on 16x16x32 MFMAs (K- or
# M/N-major operands: transposing fragment reads for the latter; gathers take
# 6); 2 = 128x128.
TILE_CFGS = {"256": 1, "256_4w": 3, "256_regstaged": 4, "256_1w": 6, "256_1w16": 7, "128": 2}
EDGE_SHAPES = [(300, 200, 264), (264, 136, 520), (64, 72, 64), (520, 64, 8)]


@pytest.mark.parametrize("cfg", list(TILE_CFGS))
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("la,lb", [("row", "col"), ("row", "row"), ("col", "col"), ("colgap", "row"),
                                   ("gather", "col")])
def test_tile_configs_16bit(hip, monkeypatch, cfg, dtype, la, lb):
    monkeypatch.setenv("OXM_GEMM_CFG", str(TILE_CFGS[cfg]))
    for si, (m, k, n) in enumerate(EDGE_SHAPES):
        a = make_operand(dtype, la, m, k, 3000 + si, "a")
        b = make_operand(dtype, lb, k, n, 4000 + si, "b")
        log(f"tile cfg {cfg} {dtype.name} {la}x{lb} M={m} K={k} N={n}")
        c = hip.matmul(a.dev, b.dev)
        assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(dtype, k),
                     f"cfg {cfg} {dtype.name} {la}x{lb} {m}x{k}x{n}")


# f32 the same way (OXM_GEMM_CFG_F32): 0 = 128x128, 5 = 256x256, 8 = 64x64 (the
# dispatcher's choice for problems of at most 64 128x128 tiles), over every
# loader kind the f32 kernels have, ragged rows included.
F32_TILE_CFGS = {"128": 0, "256": 5, "64": 8}
F32_EDGE_SHAPES = [(300, 200, 264), (129, 133, 131), (64, 72, 64), (33, 257, 70)]


@pytest.mark.parametrize("cfg", list(F32_TILE_CFGS))
@pytest.mark.parametrize("la,lb", [("row", "row"), ("row", "col"), ("col", "row"), ("gather", "flip"),
                                   ("colgap", "colgap")])
def test_tile_configs_f32(hip, monkeypatch, cfg, la, lb):
    monkeypatch.setenv("OXM_GEMM_CFG_F32", str(F32_TILE_CFGS[cfg]))
    for si, (m, k, n) in enumerate(F32_EDGE_SHAPES):
        a = make_operand(F32, la, m, k, 5000 + si, "a")
        b = make_operand(F32, lb, k, n, 6000 + si, "b")
        log(f"f32 tile cfg {cfg} {la}x{lb} M={m} K={k} N={n}")
        c = hip.matmul(a.dev, b.dev)
        assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(F32, k),
                     f"f32 cfg {cfg} {la}x{lb} {m}x{k}x{n}")


# ---- the f32 direct-to-LDS kernel (256x256 tiles) ------------------------------------
# For 256x256 f32 tiles of K- or M/N-contiguous, 16-byte aligned operands the
# dispatcher takes the direct-to-LDS kernel (OXM_GEMM_F32_DMA=0 keeps the
# register-staged one), its DMA through global_load_lds when K is a multiple
# of 32 (OXM_GEMM_GLOBAL_DMA=0: the buffer form).  On ragged M/N, K a
# multiple of 32 or not, every K/MN layout pair: the three paths give the
# same numbers, and the oracle's.
F32_DMA_SHAPES = [(300, 256, 264), (264, 200, 520), (1000, 1024, 1000), (64, 96, 68)]


# OXM_GEMM_CFG_F32: 5 = 256x256 tiles, 0 = 128x128 tiles, 9 = 256x192 tiles
# (direct-to-LDS only: with OXM_GEMM_F32_DMA=0 the host takes 256x256
# tiles), 8 = 64x64 tiles (a ring of 8 stages: K of 96-256 fits it, 1024
# refills it)
@pytest.mark.parametrize("cfg", ["5", "0", "9", "8"])
@pytest.mark.parametrize("la,lb", [("row", "row"), ("row", "col"), ("col", "row"), ("col", "col")])
def test_f32_dma_kernel_matches_register_kernel(hip, monkeypatch, la, lb, cfg):
    monkeypatch.setenv("OXM_GEMM_CFG_F32", cfg)
    for si, (m, k, n) in enumerate(F32_DMA_SHAPES):
        a = make_operand(F32, la, m, k, 9000 + si, "a")
        b = make_operand(F32, lb, k, n, 9100 + si, "b")
        log(f"f32 DMA cfg {cfg} {la}x{lb} M={m} K={k} N={n}")
        outs = {}
        for dma, glb in (("0", "1"), ("1", "0"), ("1", "1")):
            monkeypatch.setenv("OXM_GEMM_F32_DMA", dma)
            monkeypatch.setenv("OXM_GEMM_GLOBAL_DMA", glb)
            outs[(dma, glb)] = to_f32(hip.matmul(a.dev, b.dev))
        ref = outs[("0", "1")]
        for key, c in outs.items():
            assert np.array_equal(c, ref), f"{la}x{lb} {m}x{k}x{n}: path {key} differs from the register kernel"
        assert_close(ref, O.matmul(a.ora, b.ora), spec_tolerance(F32, k), f"f32 DMA {la}x{lb} {m}x{k}x{n}")


@pytest.mark.parametrize("cfg", ["5", "0", "9", "8"])
def test_f32_dma_kernel_epilogue(hip, monkeypatch, cfg):
    """Bias + GELU with the pre-activation saved, on the f32 direct-to-LDS
    kernel (K a multiple of 32: the global-load DMA)."""
    monkeypatch.setenv("OXM_GEMM_CFG_F32", cfg)
    rng = np.random.default_rng(31)
    m, k, n = 300, 256, 264
    a = contiguous_operand(F32, rng.normal(0, 1, (m, k)))
    b = make_operand(F32, "row", k, n, 32, "b")
    bias_vals = rng.normal(0, 0.5, n).astype(np.float32)
    bias = ox.Tensor.from_numpy(bias_vals, ox.Device.rocm(0), F32)
    z = ox.Tensor.empty((m, n), F32, ox.Device.rocm(0))
    c = hip.matmul(a.dev, b.dev, bias=bias, act=ox.ACT_GELU, aux=z)
    ref, ref_z = O.matmul(a.ora, b.ora, out_dtype=O.F32, bias=bias_vals, bias_dtype=O.F32, act=O.ACT_GELU,
                          want_aux=True)
    tol = spec_tolerance(F32, k)
    assert_close(to_f32(z), ref_z, tol, "pre-activation")
    assert_close(to_f32(c), ref, tol, "gelu output")


# ---- row strip: the leftover rows of a 256x256-tiled GEMM ----------------------------
# M = 2048 + r with N = 8192: 8 tile-rows x 32 tile-columns fill the 256 CUs
# once, so r <= 16 leftover rows run on the strip kernel instead of a second,
# mostly empty round of tiles (r = 17 does take the second round).  Checked
# on the strip rows, the rows either side of the split, and a few others.
STRIP_CASES = [  # dtype, out dtype, A layout, B layout, M, K, N
    (F32, F32, "row", "row", 2049, 72, 8192),
    (F32, F32, "flip", "row", 2051, 100, 8190),   # 16-byte loads of B, straddling chunk at N
    (F32, F32, "row", "col", 2050, 52, 8188),     # B not N-contiguous: element loads
    (BF16, F32, "row", "col", 2051, 136, 8192),
    (BF16, BF16, "gather", "col", 2064, 64, 8192),
    (F16, F16, "flip", "row", 2053, 40, 8192),
    (F16, F16, "row", "row", 2065, 40, 8192),
    # row-major B and K of at least 4 rows per split: the split-K strip
    (F32, F32, "row", "row", 2050, 300, 8000),
    (F32, F32, "flip", "row", 2063, 4093, 8188),
    (BF16, BF16, "row", "row", 2051, 520, 8192),
]


@pytest.mark.parametrize("case", range(len(STRIP_CASES)))
def test_row_strip(hip, case):
    dtype, out, la, lb, m, k, n = STRIP_CASES[case]
    a = make_operand(dtype, la, m, k, 50 + case, "a")
    b = make_operand(dtype, lb, k, n, 60 + case, "b")
    log(f"row strip {dtype.name}->{out.name} {la}x{lb} M={m} K={k} N={n}")
    c = to_f32(hip.matmul(a.dev, b.dev, out_dtype=out)).reshape(m, n)
    rows = np.unique(np.concatenate([np.arange(2040, m), [0, 1, 777, 1500]])).astype(np.int64)
    odt = {F32: O.F32, BF16: O.BF16, F16: O.F16}[out]
    ref = O.matmul(a.ora, b.ora, rows=rows, out_dtype=odt)
    if out == BF16:
        ref = O.bf16_to_f32(ref)
    elif out == F16:
        ref = ref.view(np.float16).astype(np.float32)
    tol = spec_tolerance(dtype, k) if out == F32 else 1e-2
    assert_close(c[rows], ref, tol, f"strip case {case}")


RAGGED = [(5, 3, 7), (129, 13, 131), (300, 257, 259), (257, 1, 6), (70, 130, 65), (33, 66, 1)]


@pytest.mark.parametrize("a_major", ["k", "m"])
@pytest.mark.parametrize("b_major", ["k", "n"])
def test_f32_ragged_unit_stride_rows(hip, a_major, b_major):
    """f32 operands with unit stride along K (or M/N) whose rows start at any
    4-byte boundary and whose length is not a multiple of 4: they take the
    vector loaders, with the last chunk of each row loaded element by element."""
    for si, (m, k, n) in enumerate(RAGGED):
        rng = np.random.default_rng(77 + si)
        off_a, off_b = 1 + si % 3, 3 - si % 3
        if a_major == "k":   # [m, k] rows of length k, leading dim k + 1
            lda = k + 1
            abuf = host_buffer(F32, rng.uniform(-1, 1, off_a + m * lda).astype(np.float32))
            a = Operand(F32, abuf, (m, k), (lda, 1), off_a)
        else:                # M-contiguous, leading dim m + 3
            lda = m + 3
            abuf = host_buffer(F32, rng.uniform(-1, 1, off_a + k * lda).astype(np.float32))
            a = Operand(F32, abuf, (m, k), (1, lda), off_a)
        if b_major == "n":   # [k, n] rows of length n, leading dim n + 2
            ldb = n + 2
            bbuf = host_buffer(F32, rng.uniform(-1, 1, off_b + k * ldb).astype(np.float32))
            b = Operand(F32, bbuf, (k, n), (ldb, 1), off_b)
        else:                # K-contiguous, leading dim k + 5
            ldb = k + 5
            bbuf = host_buffer(F32, rng.uniform(-1, 1, off_b + n * ldb).astype(np.float32))
            b = Operand(F32, bbuf, (k, n), (1, ldb), off_b)
        log(f"ragged f32 A {a_major}-major B {b_major}-major M={m} K={k} N={n}")
        c = hip.matmul(a.dev, b.dev)
        assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(F32, k), f"ragged {m}x{k}x{n}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_batched_broadcast_small(hip, dtype):
    rng = np.random.default_rng(3)
    # A [3, 2, 37, 40] (every other row), B [2, 40, 45] -> [3, 2, 37, 45]
    abuf = host_buffer(dtype, rng.uniform(-1, 1, 3 * 2 * 74 * 40).astype(np.float32))
    a = Operand(dtype, abuf, (3, 2, 37, 40), (2 * 74 * 40, 74 * 40, 80, 1))
    bbuf = host_buffer(dtype, rng.uniform(-1, 1, 2 * 40 * 45).astype(np.float32))
    b = Operand(dtype, bbuf, (2, 40, 45), (1800, 45, 1))
    c = hip.matmul(a.dev, b.dev)
    assert c.shape == (3, 2, 37, 45)
    assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(dtype, 40), "batched")


# ---- the direct-to-LDS DMA through global_load_lds (K a multiple of 64) ------------
# With K a whole number of 64-k stages the direct-to-LDS kernels issue their
# DMA as global_load_lds_dwordx4, which has no range check: rows (and
# M/N-major column chunks) past the operand's edge read the last valid ones
# and feed only outputs that are never stored.  Ragged M and N on every
# operand layout, each 16-bit configuration that uses it, must give exactly
# the buffer-load path's results (OXM_GEMM_GLOBAL_DMA=0), and the oracle's.
GLOBAL_DMA_SHAPES = [(300, 192, 264), (264, 512, 520), (72, 64, 136), (1000, 1024, 1496)]


@pytest.mark.parametrize("cfg", ["1", "2", "7"])
@pytest.mark.parametrize("la,lb", [("row", "col"), ("row", "row"), ("col", "col"), ("col", "row")])
def test_global_dma_matches_buffer_dma(hip, monkeypatch, cfg, la, lb):
    monkeypatch.setenv("OXM_GEMM_CFG", cfg)
    for si, (m, k, n) in enumerate(GLOBAL_DMA_SHAPES):
        dtype = BF16 if si % 2 == 0 else F16
        a = make_operand(dtype, la, m, k, 7000 + si, "a")
        b = make_operand(dtype, lb, k, n, 8000 + si, "b")
        log(f"global DMA cfg {cfg} {dtype.name} {la}x{lb} M={m} K={k} N={n}")
        monkeypatch.setenv("OXM_GEMM_GLOBAL_DMA", "0")
        c0 = to_f32(hip.matmul(a.dev, b.dev))
        monkeypatch.setenv("OXM_GEMM_GLOBAL_DMA", "1")
        c1 = to_f32(hip.matmul(a.dev, b.dev))
        assert np.array_equal(c0, c1), f"cfg {cfg} {la}x{lb} {m}x{k}x{n}: global and buffer DMA differ"
        assert_close(c1, O.matmul(a.ora, b.ora), spec_tolerance(dtype, k), f"cfg {cfg} {la}x{lb} {m}x{k}x{n}")


def test_global_dma_batched_broadcast(hip, monkeypatch):
    """Batch offsets and a broadcast B on the global-load DMA path."""
    rng = np.random.default_rng(9)
    nb, m, k, n = 3, 200, 128, 136
    abuf = host_buffer(BF16, rng.uniform(-1, 1, nb * m * k).astype(np.float32))
    a = Operand(BF16, abuf, (nb, m, k), (m * k, k, 1))
    bbuf = host_buffer(BF16, rng.uniform(-1, 1, n * k).astype(np.float32))
    b = Operand(BF16, bbuf, (1, k, n), (n * k, 1, k))
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("OXM_GEMM_GLOBAL_DMA", flag)
        outs.append(to_f32(hip.matmul(a.dev, b.dev)))
    assert np.array_equal(outs[0], outs[1])
    assert_close(outs[1], O.matmul(a.ora, b.ora), spec_tolerance(BF16, k), "batched global DMA")


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
def test_batched_direct_to_lds(hip, dtype):
    """Batched 16-bit GEMM whose operands both qualify for the direct-to-LDS
    path: A M-contiguous (a transposed view per batch), B K-contiguous, B
    broadcast over the batch, K with a tail."""
    rng = np.random.default_rng(5)
    nb, m, k, n = 3, 96, 328, 136
    abuf = host_buffer(dtype, rng.uniform(-1, 1, nb * k * m).astype(np.float32))
    a = Operand(dtype, abuf, (nb, m, k), (k * m, 1, m))          # per batch: [m, k] with stride_m = 1
    bbuf = host_buffer(dtype, rng.uniform(-1, 1, n * k).astype(np.float32))
    b = Operand(dtype, bbuf, (1, k, n), (n * k, 1, k))           # [1, k, n], K-contiguous
    c = hip.matmul(a.dev, b.dev)
    assert c.shape == (nb, m, n)
    assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(dtype, k), "batched direct-to-LDS")


def test_zero_sized_and_k_zero(hip):
    d = ox.Device.rocm(0)
    c = hip.matmul(ox.Tensor.empty((0, 5), F32, d), ox.Tensor.empty((5, 3), F32, d))
    assert c.shape == (0, 3)
    a = ox.Tensor.empty((4, 0), F32, d)
    b = ox.Tensor.empty((0, 6), F32, d)
    assert np.array_equal(hip.matmul(a, b).to_numpy(), np.zeros((4, 6), np.float32))


# ---- epilogues --------------------------------------------------------------------

# cfg: None = the dispatcher's choice; "1" / "6" / "7" force the 256x256
# 2x4-wave and the two one-wave-per-SIMD 16-bit kernels (OXM_GEMM_CFG), whose
# epilogues differ in wave tile (128x64 / 128x128) and accumulator layout
# (32x32 / 16x16 blocks)
EPI_CFGS = [None, "1", "6", "7"]


def _force_cfg(monkeypatch, cfg):
    if cfg is not None:
        monkeypatch.setenv("OXM_GEMM_CFG", cfg)


@pytest.mark.parametrize("cfg", EPI_CFGS, ids=["auto", "cfg1", "cfg6", "cfg7"])
@pytest.mark.parametrize("dtype,out", [(F32, F32), (BF16, F32), (BF16, BF16), (F16, F16)],
                         ids=["f32", "bf16-f32", "bf16-bf16", "f16-f16"])
def test_bias_gelu_epilogue(hip, monkeypatch, dtype, out, cfg):
    _force_cfg(monkeypatch, cfg)
    rng = np.random.default_rng(21)
    m, k, n = 130, 192, 200
    a = contiguous_operand(dtype, rng.normal(0, 1, (m, k)))
    b = make_operand(dtype, "col", k, n, 22, "b")
    bias_vals = rng.normal(0, 0.5, n).astype(np.float32)
    bias_buf = host_buffer(dtype, bias_vals)
    bias = ox.Tensor.from_numpy(bias_buf, ox.Device.rocm(0), dtype)
    z = ox.Tensor.empty((m, n), out, ox.Device.rocm(0))
    c = hip.matmul(a.dev, b.dev, out_dtype=out, bias=bias, act=ox.ACT_GELU, aux=z)
    odt = {F32: O.F32, BF16: O.BF16, F16: O.F16}[out]
    ref, ref_z = O.matmul(a.ora, b.ora, out_dtype=odt, bias=bias_buf, bias_dtype={F32: O.F32, BF16: O.BF16,
                                                                                   F16: O.F16}[dtype],
                          act=O.ACT_GELU, want_aux=True)
    widen = (lambda x: O.bf16_to_f32(x)) if out == BF16 else ((lambda x: x.view(np.float16).astype(np.float32))
                                                              if out == F16 else (lambda x: x))
    tol = spec_tolerance(dtype, k) if out == F32 else 1e-2
    assert_close(to_f32(z), widen(ref_z), tol, "pre-activation")
    assert_close(to_f32(c), widen(ref), tol, "gelu output")


def test_gelu_accuracy(hip):
    """The epilogue's GELU and GELU' (Abramowitz & Stegun 7.1.26 normal CDF)
    against float64 erf on a dense grid: a K = 1 f32 GEMM with B = 1 passes
    x through exactly, so C = GELU(x), and with A = B = 1 and aux = x,
    C = GELU'(x).  The method's erf error is <= 1.5e-7; the bound allows
    that plus f32 rounding and the hardware exp/rcp (1 ulp each)."""
    from scipy.special import erf
    d = ox.Device.rocm(0)
    x = np.concatenate([np.linspace(-12, 12, 24001), [0.0, -0.0, 1e-30, -1e-30, 1e-5, -1e-5, 30.0, -30.0, 1e4,
                                                         -1e4]]).astype(np.float32)
    m, n = x.size, 64
    xd = x.astype(np.float64)
    phi = 0.5 * (1.0 + erf(xd / np.sqrt(2.0)))
    g_ref = xd * phi
    dg_ref = phi + xd * np.exp(-0.5 * xd * xd) / np.sqrt(2.0 * np.pi)
    ones_b = ox.Tensor.from_numpy(np.ones((1, n), np.float32), d)
    g = hip.matmul(ox.Tensor.from_numpy(x.reshape(m, 1), d), ones_b, act=ox.ACT_GELU).to_numpy()
    z = ox.Tensor.from_numpy(np.repeat(x.reshape(m, 1), n, axis=1), d)
    dg = hip.matmul(ox.Tensor.from_numpy(np.ones((m, 1), np.float32), d), ones_b, act=ox.ACT_DGELU,
                    aux=z).to_numpy()
    # GELU_GRAD: GELU of x out, GELU'(x) to aux, from one evaluation
    gd_aux = ox.Tensor.empty((m, n), F32, d)
    g2 = hip.matmul(ox.Tensor.from_numpy(x.reshape(m, 1), d), ones_b, act=ox.ACT_GELU_GRAD, aux=gd_aux).to_numpy()
    assert np.array_equal(g2, g), "GELU_GRAD's output differs from GELU's"
    dg2 = gd_aux.to_numpy()
    bound = 1e-6 * np.maximum(1.0, np.abs(xd))
    for got, ref, what in ((g, g_ref, "GELU"), (dg, dg_ref, "GELU'"), (dg2, dg_ref, "GELU_GRAD aux")):
        err = np.abs(got.astype(np.float64) - ref[:, None])
        worst = int(np.argmax(err.max(axis=1) / bound))
        assert np.all(err <= bound[:, None]), f"{what}({x[worst]}) = {got[worst, 0]} vs {ref[worst]}"
    nan = hip.matmul(ox.Tensor.from_numpy(np.full((1, 1), np.nan, np.float32), d),
                     ox.Tensor.from_numpy(np.ones((1, 1), np.float32), d), act=ox.ACT_GELU).to_numpy()
    assert np.isnan(nan).all()


@pytest.mark.parametrize("cfg", EPI_CFGS, ids=["auto", "cfg1", "cfg6", "cfg7"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_dgelu_epilogue(hip, monkeypatch, dtype, cfg):
    _force_cfg(monkeypatch, cfg)
    rng = np.random.default_rng(31)
    m, k, n = 96, 160, 130
    a = contiguous_operand(dtype, rng.normal(0, 1, (m, k)))
    b = make_operand(dtype, "col", k, n, 32, "b")
    zvals = rng.normal(0, 1, (m, n)).astype(np.float32)
    zbuf = host_buffer(dtype, zvals.reshape(-1)).reshape(m, n)
    z = ox.Tensor.from_numpy(zbuf, ox.Device.rocm(0), dtype)
    c = hip.matmul(a.dev, b.dev, out_dtype=dtype, act=ox.ACT_DGELU, aux=z)
    odt = O.F32 if dtype == F32 else O.BF16
    ref = O.matmul(a.ora, b.ora, out_dtype=odt, act=O.ACT_DGELU, aux=zbuf)
    refw = ref if dtype == F32 else O.bf16_to_f32(ref)
    assert_close(to_f32(c), refw, spec_tolerance(dtype, k), "dgelu")


@pytest.mark.parametrize("cfg", EPI_CFGS, ids=["auto", "cfg1", "cfg6", "cfg7"])
@pytest.mark.parametrize("dtype,out", [(F32, F32), (BF16, BF16), (F16, F16)], ids=["f32", "bf16", "f16"])
def test_gelu_grad_epilogue(hip, monkeypatch, dtype, out, cfg):
    """GELU_GRAD: out = GELU(acc + bias), aux = GELU'(acc + bias), both
    rounded to the output dtype, against the oracle."""
    _force_cfg(monkeypatch, cfg)
    rng = np.random.default_rng(23)
    m, k, n = 130, 192, 200
    a = contiguous_operand(dtype, rng.normal(0, 1, (m, k)))
    b = make_operand(dtype, "col", k, n, 24, "b")
    bias_buf = host_buffer(dtype, rng.normal(0, 0.5, n).astype(np.float32))
    bias = ox.Tensor.from_numpy(bias_buf, ox.Device.rocm(0), dtype)
    g = ox.Tensor.empty((m, n), out, ox.Device.rocm(0))
    c = hip.matmul(a.dev, b.dev, out_dtype=out, bias=bias, act=ox.ACT_GELU_GRAD, aux=g)
    odt = {F32: O.F32, BF16: O.BF16, F16: O.F16}[out]
    ref, ref_g = O.matmul(a.ora, b.ora, out_dtype=odt, bias=bias_buf, bias_dtype=odt, act=O.ACT_GELU_GRAD,
                          want_aux=True)
    widen = (lambda x: O.bf16_to_f32(x)) if out == BF16 else ((lambda x: x.view(np.float16).astype(np.float32))
                                                              if out == F16 else (lambda x: x))
    tol = spec_tolerance(dtype, k) if out == F32 else 1e-2
    # GELU' is at most 1.13 in magnitude: the pre-activation's tolerance carries over
    assert_close(to_f32(g), widen(ref_g), 1.13 * tol, "GELU'(pre-activation)")
    assert_close(to_f32(c), widen(ref), tol, "gelu output")


@pytest.mark.parametrize("cfg", EPI_CFGS, ids=["auto", "cfg1", "cfg6", "cfg7"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_mul_aux_epilogue(hip, monkeypatch, dtype, cfg):
    """MUL_AUX: out = acc * aux (no bias), with the column sums of the stored
    output, against the oracle."""
    _force_cfg(monkeypatch, cfg)
    rng = np.random.default_rng(33)
    m, k, n = 96, 160, 136
    a = contiguous_operand(dtype, rng.normal(0, 1, (m, k)))
    b = make_operand(dtype, "col", k, n, 34, "b")
    fbuf = host_buffer(dtype, rng.uniform(0, 1.1, m * n).astype(np.float32)).reshape(m, n)
    f = ox.Tensor.from_numpy(fbuf, ox.Device.rocm(0), dtype)
    cs = ox.Tensor.empty((n,), F32, ox.Device.rocm(0))
    c = hip.matmul(a.dev, b.dev, out_dtype=dtype, act=ox.ACT_MUL_AUX, aux=f, colsum=cs)
    odt = O.F32 if dtype == F32 else O.BF16
    ref = O.matmul(a.ora, b.ora, out_dtype=odt, act=O.ACT_MUL_AUX, aux=fbuf)
    refw = ref if dtype == F32 else O.bf16_to_f32(ref)
    got = to_f32(c)
    assert_close(got, refw, spec_tolerance(dtype, k), "acc * aux")
    _check_colsum(cs, got, "MUL_AUX column sums")


def test_mul_aux_requires_aux(hip):
    d = ox.Device.rocm(0)
    x = ox.Tensor.empty((4, 8), F32, d)
    y = ox.Tensor.empty((8, 4), F32, d)
    with pytest.raises(ox.InvalidArgument):
        hip.matmul(x, y, act=ox.ACT_MUL_AUX)


def _check_colsum(cs: ox.Tensor, out: np.ndarray, what: str):
    """The fused column sums against float64 sums of the stored output, under
    the f32 summation bound rows * 2^-24 * sum |x| (plus a tiny floor)."""
    x = np.asarray(out, np.float64).reshape(-1, out.shape[-1])
    ref = x.sum(0)
    bound = x.shape[0] * 2.0 ** -24 * np.abs(x).sum(0) + 1e-30
    got = cs.to_numpy().astype(np.float64)
    assert got.shape == ref.shape, what
    worst = float(np.max(np.abs(got - ref) / bound))
    assert worst <= 1.0, f"{what}: column sum off by {worst:.3g} x the f32 summation bound"


@pytest.mark.parametrize("cfg", EPI_CFGS, ids=["auto", "cfg1", "cfg6", "cfg7"])
@pytest.mark.parametrize("case", ["f32", "f32_ragged", "bf16_dgelu", "bf16_gelu_bf16out", "f32_batched",
                                  "bf16_256tiles"])
def test_epilogue_column_sums(hip, monkeypatch, case, cfg):
    """colsum = sums over rows (and batches) of the output as stored."""
    _force_cfg(monkeypatch, cfg)
    rng = np.random.default_rng(41)
    d = ox.Device.rocm(0)
    kw = {}
    if case in ("f32", "f32_ragged"):
        m, k, n = (130, 96, 200) if case == "f32" else (77, 45, 131)
        a = contiguous_operand(F32, rng.normal(0, 1, (m, k)))
        b = contiguous_operand(F32, rng.normal(0, 1, (k, n)))
        odt = F32
    elif case == "bf16_dgelu":
        m, k, n = 200, 128, 264
        a = contiguous_operand(BF16, rng.normal(0, 1, (m, k)))
        b = make_operand(BF16, "col", k, n, 43, "b")
        zbuf = host_buffer(BF16, rng.normal(0, 1, m * n).astype(np.float32)).reshape(m, n)
        kw = dict(act=ox.ACT_DGELU, aux=ox.Tensor.from_numpy(zbuf, d, BF16))
        odt = BF16
    elif case == "bf16_gelu_bf16out":
        m, k, n = 136, 64, 200
        a = contiguous_operand(BF16, rng.normal(0, 1, (m, k)))
        b = contiguous_operand(BF16, rng.normal(0, 1, (k, n)))
        bias = ox.Tensor.from_numpy(host_buffer(BF16, rng.normal(0, 1, n).astype(np.float32)), d, BF16)
        kw = dict(bias=bias, act=ox.ACT_GELU, aux=ox.Tensor.empty((m, n), BF16, d))
        odt = BF16
    elif case == "f32_batched":
        m, k, n = 37, 40, 45
        a = Operand(F32, host_buffer(F32, rng.normal(0, 1, 3 * m * k).astype(np.float32)), (3, m, k),
                    (m * k, k, 1))
        b = contiguous_operand(F32, rng.normal(0, 1, (k, n)))
        odt = F32
    else:  # 256x256 direct-to-LDS tiles
        m, k, n = 4096, 128, 4096
        a = contiguous_operand(BF16, rng.normal(0, 1, (m, k)))
        b = make_operand(BF16, "col", k, n, 44, "b")
        odt = BF16
    log(f"colsum {case}")
    cs = ox.Tensor.empty((n,), F32, d)
    c = hip.matmul(a.dev, b.dev, out_dtype=odt, colsum=cs, **kw)
    _check_colsum(cs, to_f32(c), case)


def test_epilogue_column_sums_of_no_rows(hip):
    d = ox.Device.rocm(0)
    cs = ox.Tensor.from_numpy(np.full(7, 5.0, np.float32), d)
    c = hip.matmul(ox.Tensor.empty((0, 3), F32, d), ox.Tensor.empty((3, 7), F32, d), colsum=cs)
    assert c.shape == (0, 7)
    assert cs.to_numpy().tolist() == [0.0] * 7


# ---- refusals that need device memory ------------------------------------------------

def test_view_outside_allocation_is_refused(hip):
    d = ox.Device.rocm(0)
    base = ox.Tensor.empty((64,), F32, d)
    # a [8, 8] view with stride 9 addresses 8*9 - 1 + 1 = 72 > 64 elements
    bad = ox.Tensor(base.storage, ox.Layout((8, 8), (9, 1), 0))
    with pytest.raises(ox.IndexOutOfBounds):
        hip.matmul(bad, ox.Tensor.empty((8, 8), F32, d))


def test_dgelu_requires_aux(hip):
    d = ox.Device.rocm(0)
    with pytest.raises(ox.InvalidArgument):
        hip.matmul(ox.Tensor.empty((4, 4), F32, d), ox.Tensor.empty((4, 4), F32, d), act=ox.ACT_DGELU)


def test_host_operand_is_device_mismatch(hip):
    d = ox.Device.rocm(0)
    with pytest.raises(ox.DeviceMismatch):
        hip.matmul(ox.Tensor.empty((4, 4), F32, ox.Device.cpu()), ox.Tensor.empty((4, 4), F32, d))


# ---- the north-star configurations ------------------------------------------------------

def check_rows(c_dev, a, b, rows, dtype, k, what):
    """The listed flattened rows (all of them with rows=None) against the
    oracle, every column."""
    c = to_f32(c_dev).reshape(-1, c_dev.shape[-1])
    av, bv = k_major(a.ora, b.ora)
    ref = O.matmul(av, bv, rows=rows)
    if rows is None:
        return assert_close(c, ref.reshape(c.shape), spec_tolerance(dtype, k), what)
    return assert_close(c[rows], ref, spec_tolerance(dtype, k), what)


def check_checksums(c_dev, a, b, k, what):
    c = to_f32(c_dev)
    rerr, rscale, cerr, cscale = checksum_residuals(a.logical(), b.logical(), c)
    # rigorous f32 accumulation bound, summed over the row / column
    bound = 1.01 * k * 2.0 ** -24
    assert np.all(rerr <= bound * rscale + 1e-6), f"{what}: row checksum {np.max(rerr / (bound * rscale + 1e-6))}"
    assert np.all(cerr <= bound * cscale + 1e-6), f"{what}: column checksum {np.max(cerr / (bound * cscale + 1e-6))}"


def test_c1_f32_256(hip):
    rng = np.random.default_rng(1)
    a = contiguous_operand(F32, rng.uniform(-1, 1, (256, 256)))
    b = contiguous_operand(F32, rng.uniform(-1, 1, (256, 256)))
    c = hip.matmul(a.dev, b.dev)
    assert_close(to_f32(c), O.matmul(a.ora, b.ora), spec_tolerance(F32, 256), "C1")


@pytest.mark.parametrize("m,k,n", [(4096, 4096, 4096), (4097, 4093, 4095)], ids=["4096", "odd"])
def test_c2_f32(hip, m, k, n):
    rng = np.random.default_rng(2)
    log(f"C2 f32 {m}x{k}x{n}")
    a = contiguous_operand(F32, rng.standard_normal((m, k), dtype=np.float32))
    b = contiguous_operand(F32, rng.standard_normal((k, n), dtype=np.float32))
    c = hip.matmul(a.dev, b.dev)
    log(f"C2 f32 {m}x{k}x{n}: oracle over every output")
    check_rows(c, a, b, None, F32, k, "C2 (every output)")
    check_checksums(c, a, b, k, "C2")


def test_c3_bf16_8192_nt(hip):
    n = 8192
    rng = np.random.default_rng(3)
    log("C3 bf16 8192^3, B transposed view")
    a = Operand(BF16, host_buffer(BF16, rng.normal(0, 0.02, n * n).astype(np.float32)), (n, n), (n, 1))
    b = Operand(BF16, host_buffer(BF16, rng.normal(0, 0.02, n * n).astype(np.float32)), (n, n), (1, n))
    c = hip.matmul(a.dev, b.dev, out_dtype=F32)
    rows = sample_rows(n, 256, 6)
    assert len(rows) >= 256
    log(f"C3: oracle over {len(rows)} rows x all {n} columns")
    check_rows(c, a, b, rows, BF16, n, "C3 rows")
    check_checksums(c, a, b, n, "C3")


def test_c3_f16_8192_nt(hip):
    """configs[2]'s shape and layout with f16 operands (the bench's f16 line;
    the 16x16x32 one-wave kernel's f16 instantiation by default)."""
    n = 8192
    rng = np.random.default_rng(33)
    log("C3 f16 8192^3, B transposed view")
    a = Operand(F16, host_buffer(F16, rng.normal(0, 0.02, n * n).astype(np.float32)), (n, n), (n, 1))
    b = Operand(F16, host_buffer(F16, rng.normal(0, 0.02, n * n).astype(np.float32)), (n, n), (1, n))
    c = hip.matmul(a.dev, b.dev, out_dtype=F32)
    rows = sample_rows(n, 256, 7)
    assert len(rows) >= 256
    log(f"C3 f16: oracle over {len(rows)} rows x all {n} columns")
    check_rows(c, a, b, rows, F16, n, "C3 f16 rows")
    check_checksums(c, a, b, n, "C3 f16")


def test_256x192_shape_with_ragged_rows(hip):
    """C4's shape makes the dispatcher prefer 256x192 tiles, which only the
    direct-to-LDS kernel has; with rows of 67 floats (not 16-byte aligned)
    it takes the register-staged kernel on the tiles it would use without
    256x192 (128x128 here)."""
    rng = np.random.default_rng(44)
    log("256x192-preferred shape with ragged A rows")
    a = contiguous_operand(F32, rng.uniform(-1, 1, (32, 512, 67)))
    b = contiguous_operand(F32, rng.uniform(-1, 1, (1, 67, 768)))
    c = hip.matmul(a.dev, b.dev)
    assert c.shape == (32, 512, 768)
    check_rows(c, a, b, sample_rows(32 * 512, 256, 45), F32, 67, "ragged 256x192 fallback")


def test_c4_batched_broadcast(hip):
    rng = np.random.default_rng(4)
    log("C4 batched broadcast")
    abuf = host_buffer(F32, rng.uniform(-1, 1, 32 * 1024 * 1024).astype(np.float32))
    a = Operand(F32, abuf, (32, 512, 1024), (1048576, 2048, 1))
    b = contiguous_operand(F32, rng.uniform(-1, 1, (1, 1024, 768)))
    c = hip.matmul(a.dev, b.dev)
    assert c.shape == (32, 512, 768)
    log("C4: oracle over every output")
    check_rows(c, a, b, None, F32, 1024, "C4 (every output)")
    check_checksums(c, a, b, 1024, "C4")
