"""Pins the CPU oracle (oracle/oxm_oracle.c) before it is trusted as the checker.

Every check here comes from outside the oracle's own formula:
  * the A4 spec's hand-computed products and laws
    (exercises/a4-reference-matmul/tests/spec.rs:31-130), verbatim;
  * the A2 broadcasting hand cases (exercises/a2-broadcasting/tests/spec.rs:15-54);
  * closed forms (ones . ones = K, diagonal scaling, permutations, rank-1 outer
    products) whose answers are exact in f32;
  * numpy float64 matmul on seeded strided / batched / bf16 operands
    (tests/golden/*.npz), held to the rigorous f32 dot-product error bound
    |fl(sum) - sum| <= K * 2^-24 * sum_k |a_k b_k| (up to O(u^2));
  * scipy's erf for the GELU epilogue and numpy's float16 for the f16 rounding.
A plausible mistake -- a transposed operand, a dropped or repeated k term, a
wrong batch or broadcast index, a sign error in a flipped view -- fails at
least one of them.
"""
from pathlib import Path

import numpy as np
import pytest
from scipy.special import erf

GOLDEN = Path(__file__).resolve().parent / "golden"


def mm(o, a, b, **kw):
    return o.matmul(o.StridedView.contiguous(np.asarray(a, np.float32)),
                    o.StridedView.contiguous(np.asarray(b, np.float32)), **kw)


# ---- A4 spec, verbatim ------------------------------------------------------

def test_hand_computed_2x2(oracle):
    c = mm(oracle, [[1, 2], [3, 4]], [[5, 6], [7, 8]])
    assert c.tolist() == [[19, 22], [43, 50]]


def test_hand_computed_rectangular(oracle):
    c = mm(oracle, [[1, 2, 3], [4, 5, 6]], [[1], [10], [100]])
    assert c.shape == (2, 1) and c.tolist() == [[321], [654]]


def test_identity_leaves_a_matrix_alone(oracle):
    a = [[1.5, -2.0], [0.25, 4.0]]
    assert mm(oracle, a, np.eye(2)).tolist() == a


def test_zero_annihilates(oracle):
    a = [[3.0, -1.0, 2.0], [7.0, 0.5, -4.0]]
    assert mm(oracle, a, np.zeros((3, 2))).tolist() == [[0, 0], [0, 0]]


def test_inner_dimension_mismatch_is_a_typed_error(oracle):
    with pytest.raises(oracle.OracleError) as e:
        mm(oracle, np.ones((2, 3)), np.ones((4, 2)))
    assert e.value.kind == "ShapeMismatch"


def test_non_rank_2_operands_are_refused(oracle):
    a = oracle.StridedView(np.ones(6, np.float32), oracle.F32, [6], [1])
    with pytest.raises(oracle.OracleError):
        oracle.matmul(a, a)


def test_matmul_works_on_a_transposed_view(oracle):
    a = oracle.StridedView.contiguous(np.array([[1, 2], [3, 4]], np.float32))
    b = oracle.StridedView.contiguous(np.array([[5, 7], [6, 8]], np.float32))  # B^T in memory
    c = oracle.matmul(a, b.permute([1, 0]))
    assert c.tolist() == [[19, 22], [43, 50]]


@pytest.mark.parametrize("seed", range(32))
def test_transpose_law(oracle, seed):
    rng = np.random.default_rng(seed)
    a = oracle.StridedView.contiguous(rng.uniform(-8, 8, (2, 3)).astype(np.float32))
    b = oracle.StridedView.contiguous(rng.uniform(-8, 8, (3, 2)).astype(np.float32))
    ab_t = oracle.matmul(a, b).T
    bt_at = oracle.matmul(b.permute([1, 0]), a.permute([1, 0]))
    assert np.all(np.abs(ab_t - bt_at) <= 1e-4 * (1 + np.maximum(np.abs(ab_t), np.abs(bt_at))))


@pytest.mark.parametrize("seed", range(32))
def test_columns_are_independent(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    a = oracle.StridedView.contiguous(rng.uniform(-8, 8, (3, 3)).astype(np.float32))
    bm = rng.uniform(-8, 8, (3, 2)).astype(np.float32)
    b = oracle.StridedView.contiguous(bm)
    j = seed % 2
    full = oracle.matmul(a, b)
    col = oracle.matmul(a, oracle.StridedView(b.buf, oracle.F32, [3, 1], [2, 1], j))  # narrow(1, j, 1)
    assert np.all(np.abs(full[:, j] - col[:, 0]) <= 1e-4 * (1 + np.maximum(np.abs(full[:, j]), np.abs(col[:, 0]))))


# ---- A2 broadcasting hand cases ------------------------------------------------

BROADCAST_OK = [([2, 3], [3], [2, 3]), ([3], [2, 3], [2, 3]), ([2, 1], [1, 3], [2, 3]), ([], [2, 3], [2, 3]),
                ([2, 3], [], [2, 3]), ([], [], []), ([4, 1, 5], [3, 1], [4, 3, 5]), ([1], [1], [1]),
                ([5], [1], [5]), ([0], [1], [0]), ([2, 0], [1, 1], [2, 0])]
BROADCAST_REFUSE = [([2], [3]), ([2, 3], [2, 4]), ([4, 3], [2, 1, 2]), ([0], [2])]


def _oracle_bcast(o, a, b):
    import ctypes as C
    sa = (C.c_int64 * max(1, len(a)))(*a)
    sb = (C.c_int64 * max(1, len(b)))(*b)
    n = C.c_int(0)
    out = (C.c_int64 * 8)()
    st = o.lib().oxm_oracle_broadcast(len(a), sa, len(b), sb, C.byref(n), out)
    return st, [out[i] for i in range(n.value)]


@pytest.mark.parametrize("lhs,rhs,expected", BROADCAST_OK)
def test_oracle_broadcast_hand_cases(oracle, lhs, rhs, expected):
    assert _oracle_bcast(oracle, lhs, rhs) == (0, expected)


@pytest.mark.parametrize("lhs,rhs", BROADCAST_REFUSE)
def test_oracle_broadcast_refusals(oracle, lhs, rhs):
    assert _oracle_bcast(oracle, lhs, rhs)[0] == 2


# ---- closed forms ---------------------------------------------------------------

@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 300, 5), (33, 1000, 17)])
def test_ones_times_ones_is_k(oracle, m, k, n):
    c = mm(oracle, np.ones((m, k)), np.ones((k, n)))
    assert np.all(c == k)


def test_diagonal_scaling_is_exact(oracle):
    rng = np.random.default_rng(7)
    a = rng.normal(size=(9, 6)).astype(np.float32)
    d = rng.normal(size=6).astype(np.float32)
    assert np.array_equal(mm(oracle, a, np.diag(d)), a * d)
    assert np.array_equal(mm(oracle, np.diag(d), a.T), d[:, None] * a.T)


def test_permutation_matrix_permutes_columns(oracle):
    rng = np.random.default_rng(8)
    a = rng.normal(size=(5, 7)).astype(np.float32)
    perm = rng.permutation(7)
    p = np.eye(7, dtype=np.float32)[:, perm]
    assert np.array_equal(mm(oracle, a, p), a[:, perm])


def test_rank_one_outer_product(oracle):
    u = np.arange(1, 6, dtype=np.float32)[:, None]
    v = np.arange(-3, 4, dtype=np.float32)[None, :]
    assert np.array_equal(mm(oracle, u, v), u * v)


def test_brute_force_tiny(oracle):
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, (3, 4)).astype(np.float32)
    b = rng.uniform(-1, 1, (4, 5)).astype(np.float32)
    c = mm(oracle, a, b)
    for i in range(3):
        for j in range(5):
            s = 0.0
            for k in range(4):
                s += float(a[i, k]) * float(b[k, j])
            assert abs(c[i, j] - s) <= 4 * 2.0 ** -24 * sum(abs(float(a[i, k]) * float(b[k, j])) for k in range(4))


def test_k_zero_gives_zeros(oracle):
    a = oracle.StridedView(np.zeros(1, np.float32), oracle.F32, [3, 0], [0, 1])
    b = oracle.StridedView(np.zeros(1, np.float32), oracle.F32, [0, 4], [4, 1])
    assert np.array_equal(oracle.matmul(a, b), np.zeros((3, 4), np.float32))


# ---- golden fixtures (numpy float64) --------------------------------------------

def _load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


GOLDEN_NAMES = ["f32_contiguous", "f32_b_transposed", "f32_a_strided_offset", "f32_negative_stride",
                "f32_batched_broadcast", "f32_batch1_broadcast", "bf16_nt"]


def golden_views(o, g):
    dt = o.BF16 if str(g["dtype"]) == "bf16" else o.F32
    a = o.StridedView(g["a_buf"], dt, g["a_shape"], g["a_strides"], int(g["a_offset"]))
    b = o.StridedView(g["b_buf"], dt, g["b_shape"], g["b_strides"], int(g["b_offset"]))
    return a, b


def dot_bound(g, k):
    """Rigorous f32 bound for a length-k dot product, with 1 % slack for O(u^2)."""
    return 1.01 * k * 2.0 ** -24 * g["absprod"] + 1e-30


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_golden_fixture(oracle, name):
    g = _load(name)
    a, b = golden_views(oracle, g)
    c = oracle.matmul(a, b)
    assert c.shape == g["expected"].shape
    k = int(g["a_shape"][-1])
    err = np.abs(c.astype(np.float64) - g["expected"])
    assert np.all(err <= dot_bound(g, k)), float(np.max(err / dot_bound(g, k)))


def test_golden_sampled_rows_match_full(oracle):
    g = _load("f32_batched_broadcast")
    a, b = golden_views(oracle, g)
    full = oracle.matmul(a, b)
    flat = full.reshape(-1, full.shape[-1])
    rows = np.array([0, 5, 17, 40, flat.shape[0] - 1])
    assert np.array_equal(oracle.matmul(a, b, rows=rows), flat[rows])


def test_golden_bias_gelu_epilogue(oracle):
    g = _load("f32_bias_gelu")
    a, b = golden_views(oracle, g)
    k = int(g["a_shape"][-1])
    c, pre = oracle.matmul(a, b, bias=g["bias"], act=oracle.ACT_GELU, want_aux=True)
    bound = dot_bound(g, k) + 2.0 ** -24 * np.abs(g["preact"])
    assert np.all(np.abs(pre - g["preact"]) <= bound)
    # |d gelu / dz| <= 1.13, plus a few ulps for erf and the products
    assert np.all(np.abs(c - g["gelu"]) <= 1.13 * bound + 4e-7 * np.abs(g["gelu"]) + 1e-7)


def test_dgelu_epilogue_multiplies_by_the_derivative(oracle):
    rng = np.random.default_rng(11)
    a = rng.uniform(-1, 1, (6, 8)).astype(np.float32)
    b = rng.uniform(-1, 1, (8, 5)).astype(np.float32)
    z = rng.normal(size=(6, 5)).astype(np.float32)
    plain = mm(oracle, a, b)
    fused = mm(oracle, a, b, act=oracle.ACT_DGELU, aux=z)
    zd = z.astype(np.float64)
    deriv = 0.5 * (1 + erf(zd / np.sqrt(2))) + zd * np.exp(-zd * zd / 2) / np.sqrt(2 * np.pi)
    assert np.allclose(fused, plain * deriv, rtol=2e-6, atol=1e-7)


def test_gelu_grad_epilogue_saves_the_derivative(oracle):
    """GELU_GRAD: the output is GELU of the pre-activation (as the GELU
    epilogue gives it) and the aux its derivative, against the closed form
    of the pre-activation the GELU epilogue saves."""
    g = _load("f32_bias_gelu")
    a, b = golden_views(oracle, g)
    c1, pre = oracle.matmul(a, b, bias=g["bias"], act=oracle.ACT_GELU, want_aux=True)
    c2, deriv = oracle.matmul(a, b, bias=g["bias"], act=oracle.ACT_GELU_GRAD, want_aux=True)
    assert np.array_equal(c1, c2)
    zd = pre.astype(np.float64)
    exact = 0.5 * (1 + erf(zd / np.sqrt(2))) + zd * np.exp(-zd * zd / 2) / np.sqrt(2 * np.pi)
    assert np.all(np.abs(deriv - exact) <= 1e-6)


def test_mul_aux_epilogue_multiplies_elementwise(oracle):
    rng = np.random.default_rng(12)
    a = rng.uniform(-1, 1, (6, 8)).astype(np.float32)
    b = rng.uniform(-1, 1, (8, 5)).astype(np.float32)
    f = rng.normal(size=(6, 5)).astype(np.float32)
    plain = mm(oracle, a, b)
    fused = mm(oracle, a, b, act=oracle.ACT_MUL_AUX, aux=f)
    # one f32 product of the accumulated sum and the factor, correctly rounded
    assert np.array_equal(fused, (plain.astype(np.float64) * f).astype(np.float32))


# ---- GELU and dtype conversions --------------------------------------------------

def test_gelu_matches_scipy_erf(oracle):
    xs = np.linspace(-8, 8, 2001)
    exact = 0.5 * xs * (1 + erf(xs / np.sqrt(2)))
    got = np.array([oracle.gelu(float(np.float32(x))) for x in xs])
    x32 = xs.astype(np.float32).astype(np.float64)
    exact32 = 0.5 * x32 * (1 + erf(x32 / np.sqrt(2)))
    assert np.all(np.abs(got - exact32) <= 3e-7 * np.maximum(1, np.abs(exact32)))
    assert np.all(np.abs(exact - exact32) < 1e-5)


def test_gelu_odd_part_identity(oracle):
    # gelu(x) - gelu(-x) = x * (Phi(x) + Phi(-x)) = x
    for x in np.linspace(-5, 5, 101, dtype=np.float32):
        assert abs(oracle.gelu(float(x)) - oracle.gelu(float(-x)) - float(x)) <= 1e-6 * max(1, abs(float(x)))


def test_dgelu_matches_closed_form(oracle):
    xs = np.linspace(-6, 6, 1201).astype(np.float32).astype(np.float64)
    exact = 0.5 * (1 + erf(xs / np.sqrt(2))) + xs * np.exp(-xs * xs / 2) / np.sqrt(2 * np.pi)
    got = np.array([oracle.dgelu(float(x)) for x in xs])
    assert np.all(np.abs(got - exact) <= 1e-6)


def test_bf16_rounding_known_bits(oracle):
    import ctypes as C
    L = oracle.lib()
    L.oxm_oracle_f32_to_bf16.restype = C.c_uint16
    L.oxm_oracle_f32_to_bf16.argtypes = [C.c_float]
    cases = {1.0: 0x3F80, 1 + 2 ** -8: 0x3F80, 1 + 3 * 2 ** -8: 0x3F82, -2.0: 0xC000, 0.0: 0x0000,
             1 + 2 ** -8 + 2 ** -20: 0x3F81, float("inf"): 0x7F80, 3.0e38: 0x7F62}
    for x, bits in cases.items():
        assert L.oxm_oracle_f32_to_bf16(x) == bits, (x, hex(L.oxm_oracle_f32_to_bf16(x)))


def test_f16_roundtrip_matches_numpy(oracle):
    import ctypes as C
    L = oracle.lib()
    L.oxm_oracle_f32_to_f16.restype = C.c_uint16
    L.oxm_oracle_f32_to_f16.argtypes = [C.c_float]
    L.oxm_oracle_f16_to_f32.restype = C.c_float
    L.oxm_oracle_f16_to_f32.argtypes = [C.c_uint16]
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.normal(0, 100, 3000), rng.normal(0, 1e-5, 1000), [65504, 65519, 65520, 1e6, -0.0,
                                                                              6e-8, 2.98e-8, 3e-8]]).astype(np.float32)
    for x in xs:
        want = int(np.float32(x).astype(np.float16).view(np.uint16))
        assert L.oxm_oracle_f32_to_f16(float(x)) == want, x
    for bits in range(0, 0x10000, 7):
        h = np.uint16(bits).view(np.float16)
        if np.isnan(h):
            continue
        assert L.oxm_oracle_f16_to_f32(bits) == float(h)


def test_f16_inputs_are_widened_exactly(oracle):
    rng = np.random.default_rng(5)
    a = rng.normal(size=(4, 6)).astype(np.float16)
    b = rng.normal(size=(6, 3)).astype(np.float16)
    c = oracle.matmul(oracle.StridedView.contiguous(a), oracle.StridedView.contiguous(b))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    bound = 1.01 * 6 * 2.0 ** -24 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
    assert np.all(np.abs(c - ref) <= bound)


def test_colsum(oracle):
    rng = np.random.default_rng(6)
    x = rng.uniform(-1, 1, (50, 9)).astype(np.float32)
    got = oracle.colsum(x, oracle.F32)
    bound = 1.01 * 50 * 2.0 ** -24 * np.abs(x).sum(0)
    assert np.all(np.abs(got - x.astype(np.float64).sum(0)) <= bound)


def test_k_major_copies_give_bit_identical_oracle_results(oracle):
    """The full-size GPU checks hand the oracle K-contiguous copies of their
    operands (tests/parity.k_major) for speed; each output is still summed in
    ascending k, so the results must match the original views bit for bit."""
    from tests.parity import k_major
    O = oracle
    rng = np.random.default_rng(12)
    for dt, mk in ((O.F32, lambda x: x.astype(np.float32)), (O.BF16, O.bf16_round)):
        abuf = mk(rng.normal(0, 1, 3 + 2 * 37 * 41))
        bbuf = mk(rng.normal(0, 1, 41 * 29))
        a = O.StridedView(abuf, dt, (37, 41), (2 * 41, 1), 3)           # every other row, offset
        b = O.StridedView(bbuf, dt, (41, 29), (29, 1))                   # row-major B (N-contiguous)
        bt = O.StridedView(bbuf, dt, (29, 41), (41, 1)).permute([1, 0])  # a transposed view
        for bb in (b, bt):
            want = O.matmul(a, bb)
            got = O.matmul(*k_major(a, bb))
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        rows = np.array([0, 5, 36])
        np.testing.assert_array_equal(O.matmul(*k_major(a, b), rows=rows), O.matmul(a, b, rows=rows))
    # batched, broadcast B
    abuf = rng.normal(0, 1, (3, 7, 11)).astype(np.float32)
    bbuf = rng.normal(0, 1, (1, 11, 5)).astype(np.float32)
    a, b = O.StridedView.contiguous(abuf), O.StridedView.contiguous(bbuf)
    np.testing.assert_array_equal(O.matmul(*k_major(a, b)), O.matmul(a, b))
