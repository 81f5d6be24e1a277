"""Pinning of the gradient and SGD oracle (oracle/autograd_ref.py) on the CPU.

Every vector-Jacobian product is checked against central finite
differences in float64 (directional derivatives along random directions);
max's tie rule, the broadcast sums and SGD by closed forms.
"""
import numpy as np
import pytest

from oracle import autograd_ref as G
from oracle import oracle as O


def fd_check(f, args, grads, g, eps=1e-6, seed=0):
    """<dL/dx_i, u> == (L(x_i + eps u) - L(x_i - eps u)) / 2 eps, L = sum(f * g)."""
    rng = np.random.default_rng(seed)
    for i, gi in enumerate(grads):
        u = rng.normal(0, 1, args[i].shape)
        hi = [a.copy() for a in args]
        lo = [a.copy() for a in args]
        hi[i] = hi[i] + eps * u
        lo[i] = lo[i] - eps * u
        fd = (np.sum(f(*hi) * g) - np.sum(f(*lo) * g)) / (2 * eps)
        an = np.sum(gi * u)
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (i, fd, an)


@pytest.mark.parametrize("op", [G.ADD, G.SUB, G.MUL, G.DIV])
@pytest.mark.parametrize("sa,sb", [((4, 5), (4, 5)), ((3, 4, 5), (5,)), ((4, 1), (1, 6)), ((2, 1, 3), (4, 1))])
def test_binary_vjp_fd(op, sa, sb):
    rng = np.random.default_rng(op)
    a = rng.normal(0, 1, sa)
    b = rng.normal(0, 1, sb) + 3.0 * np.sign(rng.normal(0, 1, sb))   # away from 0 for div
    g = rng.normal(0, 1, np.broadcast_shapes(sa, sb))
    ga, gb = G.vjp_binary(op, a, b, g)
    assert ga.shape == a.shape and gb.shape == b.shape
    fd_check(lambda x, y: G.binary(op, x, y), [a, b], [ga, gb], g)


@pytest.mark.parametrize("op", [G.NEG, G.EXP, G.LN, G.ABS])
def test_unary_vjp_fd(op):
    rng = np.random.default_rng(10 + op)
    a = rng.uniform(0.5, 2.0, (6, 7)) * (1 if op == G.LN else np.sign(rng.normal(0, 1, (6, 7))))
    g = rng.normal(0, 1, a.shape)
    fd_check(lambda x: G.unary(op, x), [a], [G.vjp_unary(op, a, g)], g)


@pytest.mark.parametrize("axes", [[0], [1], [0, 2], []])
def test_reduce_vjp_fd(axes):
    rng = np.random.default_rng(20)
    a = rng.normal(0, 1, (3, 4, 5))
    ax = tuple(axes) if axes else (0, 1, 2)
    g = rng.normal(0, 1, np.sum(a, axis=ax).shape)
    fd_check(lambda x: np.sum(x, axis=ax), [a], [G.vjp_sum(a, axes, g)], g)
    fd_check(lambda x: np.max(x, axis=ax), [a], [G.vjp_max(a, axes, g)], g)   # distinct values: no ties


def test_max_ties_share():
    a = np.array([[1.0, 3.0, 3.0], [2.0, 2.0, 0.0]])
    assert G.vjp_max(a, [1], np.array([1.0, 4.0])).tolist() == [[0, 0.5, 0.5], [2, 2, 0]]
    assert G.vjp_max(a, [], np.array(6.0)).tolist() == [[0, 3, 3], [0, 0, 0]]


@pytest.mark.parametrize("sa,sb", [((5, 7), (7, 3)), ((2, 5, 7), (7, 3)), ((4, 5, 7), (1, 7, 3)), ((3, 1, 5, 7), (2, 7, 4))])
def test_matmul_vjp_fd(sa, sb):
    rng = np.random.default_rng(30)
    a, b = rng.normal(0, 1, sa), rng.normal(0, 1, sb)
    g = rng.normal(0, 1, (a @ b).shape)
    ga, gb = G.vjp_matmul(a, b, g)
    assert ga.shape == a.shape and gb.shape == b.shape
    fd_check(lambda x, y: x @ y, [a, b], [ga, gb], g)


def test_linear_gelu_vjp_fd():
    rng = np.random.default_rng(40)
    x, w, b = rng.normal(0, 1, (6, 5)), rng.normal(0, 0.5, (5, 4)), rng.normal(0, 0.5, 4)
    g = rng.normal(0, 1, (6, 4))
    fd_check(lambda x_, w_, b_: G.gelu(x_ @ w_ + b_), [x, w, b], list(G.vjp_linear_gelu(x, w, b, g)), g)


def test_unbroadcast_closed_form():
    g = np.ones((2, 3, 4))
    assert G.unbroadcast(g, (4,)).tolist() == [6.0] * 4
    assert G.unbroadcast(g, (3, 1)).tolist() == [[8.0]] * 3


# ---- SGD ---------------------------------------------------------------------------

def test_sgd_plain_exact():
    p = np.array([1.0, -2.0, 0.5], np.float32)
    g = np.array([0.5, 0.25, -4.0], np.float32)
    new, v = G.sgd_step(p, O.F32, g, None, lr=0.5)
    assert new.tolist() == [0.75, -2.125, 2.5] and v is None


def test_sgd_momentum_geometric():
    # constant g, mu = 1/2: v_t = g (2 - 2^(1-t)); all values dyadic, so exact
    p, v = np.zeros(4, np.float32), np.zeros(4, np.float32)
    g = np.full(4, 1.0, np.float32)
    total = 0.0
    for t in range(1, 6):
        p, v = G.sgd_step(p, O.F32, g, v, lr=0.25, momentum=0.5)
        assert v[0] == 2 - 2.0 ** (1 - t)
        total += 0.25 * (2 - 2.0 ** (1 - t))
        assert p[0] == -total


def test_sgd_nesterov_and_weight_decay():
    p, v = np.array([2.0], np.float32), np.zeros(1, np.float32)
    # weight decay with zero gradient: p (1 - lr wd)
    q, _ = G.sgd_step(p, O.F32, np.zeros(1, np.float32), None, lr=0.5, weight_decay=0.25)
    assert q[0] == 2.0 * (1 - 0.125)
    # Nesterov, first step from v = 0: v = g, update g + mu g
    q, v1 = G.sgd_step(p, O.F32, np.array([1.0], np.float32), v, lr=0.5, momentum=0.5, nesterov=True)
    assert v1[0] == 1.0 and q[0] == 2.0 - 0.5 * 1.5


def test_sgd_rounds_param_once():
    # bf16 param 1.0, update -2^-9: f32 result 1 - 2^-9 rounds (RNE) back to 1.0 in bf16
    p = O.bf16_round(np.array([1.0], np.float32))
    new, _ = G.sgd_step(p, O.BF16, np.array([2.0 ** -9], np.float32), None, lr=1.0)
    assert new[0] == 0x3F80
    new, _ = G.sgd_step(p, O.BF16, np.array([2.0 ** -7], np.float32), None, lr=1.0)
    assert O.bf16_to_f32(new)[0] == 1 - 2.0 ** -7
    h = np.array([1.0], np.float16)
    new, _ = G.sgd_step(h, O.F16, np.array([2.0 ** -12], np.float32), None, lr=1.0)
    assert new[0] == np.float16(1.0)
