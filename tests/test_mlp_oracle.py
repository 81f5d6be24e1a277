"""Pins the MLP reference used to check the GPU training step.

  * the float64 analytic gradient (oracle/mlp_ref.step_float64) against
    central finite differences of the float64 loss -- the chain rule, GELU'
    and the MSE scaling are fixed by mathematics, not by the code under test;
  * the bf16-rounded oracle step (step_oracle, built from the oracle GEMM)
    against that float64 step, within bf16 tolerance.
"""
import numpy as np
import pytest

from oracle import mlp_ref as R
from oracle import oracle as O


def tiny_model(seed, n=6, d=5, h=7):
    rng = np.random.default_rng(seed)
    return (rng.normal(0, 1, (n, d)), rng.normal(0, 0.5, (d, h)), rng.normal(0, 0.3, h),
            rng.normal(0, 0.5, (h, d)), rng.normal(0, 0.3, d), rng.normal(0, 1, (n, d)))


@pytest.mark.parametrize("seed", range(3))
def test_float64_gradient_matches_finite_differences(seed):
    x, w1, b1, w2, b2, t = tiny_model(seed)
    g = R.step_float64(x, w1, b1, w2, b2, t)
    params = dict(x=x, w1=w1, b1=b1, w2=w2, b2=b2)
    grads = dict(x=g["dx"], w1=g["dw1"], b1=g["db1"], w2=g["dw2"], b2=g["db2"])
    eps = 1e-6
    for name, p in params.items():
        fd = np.zeros_like(p)
        it = np.nditer(p, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            old = p[i]
            p[i] = old + eps
            lp = R.loss_float64(x, w1, b1, w2, b2, t)
            p[i] = old - eps
            lm = R.loss_float64(x, w1, b1, w2, b2, t)
            p[i] = old
            fd[i] = (lp - lm) / (2 * eps)
        assert np.allclose(grads[name], fd, rtol=1e-5, atol=1e-8), name


def bf16(a):
    return O.bf16_round(np.asarray(a, np.float32))


def rel_close(got, ref, tol):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) or 1e-30
    return float(np.max(np.abs(got - ref) / (tol * np.maximum(np.abs(ref), rms))))


@pytest.mark.parametrize("seed", range(3))
def test_oracle_step_matches_float64_within_bf16(seed):
    rng = np.random.default_rng(50 + seed)
    n, d, h = 32, 24, 40
    x, w1, b1 = bf16(rng.normal(0, 1, (n, d))), bf16(rng.normal(0, 0.2, (d, h))), bf16(rng.normal(0, 0.2, h))
    w2, b2, t = bf16(rng.normal(0, 0.2, (h, d))), bf16(rng.normal(0, 0.2, d)), bf16(rng.normal(0, 1, (n, d)))
    got = R.step_oracle(x, w1, b1, w2, b2, t)
    f = lambda b: O.bf16_to_f32(b).astype(np.float64)
    ref = R.step_float64(f(x), f(w1), f(b1), f(w2), f(b2), f(t))
    # bf16 storage of activations gives ~2^-8 relative error per rounding; the
    # backward chain compounds a few of them.
    assert abs(got["loss"] - ref["loss"]) <= 2e-2 * ref["loss"]
    for k in ("g1", "h", "y", "dy", "dz1", "dx"):
        assert rel_close(O.bf16_to_f32(got[k]), ref[k], 3e-2) <= 1.0, k
    for k in ("dw1", "dw2", "db1", "db2"):
        assert rel_close(got[k], ref[k], 3e-2) <= 1.0, k
