"""GPU parity of the autograd tape and SGD (oxmera_amd.autograd / .optim)
against oracle/autograd_ref.py, through the C-ABI.

Each op's gradient is checked by differentiating L = sum(op(...) * R) for a
random R (so the op's incoming gradient is exactly R) and comparing with
the float64 vector-Jacobian product of the same inputs.  Bars: F64
relative 1e-12 of the largest reference gradient (elementwise kernels in
f64); F32 1e-5 (elementwise, reductions) and 1e-5 * sqrt(K) for GEMM
gradients (the north star's f32 GEMM tolerance).  SGD: bit-exact against
the float32 one-rounding-per-operation restatement.
"""
import numpy as np
import pytest

import oxmera_amd as ox
from oxmera_amd import autograd as A
from oxmera_amd.nn import MLP2, Linear
from oxmera_amd.optim import SGD
from oracle import autograd_ref as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

D = ox.Device.rocm(0)


@pytest.fixture(autouse=True)
def _backend(hip):
    return hip


def log(msg):
    print(msg, flush=True)


def var(a, dtype=ox.DType.F32, rg=True):
    return A.Var(ox.Tensor.from_numpy(np.asarray(a), D, dtype), rg)


def host(v_or_t):
    t = v_or_t.t if isinstance(v_or_t, A.Var) else v_or_t
    return t.to_numpy().astype(np.float64)


def close(got, ref, rtol, what):
    scale = max(np.max(np.abs(ref)), 1e-30)
    err = np.max(np.abs(got - ref)) if ref.size else 0.0
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert err <= rtol * scale, f"{what}: max err {err:.3e} vs {rtol * scale:.3e}"


def loss_against(y: A.Var, rng, dtype):
    r = rng.normal(0, 1, y.shape)
    R = var(r.astype(np.float64 if dtype == ox.DType.F64 else np.float32), dtype, rg=False)
    (y * R).sum().backward()
    return host(R)


DTS = [(ox.DType.F32, np.float32, 1e-5), (ox.DType.F64, np.float64, 1e-12)]


@pytest.mark.parametrize("dtype,npdt,tol", DTS, ids=["f32", "f64"])
@pytest.mark.parametrize("op", [G.ADD, G.SUB, G.MUL, G.DIV], ids=["add", "sub", "mul", "div"])
@pytest.mark.parametrize("sa,sb", [((40, 50), (40, 50)), ((3, 40, 64), (64,)), ((40, 1), (1, 24)), ((2, 1, 3), (4, 1))])
def test_binary_grads(dtype, npdt, tol, op, sa, sb):
    rng = np.random.default_rng(op + 7)
    a = rng.normal(0, 1, sa).astype(npdt)
    b = (rng.normal(0, 1, sb) + 3.0 * np.sign(rng.normal(0, 1, sb))).astype(npdt)
    va, vb = var(a, dtype), var(b, dtype)
    log(f"binary grad {op} {dtype.name} {sa} {sb}")
    y = [A.add, A.sub, A.mul, A.div][op](va, vb)
    r = loss_against(y, rng, dtype)
    ga, gb = G.vjp_binary(op, a.astype(np.float64), b.astype(np.float64), r)
    close(host(va.grad), ga, tol, "da")
    close(host(vb.grad), gb, tol, "db")


@pytest.mark.parametrize("dtype,npdt,tol", DTS, ids=["f32", "f64"])
@pytest.mark.parametrize("op", [G.NEG, G.EXP, G.LN, G.ABS], ids=["neg", "exp", "ln", "abs"])
def test_unary_grads(dtype, npdt, tol, op):
    rng = np.random.default_rng(op + 17)
    a = rng.uniform(0.5, 2.0, (33, 65)) * (1 if op == G.LN else np.sign(rng.normal(0, 1, (33, 65))))
    a = a.astype(npdt)
    va = var(a, dtype)
    log(f"unary grad {op} {dtype.name}")
    y = [A.neg, A.exp, A.ln, A.abs_][op](va)
    r = loss_against(y, rng, dtype)
    close(host(va.grad), G.vjp_unary(op, a.astype(np.float64), r), 4 * tol, "da")


@pytest.mark.parametrize("dtype,npdt,tol", DTS, ids=["f32", "f64"])
@pytest.mark.parametrize("axes", [[0], [1], [0, 2], []], ids=["a0", "a1", "a02", "all"])
def test_reduce_grads(dtype, npdt, tol, axes):
    rng = np.random.default_rng(27)
    a = rng.normal(0, 1, (6, 50, 70)).astype(npdt)
    for name, fn, vjp in [("sum", A.sum_, G.vjp_sum), ("max", A.max_, G.vjp_max)]:
        va = var(a, dtype)
        log(f"{name} grad {dtype.name} {axes}")
        r = loss_against(fn(va, axes), rng, dtype)
        close(host(va.grad), vjp(a.astype(np.float64), axes, r), tol, name)


def test_max_ties_share_gradient(hip):
    va = var(np.array([[1.0, 3.0, 3.0], [2.0, 2.0, 0.0]], np.float32))
    A.max_(va, [1]).sum().backward()
    assert host(va.grad).tolist() == [[0, 0.5, 0.5], [0.5, 0.5, 0]]


@pytest.mark.parametrize("sa,sb", [((64, 96), (96, 48)), ((3, 64, 96), (96, 48)), ((4, 40, 72), (1, 72, 56)),
                                   ((3, 1, 40, 72), (2, 72, 24))])
def test_matmul_grads(hip, sa, sb):
    rng = np.random.default_rng(37)
    a, b = rng.normal(0, 1, sa).astype(np.float32), rng.normal(0, 1, sb).astype(np.float32)
    va, vb = var(a), var(b)
    log(f"matmul grad {sa} {sb}")
    y = A.matmul(va, vb)
    r = loss_against(y, rng, ox.DType.F32)
    ga, gb = G.vjp_matmul(a.astype(np.float64), b.astype(np.float64), r)
    tol = 1e-5 * np.sqrt(max(sa[-1], sa[-2], sb[-1]) * 4)
    close(host(va.grad), ga, tol, "da")
    close(host(vb.grad), gb, tol, "db")


def test_matmul_grads_of_views(hip):
    # A a transposed view, B an every-other-row slice: gradients land in the operands' shapes
    rng = np.random.default_rng(38)
    abuf = rng.normal(0, 1, (96, 64)).astype(np.float32)
    bbuf = rng.normal(0, 1, (192, 48)).astype(np.float32)
    ta = ox.Tensor.from_numpy(abuf, D).transpose_last()
    tb = ox.Tensor.from_numpy(bbuf, D).with_layout((96, 48), (96, 1), 0)
    va, vb = A.Var(ta, True), A.Var(tb, True)
    r = loss_against(A.matmul(va, vb), rng, ox.DType.F32)
    ga, gb = G.vjp_matmul(abuf.T.astype(np.float64), bbuf[::2].astype(np.float64), r)
    close(host(va.grad), ga, 1e-4, "da")
    close(host(vb.grad), gb, 1e-4, "db")


def test_accumulation_and_composite(hip):
    rng = np.random.default_rng(47)
    a = rng.uniform(0.5, 1.5, (30, 40)).astype(np.float32)
    w = rng.normal(0, 0.3, (40, 20)).astype(np.float32)
    c = rng.normal(0, 1, (20,)).astype(np.float32)
    va, vw, vc = var(a), var(w), var(c)
    # L = sum( ln(|a w| + 1) * c ) + sum(a * a) + sum(a): a used three times
    h = A.matmul(va, vw)
    one = var(np.ones((1,), np.float32), rg=False)
    L = (A.ln(A.abs_(h) + one) * vc).sum() + (va * va).sum() + va.sum()
    L.backward()
    a64, w64, c64 = a.astype(np.float64), w.astype(np.float64), c.astype(np.float64)
    h64 = a64 @ w64
    gu = np.broadcast_to(c64, h64.shape) / (np.abs(h64) + 1) * np.sign(h64)
    ga_mm, gw = G.vjp_matmul(a64, w64, gu)
    close(host(va.grad), ga_mm + 2 * a64 + 1, 1e-5, "da")
    close(host(vw.grad), gw, 1e-4, "dw")
    close(host(vc.grad), np.log(np.abs(h64) + 1).sum(axis=0), 1e-5, "dc")
    # a second backward accumulates into the leaves
    g1 = host(vc.grad)
    L2 = (A.ln(A.abs_(A.matmul(va, vw)) + one) * vc).sum()
    L2.backward()
    close(host(vc.grad), 2 * g1, 1e-5, "dc accumulated")


def test_linear_gelu_with_generic_consumer(hip):
    # the GELU layer's output feeds a mul, not a Linear: dz = g * GELU'(z) by the
    # elementwise kernel, db by a column-sum pass
    rng = np.random.default_rng(57)
    x = rng.normal(0, 1, (64, 96)).astype(np.float32)
    w = rng.normal(0, 0.1, (96, 32)).astype(np.float32)
    b = rng.normal(0, 0.1, (32,)).astype(np.float32)
    vx, vw, vb = var(x), var(w), var(b)
    h = A.linear(vx, vw, vb, ox.ACT_GELU)
    r = loss_against(h, rng, ox.DType.F32)
    dx, dw, db = G.vjp_linear_gelu(x.astype(np.float64), w.astype(np.float64), b.astype(np.float64), r)
    close(host(vx.grad), dx, 1e-4, "dx")
    close(host(vw.grad), dw, 1e-4, "dw")
    close(host(vb.grad), db, 1e-4, "db")


def test_mse_of_a_shared_output(hip):
    # y = linear(x) feeds both the MSE and a sum: the MSE pass's bias sums are
    # not the whole gradient, so the tape must not use them
    rng = np.random.default_rng(67)
    x = rng.normal(0, 1, (32, 64)).astype(np.float32)
    w = rng.normal(0, 0.1, (64, 16)).astype(np.float32)
    b = rng.normal(0, 0.1, (16,)).astype(np.float32)
    t = rng.normal(0, 1, (32, 16)).astype(np.float32)
    vx, vw, vb = var(x, rg=False), var(w), var(b)
    y = A.linear(vx, vw, vb)
    L = A.mse_loss(y, ox.Tensor.from_numpy(t, D)) + y.sum()
    L.backward()
    y64 = x.astype(np.float64) @ w + b
    dy = 2 * (y64 - t) / y64.size + 1.0
    close(host(vb.grad), dy.sum(axis=0), 1e-5, "db")
    close(host(vw.grad), x.T.astype(np.float64) @ dy, 1e-4, "dw")


# ---- SGD ---------------------------------------------------------------------------

@pytest.mark.parametrize("pdt,gdt", [(ox.DType.F32, ox.DType.F32), (ox.DType.BF16, ox.DType.F32),
                                     (ox.DType.BF16, ox.DType.BF16), (ox.DType.F16, ox.DType.F32),
                                     (ox.DType.F16, ox.DType.F16)], ids=["f32", "bf16-f32", "bf16", "f16-f32", "f16"])
@pytest.mark.parametrize("cfg", [dict(), dict(weight_decay=0.01), dict(momentum=0.9),
                                 dict(momentum=0.9, nesterov=True, weight_decay=0.05)],
                         ids=["plain", "wd", "momentum", "nesterov-wd"])
@pytest.mark.parametrize("n", [10007, 10008], ids=["n-odd", "n-vec"])  # 10008: the 8-per-thread vector kernel
def test_sgd_bit_exact(hip, pdt, gdt, cfg, n):
    rng = np.random.default_rng(77)
    odt = {ox.DType.F32: O.F32, ox.DType.BF16: O.BF16, ox.DType.F16: O.F16}
    p0 = rng.normal(0, 1, n).astype(np.float32)
    p_raw = O.bf16_round(p0) if pdt == ox.DType.BF16 else p0.astype(np.float16 if pdt == ox.DType.F16 else np.float32)
    P = A.Var(ox.Tensor.from_numpy(p_raw, D, pdt), True)
    opt = SGD([P], lr=0.01, **cfg)
    v = np.zeros(n, np.float32) if cfg.get("momentum") else None
    for step in range(3):
        g = rng.normal(0, 1, n).astype(np.float32)
        g_raw = O.bf16_round(g) if gdt == ox.DType.BF16 else g.astype(np.float16 if gdt == ox.DType.F16 else np.float32)
        P.grad = ox.Tensor.from_numpy(g_raw, D, gdt)
        opt.step()
        g_val = O.bf16_to_f32(g_raw) if gdt == ox.DType.BF16 else g_raw.astype(np.float32)
        p_raw, v = G.sgd_step(p_raw, odt[pdt], g_val, v, 0.01, cfg.get("momentum", 0.0),
                              cfg.get("weight_decay", 0.0), cfg.get("nesterov", False))
        got = P.t.to_numpy()
        want = O.bf16_to_f32(p_raw) if pdt == ox.DType.BF16 else p_raw.astype(np.float32)
        assert np.array_equal(got.astype(np.float32), want), f"step {step}"


def test_sgd_refusals(hip):
    P = A.Var(ox.Tensor.from_numpy(np.zeros(8, np.float32), D), True)
    P.grad = ox.Tensor.from_numpy(np.zeros(8, np.float64), D)
    with pytest.raises(ox.DTypeMismatch):
        SGD([P], lr=0.1).step()
    P.grad = ox.Tensor.from_numpy(np.zeros(9, np.float32), D)
    with pytest.raises(ox.ShapeMismatch):
        SGD([P], lr=0.1).step()
    with pytest.raises(ox.InvalidArgument):
        SGD([P], lr=0.1, nesterov=True)


def test_mlp_sgd_training_reduces_loss(hip):
    rng = np.random.default_rng(87)
    n, d, h = 256, 128, 512
    bf = lambda a: ox.Tensor.from_numpy(a.astype(np.float32), D, ox.DType.BF16)
    fc1 = Linear(bf(rng.normal(0, 0.05, (d, h))), bf(rng.normal(0, 0.02, h)), act=ox.ACT_GELU)
    fc2 = Linear(bf(rng.normal(0, 0.05, (h, d))), bf(rng.normal(0, 0.02, d)))
    model = MLP2(fc1, fc2)
    x = A.Var(bf(rng.normal(0, 1, (n, d))), False)
    t = bf(0.5 * rng.normal(0, 1, (n, d)))
    opt = SGD(model.parameters(), lr=0.5, momentum=0.9)
    losses = []
    for _ in range(30):
        loss = model.train_step(x, t)
        opt.step()
        losses.append(float(loss.t.to_numpy()[0]))
    log(f"losses {losses[0]:.4f} -> {losses[-1]:.4f}")
    assert all(np.isfinite(losses)) and losses[-1] < 0.8 * losses[0]
