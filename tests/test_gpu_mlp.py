"""GPU parity of the MLP training step through the
autograd tape, against the oracle.

  * reduced size (X [256, 512], 512 -> 2048 -> 512): every intermediate and
    gradient of the GPU step against oracle/mlp_ref.step_oracle on the same
    bf16 inputs, and every GEMM against the oracle fed the GPU's own inputs;
  * full size (X [8192, 4096], 4096 -> 16384 -> 4096): each of the six GEMMs
    (X.W1, H.W2, H^T.dY, dY.W2^T, X^T.dZ1, dZ1.W1^T) on sampled rows of its
    own GPU-side inputs, the bias gradients in full, loss and dY in full.
Tolerance (north star, bf16 in / f32 accumulate): |c-r| <= 1e-2 max(|r|, rms(r)).
"""
import numpy as np
import pytest

import oxmera_amd as ox
from oracle import mlp_ref as R
from oracle import oracle as O
from oxmera_amd.autograd import Var
from oxmera_amd.nn import MLP2, Linear
from tests.parity import assert_close, k_major, sample_rows

pytestmark = pytest.mark.gpu
TOL = 1e-2
BF16 = ox.DType.BF16


def log(msg):
    print(msg, flush=True)


def bits(t: ox.Tensor) -> np.ndarray:
    """Raw bf16 bits of a contiguous device tensor."""
    return ox.f32_to_bf16_bits(t.to_numpy())  # exact: the values are bf16


def build(n, d, h, seed):
    rng = np.random.default_rng(seed)
    dev = ox.Device.rocm(0)
    host = dict(x=O.bf16_round(rng.normal(0, 1, (n, d)).astype(np.float32)),
                w1=O.bf16_round(rng.normal(0, 0.02, (d, h)).astype(np.float32)),
                b1=O.bf16_round(rng.normal(0, 0.02, h).astype(np.float32)),
                w2=O.bf16_round(rng.normal(0, 0.02, (h, d)).astype(np.float32)),
                b2=O.bf16_round(rng.normal(0, 0.02, d).astype(np.float32)),
                t=O.bf16_round(rng.normal(0, 1, (n, d)).astype(np.float32)))
    T = {k: ox.Tensor.from_numpy(v, dev, BF16) for k, v in host.items()}
    fc1 = Linear(T["w1"], T["b1"], act=ox.ACT_GELU)
    fc2 = Linear(T["w2"], T["b2"])
    model = MLP2(fc1, fc2)
    x = Var(T["x"], requires_grad=True)
    return host, T, model, x


def intermediates(model, x, t):
    """Forward + backward, returning every tensor the step produced."""
    from oxmera_amd.autograd import linear, mse_loss
    fc1, fc2 = model.fc1, model.fc2
    fc1.zero_grad()
    fc2.zero_grad()
    x.grad = None
    hv = fc1(x)
    yv = fc2(hv)
    lv = mse_loss(yv, t)
    lv.backward()
    return dict(g1=hv.node.gd, h=hv.t, y=yv.t, loss=lv.t, dy=yv.grad, dw2=fc2.w.grad, db2=fc2.b.grad,
                dz1=hv.grad, dw1=fc1.w.grad, db1=fc1.b.grad, dx=x.grad)


def test_mlp_small_end_to_end(hip):
    n, d, h = 256, 512, 2048
    host, T, model, x = build(n, d, h, 7)
    got = intermediates(model, x, T["t"])
    ref = R.step_oracle(host["x"], host["w1"], host["b1"], host["w2"], host["b2"], host["t"])
    assert abs(float(got["loss"].to_numpy()[0]) - float(ref["loss"])) <= 1e-3 * float(ref["loss"])
    for k in ("g1", "h", "y", "dy", "dz1", "dx"):
        assert_close(got[k].to_numpy(), O.bf16_to_f32(ref[k]), TOL, k)
    for k in ("dw1", "dw2", "db1", "db2"):
        assert_close(got[k].to_numpy(), ref[k], TOL, k)


def gemm_checks(got, host, rows_per=6, seed=0):
    """Each GEMM of the step on sampled rows, fed the GPU's own inputs."""
    xb, w1b, w2b = host["x"], host["w1"], host["w2"]
    hb, g1b, dyb, dz1b = bits(got["h"]), bits(got["g1"]), bits(got["dy"]), bits(got["dz1"])
    V = lambda b: O.StridedView.contiguous(b, O.BF16)
    VT = lambda b: O.StridedView.contiguous(b, O.BF16).permute([1, 0])
    # the oracle reads K-contiguous copies of the same operands (bit-identical
    # results, far fewer cache misses at full size)
    F = lambda a, b, **kw: O.matmul(*k_major(a, b), **kw)
    n = xb.shape[0]
    checks = []
    r = sample_rows(n, rows_per, seed)
    h_ref, g_ref = F(V(xb), V(w1b), out_dtype=O.BF16, bias=host["b1"], bias_dtype=O.BF16,
                     act=O.ACT_GELU_GRAD, rows=r, want_aux=True)
    checks += [("GELU'(X.W1+b1)", g1b[r], g_ref, True), ("GELU(X.W1+b1)", hb[r], h_ref, True)]
    y_ref = F(V(hb), V(w2b), out_dtype=O.BF16, bias=host["b2"], bias_dtype=O.BF16, rows=r)
    checks.append(("H.W2+b2", bits(got["y"])[r], y_ref, True))
    rh = sample_rows(hb.shape[1], rows_per, seed + 1)
    checks.append(("H^T.dY", got["dw2"].to_numpy()[rh], F(VT(hb), V(dyb), rows=rh), False))
    dz_ref = F(V(dyb), VT(w2b), out_dtype=O.BF16, act=O.ACT_MUL_AUX, aux=g1b, rows=r)
    checks.append(("dY.W2^T * GELU'", dz1b[r], dz_ref, True))
    rx = sample_rows(xb.shape[1], rows_per, seed + 2)
    checks.append(("X^T.dZ1", got["dw1"].to_numpy()[rx], F(VT(xb), V(dz1b), rows=rx), False))
    checks.append(("dZ1.W1^T", bits(got["dx"])[r], F(V(dz1b), VT(w1b), out_dtype=O.BF16, rows=r), True))
    for name, g, ref, is_bits in checks:
        log(f"  check {name}")
        if is_bits:
            assert_close(O.bf16_to_f32(g), O.bf16_to_f32(ref), TOL, name)
        else:
            assert_close(g, ref, TOL, name)
    # bias gradients (full) and the loss / dY (full)
    assert_close(got["db2"].to_numpy(), O.colsum(dyb, O.BF16), TOL, "db2")
    assert_close(got["db1"].to_numpy(), O.colsum(dz1b, O.BF16), TOL, "db1")
    yf, tf = got["y"].to_numpy().astype(np.float64), O.bf16_to_f32(host["t"]).astype(np.float64)
    loss_ref = np.mean((yf - tf) ** 2)
    assert abs(float(got["loss"].to_numpy()[0]) - loss_ref) <= 1e-4 * loss_ref
    assert_close(got["dy"].to_numpy(), 2 * (yf - tf) / yf.size, TOL, "dY")


@pytest.mark.parametrize("shape,dtype", [((300, 520), ox.DType.BF16), ((33, 37), ox.DType.F32),
                                         ((2, 5, 64), ox.DType.F16), ((64, 256), ox.DType.F32)],
                         ids=["bf16_vec", "f32_scalar", "f16_rank3", "f32_vec"])
def test_mse_with_column_sums(hip, shape, dtype):
    """loss, dy and the column sums of dy (the producing layer's bias
    gradient) from one pass, against float64 on the host."""
    from tests.parity import host_buffer
    rng = np.random.default_rng(51)
    n = int(np.prod(shape))
    ybuf = host_buffer(dtype, rng.normal(0, 1, n).astype(np.float32)).reshape(shape)
    tbuf = host_buffer(dtype, rng.normal(0, 1, n).astype(np.float32)).reshape(shape)
    dev = ox.Device.rocm(0)
    y, t = ox.Tensor.from_numpy(ybuf, dev, dtype), ox.Tensor.from_numpy(tbuf, dev, dtype)
    cs = ox.Tensor.empty((shape[-1],), ox.DType.F32, dev)
    loss, dy = hip.mse_loss_grad(y, t, dy_colsum=cs)
    yf, tf = y.to_numpy().astype(np.float64), t.to_numpy().astype(np.float64)
    loss_ref = np.mean((yf - tf) ** 2)
    assert abs(float(loss.to_numpy()[0]) - loss_ref) <= 1e-5 * loss_ref
    dyg = dy.to_numpy().astype(np.float64)
    assert_close(dyg, 2 * (yf - tf) / n, TOL if dtype != ox.DType.F32 else 1e-6, "dy")
    x = dyg.reshape(-1, shape[-1])
    bound = x.shape[0] * 2.0 ** -24 * np.abs(x).sum(0) + 1e-30
    assert np.all(np.abs(cs.to_numpy() - x.sum(0)) <= bound), "column sums of dy"


def test_mlp_small_per_gemm(hip):
    host, T, model, x = build(256, 512, 2048, 8)
    got = intermediates(model, x, T["t"])
    gemm_checks(got, host, rows_per=32)


def test_mlp_full_size_c5(hip):
    log("C5 MLP X [8192,4096], 4096->16384->4096, bf16")
    host, T, model, x = build(8192, 4096, 16384, 9)
    got = intermediates(model, x, T["t"])
    assert got["dw1"].shape == (4096, 16384) and got["dx"].shape == (8192, 4096)
    gemm_checks(got, host, rows_per=64)
