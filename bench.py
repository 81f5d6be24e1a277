"""Benchmark of the MI355X GEMM backend (one JSON line on stdout).

Metric: GEMM TFLOP/s and % of MI355X dense MFMA peak.
A "step" is one GEMM launch over inputs already resident in HBM.

  default workload  configs[1]: f32 C = A.B, 4096 x 4096 x 4096, row-major,
                    A, B ~ N(0,1) from a seed                    -> "value"
  second line item  configs[2]: bf16 in / f32 out, 8192^3, A row-major,
                    B a transposed strided view (strides [1, 8192]),
                    N(0, 0.02)                                  -> "extra"

Timing: W untimed warm-up launches (and at least 0.3 s of them), then K
launches bracketed by HIP events
on the stream the kernel runs on (a dedicated non-default stream handed to
oxm_gemm, so launches are asynchronous), with device synchronisation on
both sides.  The roofline figure
is algorithmic flops per launch / average launch time against the dense
MFMA peak of the dtype.  cpu_baseline times the naive CPU oracle on a
bounded sample of output rows on this host and extrapolates.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload f32|bf16|mlp]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK = {"f32": 157.3, "bf16": 2516.6}  # TFLOP/s, dense MFMA, MI355X (256 CU x 2.4 GHz)
WARMUP_S = 0.3  # minimum warm-up time per workload (s)


def _rng(seed: int):
    return np.random.default_rng(seed)


def make_inputs(kind: str):
    """Device operands, an output tensor, the host buffers the CPU oracle
    reads (buffer, oracle dtype, shape, strides per operand) and a config
    description, for one BASELINE configuration:
      f32    configs[1] C2: 4096^3, row-major, N(0,1)
      bf16   configs[2] C3: 8192^3, B a transposed view, N(0,0.02)
      c1     configs[0] C1: 256^3 f32, U[-1,1)
      c2odd  configs[1] C2-odd: 4097x4093 . 4093x4095 f32 (row strides not 16-byte multiples), N(0,1)
      c4     configs[3] C4: A [32,512,1024] = every other row of a [32,1024,1024]
             buffer, B [1,1024,768] broadcast over the batch, U[-1,1)"""
    import oxmera_amd as ox
    from oracle import oracle as O
    dev = ox.Device.rocm(0)
    if kind in ("f32", "c1", "c2odd"):
        m, k, n, seed = {"f32": (4096, 4096, 4096, 12345), "c1": (256, 256, 256, 111),
                         "c2odd": (4097, 4093, 4095, 2222)}[kind]
        rng = _rng(seed)
        if kind == "c1":
            a_h = rng.uniform(-1, 1, (m, k)).astype(np.float32)
            b_h = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        else:
            a_h = rng.standard_normal((m, k), dtype=np.float32)
            b_h = rng.standard_normal((k, n), dtype=np.float32)
        a = ox.Tensor.from_numpy(a_h, dev, ox.DType.F32)
        b = ox.Tensor.from_numpy(b_h, dev, ox.DType.F32)
        host = ((a_h, O.F32, (m, k), (k, 1)), (b_h, O.F32, (k, n), (n, 1)))
        name = {"f32": "f32 matmul 4096x4096x4096, A and B contiguous row-major (BASELINE configs[1])",
                "c1": "f32 matmul 256x256x256, contiguous, U[-1,1) (BASELINE configs[0])",
                "c2odd": "f32 matmul 4097x4093 . 4093x4095, contiguous, N(0,1) (BASELINE configs[1], odd shape)"}[kind]
        desc = {"workload": name, "M": m, "N": n, "K": k, "batch": 1, "a_strides": [k, 1], "b_strides": [n, 1],
                "seed": seed}
        oshape = (m, n)
    elif kind == "bf16":
        m = k = n = 8192
        rng = _rng(54321)
        a_h = ox.f32_to_bf16_bits(rng.normal(0, 0.02, (m, k)).astype(np.float32))
        bbuf = ox.f32_to_bf16_bits(rng.normal(0, 0.02, (n, k)).astype(np.float32))
        a = ox.Tensor.from_numpy(a_h, dev, ox.DType.BF16)
        b = ox.Tensor.from_numpy(bbuf, dev, ox.DType.BF16).permute([1, 0])  # [K, N], strides [1, K]
        host = ((a_h, O.BF16, (m, k), (k, 1)), (bbuf, O.BF16, (k, n), (1, k)))
        desc = {"workload": "bf16-in f32-out matmul 8192^3, A row-major, B transposed view strides [1,8192] "
                            "(BASELINE configs[2])",
                "M": m, "N": n, "K": k, "batch": 1, "a_strides": [k, 1], "b_strides": [1, k], "seed": 54321}
        oshape = (m, n)
    elif kind == "f16":
        m = k = n = 8192
        rng = _rng(54322)
        a_h = rng.normal(0, 0.02, (m, k)).astype(np.float16)
        bbuf = rng.normal(0, 0.02, (n, k)).astype(np.float16)
        a = ox.Tensor.from_numpy(a_h, dev, ox.DType.F16)
        b = ox.Tensor.from_numpy(bbuf, dev, ox.DType.F16).permute([1, 0])  # [K, N], strides [1, K]
        host = ((a_h, O.F16, (m, k), (k, 1)), (bbuf, O.F16, (k, n), (1, k)))
        desc = {"workload": "f16-in f32-out matmul 8192^3, A row-major, B transposed view strides [1,8192] "
                            "(configs[2]'s shape and layout in f16)",
                "M": m, "N": n, "K": k, "batch": 1, "a_strides": [k, 1], "b_strides": [1, k], "seed": 54322}
        oshape = (m, n)
    elif kind == "c4":
        bt, m, k, n = 32, 512, 1024, 768
        rng = _rng(4444)
        abuf = rng.uniform(-1, 1, (bt, 2 * m, k)).astype(np.float32)
        b_h = rng.uniform(-1, 1, (1, k, n)).astype(np.float32)
        full = ox.Tensor.from_numpy(abuf, dev, ox.DType.F32)
        a = full.with_layout((bt, m, k), (2 * m * k, 2 * k, 1), 0)  # every other row, no copy
        b = ox.Tensor.from_numpy(b_h, dev, ox.DType.F32)
        host = ((abuf, O.F32, (bt, m, k), (2 * m * k, 2 * k, 1)), (b_h, O.F32, (1, k, n), (k * n, n, 1)))
        desc = {"workload": "batched f32 matmul: A [32,512,1024] every other row of a [32,1024,1024] buffer "
                            "(strides [1048576,2048,1]), B [1,1024,768] broadcast, U[-1,1) (BASELINE configs[3])",
                "M": m, "N": n, "K": k, "batch": bt, "a_strides": [2 * m * k, 2 * k, 1],
                "b_strides": [k * n, n, 1], "seed": 4444}
        oshape = (bt, m, n)
    else:
        raise ValueError(kind)
    out = ox.Tensor.empty(oshape, ox.DType.F32, dev)
    ws = sum(h[0].nbytes for h in host) + out.storage.nbytes
    desc["working_set_bytes"] = int(ws)
    desc["exceeds_256MB_infinity_cache"] = bool(ws > 256 * 2 ** 20)
    return a, b, out, host, desc


def time_gpu(kind: str, steps: int, warmup: int):
    import torch
    import oxmera_amd as ox
    ox.init()
    be = ox.backend_for(ox.Device.rocm(0))
    a, b, out, host, desc = make_inputs(kind)
    # A dedicated (non-null) stream: launches are asynchronous and the HIP
    # events below are recorded on the stream the kernels run on.  (The null
    # stream means "synchronous" at the C-ABI.)
    ts = torch.cuda.Stream()
    stream = ts.cuda_stream
    with torch.cuda.stream(ts):
        # W launches, and at least WARMUP_S seconds of them: after an idle
        # stretch (the CPU baseline) the clock takes a while to ramp up.
        t0, n = time.perf_counter(), 0
        while n < warmup or time.perf_counter() - t0 < WARMUP_S:
            be.matmul(a, b, out=out, stream=stream)
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(ts)
        for _ in range(steps):
            be.matmul(a, b, out=out, stream=stream)
        stop.record(ts)
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(stop)
        # per-launch durations for a median (separate pass, same stream)
        per = []
        for _ in range(min(steps, 20)):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(ts)
            be.matmul(a, b, out=out, stream=stream)
            e.record(ts)
            per.append((s, e))
        torch.cuda.synchronize()
    per_ms = sorted(s.elapsed_time(e) for s, e in per)
    flops = 2.0 * desc["batch"] * desc["M"] * desc["N"] * desc["K"]
    return dict(total_ms=total_ms, per_ms=per_ms, flops=flops, desc=desc, host=host, out=out, a=a, b=b)


def time_mlp(steps: int, warmup: int):
    """one MLP training step (forward, MSE, backward) through the
    autograd tape: X [8192, 4096] bf16, Linear 4096->16384 + bias + GELU,
    Linear 16384->4096 + bias.  Six GEMMs of 2*8192*4096*16384 flops each."""
    import torch
    import oxmera_amd as ox
    from oxmera_amd.autograd import Var
    from oxmera_amd.nn import MLP2, Linear
    ox.init()
    dev = ox.Device.rocm(0)
    rng = np.random.default_rng(777)
    n, d, h = 8192, 4096, 16384
    bf = lambda a: ox.Tensor.from_numpy(a.astype(np.float32), dev, ox.DType.BF16)
    fc1 = Linear(bf(rng.normal(0, 0.02, (d, h))), bf(rng.normal(0, 0.02, h)), act=ox.ACT_GELU)
    fc2 = Linear(bf(rng.normal(0, 0.02, (h, d))), bf(rng.normal(0, 0.02, d)))
    model = MLP2(fc1, fc2)
    x = Var(bf(rng.normal(0, 1, (n, d))), requires_grad=True)
    t = bf(rng.normal(0, 1, (n, d)))
    # Asynchronous on one stream: the host issues the whole step, device
    # storage is recycled in stream order by the caching allocator.
    stream = torch.cuda.Stream()
    be = ox.backend_for(dev)
    be.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            w0, nw = time.perf_counter(), 0
            while nw < warmup or time.perf_counter() - w0 < WARMUP_S:
                model.train_step(x, t)
                nw += 1
                torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(steps):
                loss = model.train_step(x, t)
            stop.record(stream)
            torch.cuda.synchronize()
            dt = start.elapsed_time(stop) / steps / 1e3
    finally:
        be.set_stream(None)
    flops = 6 * 2.0 * n * d * h
    return {"config": {"workload": "MLP fwd+bwd, X [8192,4096] bf16, 4096->16384 (+bias, GELU) ->4096 (+bias), "
                                   "MSE (BASELINE configs[4]); whole step issued asynchronously on one stream",
                       "gemm_flops_per_step": flops},
            "ms_per_step": round(dt * 1e3, 3), "value": round(flops / dt / 1e12, 1), "unit": "TFLOP/s (6 GEMMs)",
            "pct_of_peak": round(100 * flops / dt / 1e12 / PEAK["bf16"], 2),
            "loss": float(loss.t.to_numpy()[0])}


def mlp_cpu_baseline(rows: int = 32) -> dict:
    """configs[4]'s six GEMMs timed with the naive oracle on the host, each on
    `rows` seeded output rows with the operand layouts the GPU step uses
    (transposed operands read through their strides), per-row rates summed
    into an extrapolated time per training step.  The oracle's work does not
    depend on the values, so the operands are synthetic bf16 (a tiled random
    N(0, 0.02) block) of the step's shapes."""
    from oracle import oracle as O
    threads = min(os.cpu_count() or 1, CPU_THREADS)
    n, d, h = 8192, 4096, 16384
    block = O.bf16_round(np.random.default_rng(99).normal(0, 0.02, 1 << 22).astype(np.float32))
    mats = {}

    def mat(name, r, c):
        if name not in mats:
            mats[name] = np.resize(block, r * c)
        return mats[name]

    def view(name, r, c, transposed=False):
        # logical [r, c]; transposed: a view of a row-major [c, r] buffer
        buf = mat(name, c, r) if transposed else mat(name, r, c)
        return O.StridedView(buf, O.BF16, (r, c), (1, r) if transposed else (c, 1))

    gemms = [  # (name, A view, B view, output rows, K, N)
        ("Z1 = X.W1 (+b1, GELU)", view("X", n, d), view("W1", d, h), n, d, h),
        ("Y = H.W2 (+b2)", view("H", n, h), view("W2", h, d), n, h, d),
        ("dW2 = H^T.dY", view("H", h, n, True), view("dY", n, d), h, n, d),
        ("dZ1 = dY.W2^T * GELU'", view("dY", n, d), view("W2", d, h, True), n, d, h),
        ("dW1 = X^T.dZ1", view("X", d, n, True), view("dZ1", n, h), d, n, h),
        ("dX = dZ1.W1^T", view("dZ1", n, h), view("W1", h, d, True), n, h, d),
    ]
    per, total = [], 0.0
    for name, av, bv, m, k, nn in gemms:
        sel = np.sort(np.random.default_rng(5).choice(m, size=rows, replace=False)).astype(np.int64)
        t0 = time.perf_counter()
        O.matmul(av, bv, rows=sel, nthreads=threads)
        dt = time.perf_counter() - t0
        full = dt * m / rows
        total += full
        per.append({"gemm": name, "rows": rows, "of_rows": m, "s": round(dt, 3), "extrapolated_full_s": round(full, 1)})
    flops = 6 * 2.0 * n * d * h
    return {"value": round(flops / total / 1e12, 6), "unit": "TFLOP/s (6 GEMMs)", "cores": threads, "kind": "port",
            "extrapolated_step_s": round(total, 1), "extrapolated": True, "per_gemm": per,
            "sample": f"{rows} seeded output rows of each of the step's six GEMMs (synthetic bf16 operands in the "
                      f"GPU step's layouts) by the naive oracle (oracle/oxm_oracle.c, f32 ascending-k, strided "
                      f"reads, threaded over rows); the step time is extrapolated from the per-row rates",
            "host_cpu": host_cpu(), "host_threads": os.cpu_count()}


def time_vendor(kind: str, steps: int, warmup: int) -> dict:
    """torch.matmul (hipBLASLt) on the same shapes, input dtypes and layout
    (bf16: B a transposed view of an [N, K] buffer).  torch returns bf16 for
    bf16 inputs, so its C is half the bytes of this backend's f32 C."""
    import torch
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(1)
    if kind == "bf16":
        n = 8192
        a = (torch.randn(n, n, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        b = (torch.randn(n, n, device=dev, generator=g) * 0.02).to(torch.bfloat16).t()
        flops = 2.0 * n ** 3
    elif kind == "f32":
        n = 4096
        a = torch.randn(n, n, device=dev, generator=g)
        b = torch.randn(n, n, device=dev, generator=g)
        flops = 2.0 * n ** 3
    else:
        raise SystemExit("--vendor times the f32 and bf16 workloads")
    for _ in range(warmup):
        c = torch.matmul(a, b)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARMUP_S:
        c = torch.matmul(a, b)
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        c = torch.matmul(a, b)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    del c
    return {"vendor": "torch.matmul (hipBLASLt), black box", "workload": kind, "out_dtype": str(a.dtype),
            "ms_per_launch": round(ms, 4), "TFLOP/s": round(flops / ms / 1e9, 1)}


def time_ops(steps: int = 20) -> dict:
    """The HBM-bound ops of the rest of the Backend at [8192, 8192]: bytes
    moved (one read of each input element, one write of each output
    element) per launch / launch time, against the 8 TB/s HBM peak."""
    import torch
    import oxmera_amd as ox
    ox.init()
    dev = ox.Device.rocm(0)
    be = ox.backend_for(dev)
    n = 8192
    rng = np.random.default_rng(99)
    a = ox.Tensor.from_numpy(rng.standard_normal((n, n), dtype=np.float32), dev)
    b = ox.Tensor.from_numpy(rng.standard_normal((n, n), dtype=np.float32), dev)
    hb = ox.Tensor.from_numpy(ox.f32_to_bf16_bits(rng.standard_normal((n, n), dtype=np.float32)), dev, ox.DType.BF16)
    ts = torch.cuda.Stream()
    s = ts.cuda_stream
    cases = {
        "add f32 [8192,8192] + [8192,8192]": (lambda: be.add(a, b, stream=s), 3 * n * n * 4),
        "add f32 [8192,8192] + [8192] (broadcast row)": (None, 2 * n * n * 4 + n * 4),
        "exp bf16 [8192,8192]": (lambda: be.exp(hb, stream=s), 2 * n * n * 2),
        "contiguous of a transposed bf16 [8192,8192] view": (lambda: be.contiguous(hb.permute([1, 0]), stream=s),
                                                             2 * n * n * 2),
        "sum f32 [8192,8192] over axis 0": (lambda: be.sum(a, [0], stream=s), n * n * 4 + n * 4),
        "sum f32 [8192,8192] over axis 1": (lambda: be.sum(a, [1], stream=s), n * n * 4 + n * 4),
        "max f32 [8192,8192] over all axes": (lambda: be.max(a, [], stream=s), n * n * 4),
    }
    row = ox.Tensor.from_numpy(rng.standard_normal(n, dtype=np.float32), dev)
    cases["add f32 [8192,8192] + [8192] (broadcast row)"] = (lambda: be.add(a, row, stream=s), 2 * n * n * 4 + n * 4)
    col = ox.Tensor.from_numpy(ox.f32_to_bf16_bits(rng.standard_normal((n, 1), dtype=np.float32)), dev, ox.DType.BF16)
    cases["mul bf16 [8192,8192] * [8192,1] (broadcast column)"] = (lambda: be.mul(hb, col, stream=s),
                                                                  2 * n * n * 2 + n * 2)
    cases["sum bf16 [8192,8192] over axis 1"] = (lambda: be.sum(hb, [1], stream=s), n * n * 2 + n * 2)
    # SGD with momentum on a bf16 [4096, 16384] weight with its f32 gradient:
    # reads p, g, v and writes p, v
    pw = ox.Tensor.from_numpy(ox.f32_to_bf16_bits(rng.standard_normal((4096, 16384), dtype=np.float32)), dev,
                              ox.DType.BF16)
    gw = ox.Tensor.from_numpy(rng.standard_normal((4096, 16384), dtype=np.float32) * 1e-3, dev)
    vw = ox.Tensor.from_numpy(np.zeros((4096, 16384), np.float32), dev)
    cases["sgd momentum, bf16 param [4096,16384], f32 grad"] = (
        lambda: be.sgd_step(pw, gw, vw, 1e-3, 0.9, 0.0, False, stream=s), 4096 * 16384 * (2 + 4 + 4 + 2 + 4))
    # a practical ceiling for the read + write kernels above: a plain device
    # copy of the same 256 MiB by the vendor runtime (torch, black box)
    tsrc = torch.empty(n * n, dtype=torch.float32, device="cuda:0").normal_()
    tdst = torch.empty_like(tsrc)
    cases["reference: torch device copy of 256 MiB (vendor runtime, not this backend)"] = (
        lambda: tdst.copy_(tsrc), 2 * n * n * 4)
    out = {}
    with torch.cuda.stream(ts):
        for name, (fn, nbytes) in cases.items():
            w0 = time.perf_counter()
            while time.perf_counter() - w0 < 0.1:
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(ts)
            for _ in range(steps):
                fn()
            e1.record(ts)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            out[name] = {"ms": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1),
                         "frac_of_8TB/s": round(nbytes / ms / 1e6 / 8000.0, 3)}
    return out


def host_cpu() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _views(host):
    from oracle import oracle as O
    (ab, adt, ash, ast), (bb, bdt, bsh, bst) = host
    return (O.StridedView(ab.reshape(-1), adt, ash, ast, 0), O.StridedView(bb.reshape(-1), bdt, bsh, bst, 0))


CPU_THREADS = 16  # the GPU box's CPU share for one GPU, whatever cpu_count() reports there


def cpu_baseline(kind: str, host, desc, budget_s: float = 30.0, rows: int | None = None):
    """The naive oracle (oracle/oxm_oracle.c: three loops, f32 ascending-k,
    reading through the operands' own strides; one output row per task) on
    CPU_THREADS host threads.  rows=None: the whole output when it fits the
    budget, else a bounded random sample grown until it takes ~budget/8;
    rows=n: exactly n seeded rows.  A sample reports its per-row rate and the
    full time extrapolated from it, labelled so.  Returns (line, (rows, result))
    so that the same run also serves as the parity reference."""
    from oracle import oracle as O
    threads = min(os.cpu_count() or 1, CPU_THREADS)
    av, bv = _views(host)
    rows_total = desc["batch"] * desc["M"]
    N, K = desc["N"], desc["K"]
    rng = np.random.default_rng(7)
    if rows is not None:
        n = min(rows, rows_total)
        sel = np.arange(rows_total, dtype=np.int64) if n == rows_total else \
            np.sort(rng.choice(rows_total, size=n, replace=False)).astype(np.int64)
        t0 = time.perf_counter()
        res = O.matmul(av, bv, rows=sel, nthreads=threads)
        dt = time.perf_counter() - t0
    else:
        n = threads
        while True:
            sel = np.sort(rng.choice(rows_total, size=n, replace=False)).astype(np.int64) if n < rows_total else \
                np.arange(rows_total, dtype=np.int64)
            t0 = time.perf_counter()
            res = O.matmul(av, bv, rows=sel, nthreads=threads)
            dt = time.perf_counter() - t0
            if n >= rows_total or dt >= budget_s / 8:
                break
            est_full = dt * rows_total / n
            n = rows_total if est_full <= budget_s * 0.6 else min(rows_total, n * max(2, int(budget_s / 8 / max(dt, 1e-3))))
    tflops = 2.0 * n * N * K / dt / 1e12
    full = n == rows_total
    line = {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "host_cpu": host_cpu(), "host_threads": os.cpu_count()}
    if full:
        line["sample"] = (f"all {rows_total} output rows ({n * N} outputs, K={K}): full wall time {dt:.2f} s "
                          f"by the naive oxmera-cpu-style oracle (oracle/oxm_oracle.c, -O2, f32 ascending-k, "
                          f"strided reads, threaded over rows)")
        line["full_s"] = round(dt, 3)
    else:
        line["sample"] = (f"{n} seeded rows of {rows_total} ({n * N} outputs, K={K}) in {dt:.2f} s by the naive "
                          f"oxmera-cpu-style oracle (oracle/oxm_oracle.c, -O2, f32 ascending-k, strided reads, "
                          f"threaded over rows)")
        line["s_per_row"] = dt / n
        line["extrapolated_full_s"] = round(dt * rows_total / n, 1)
        line["extrapolated"] = True
    return line, (sel, res)


def _abs_product(host, sel, desc):
    """sum_k |a_ik| |b_kj| for the selected flattened rows (float32 is ample
    for an error denominator)."""
    from oracle import oracle as O
    (ab, adt, ash, ast), (bb, bdt, bsh, bst) = host

    def dense_abs(buf, dt, shape, strides):
        arr = np.lib.stride_tricks.as_strided(buf.reshape(-1), shape=shape,
                                              strides=[st * buf.itemsize for st in strides])
        return np.abs(O.bf16_to_f32(np.ascontiguousarray(arr)) if dt == O.BF16 else arr.astype(np.float32))

    M = desc["M"]
    A = dense_abs(ab, adt, ash, ast).reshape(-1, desc["K"])
    B = dense_abs(bb, bdt, bsh, bst)
    if B.ndim == 2:
        return (A[sel] @ B).astype(np.float64)
    out = np.empty((len(sel), desc["N"]), np.float64)
    for bi in np.unique(sel // M):
        pick = np.nonzero(sel // M == bi)[0]
        out[pick] = A[sel[pick]] @ B[0 if B.shape[0] == 1 else bi]
    return out


def spot_check(kind: str, res, sample, host=None, comp_rows: int = 64):
    """Parity of the timed output against the oracle on its rows, with the
    |c - r| <= tol * max(|r|, rms(r)), tol = 1e-5*sqrt(K)
    (f32) or 1e-2 (bf16).  Also the componentwise error |c - r| / sum_k |a||b|
    on up to comp_rows of those rows."""
    sel, ref = sample
    out = res["out"].to_numpy().reshape(-1, res["desc"]["N"])
    got = out[sel].astype(np.float64)
    ref = ref.astype(np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) or 1e-30
    tol = 1e-2 if kind in ("bf16", "f16") else 1e-5 * np.sqrt(res["desc"]["K"])
    worst = float(np.max(np.abs(got - ref) / (tol * np.maximum(np.abs(ref), rms))))
    d = {"rows": int(len(sel)), "tol": float(tol), "max_err_over_tol": round(worst, 4), "pass": worst <= 1.0}
    if host is not None:
        idx = np.arange(len(sel)) if len(sel) <= comp_rows else np.linspace(0, len(sel) - 1, comp_rows).astype(int)
        denom = _abs_product(host, sel[idx], res["desc"])
        comp = np.abs(got[idx] - ref[idx]) / np.maximum(denom, 1e-30)
        d["max_componentwise_err"] = float(np.max(comp))
    return d


def kernel_name(kind: str) -> str:
    if kind == "f16":
        return "gemm_kernel_dli16<f16_t, true> (global_load_lds DMA, 2 stages of 64 k, 4 waves, 16x16x32 MFMA)"
    if kind == "bf16":
        return "gemm_kernel_dli16<bf16_t, true> (global_load_lds DMA, 2 stages of 64 k, 4 waves, 16x16x32 MFMA)"
    if kind == "f32":
        return ("gemm_kernel_dlf32<256, 256, 2, 4, false, true, true> (direct-to-LDS f32: global_load_lds DMA, "
                "2 stages of 32 k, 8 waves)")
    if kind == "c2odd":
        return ("gemm_kernel<float,256,256,2,4,Ld::KR,Ld::MNR> (rows 0-4095) + gemm_strip_splitk<float> and "
                "strip_sum (row 4096); time per launch covers all three")
    if kind == "c4":
        return ("gemm_kernel_dlf32<256, 192, 4, 3, false, true, true> (direct-to-LDS f32, 256x192 tiles: 256 tiles, "
                "one round; 12 waves)")
    if kind == "c1":
        return ("gemm_kernel_dlf32<64, 64, 2, 2, false, true, true, 8> (16 tiles on 16 CUs, all 8 K steps in "
                "flight; launch-latency bound)")
    return "gemm_kernel<float,...> (register-staged; tile chosen by the dispatcher)"


def traffic_for(kind: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    p = ROOT / "profiles" / f"traffic_{kind}.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def roofline(kind: str, res):
    avg_ms = res["total_ms"] / res["steps"]
    achieved = res["flops"] / (avg_ms * 1e-3) / 1e12
    peak = PEAK["bf16" if kind in ("bf16", "f16") else "f32"]
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic_for(kind),
            "kernel": kernel_name(kind), "avg_launch_ms": round(avg_ms, 4)}


# Rows of the oracle run (CPU baseline and parity reference at once) per
# configuration: None = every output row; n = n seeded rows (the per-row
# rate is then extrapolated to the full output).
ORACLE_ROWS = {"f32": None, "c1": None, "c2odd": None, "c4": None, "bf16": 256, "f16": 64}


def extra_line(kind: str, steps: int, warmup: int) -> dict:
    """Timing plus the oracle run for one more configuration: its CPU
    baseline and the parity check of the timed output against it (the whole
    output for C1, C2-odd and C4; 256 seeded rows x every column for C3)."""
    steps = max(10, steps // 2) if kind not in ("c1",) else max(50, steps)
    r = time_gpu(kind, steps, warmup)
    r["steps"] = steps
    d = r["desc"]
    v = r["flops"] * steps / (r["total_ms"] * 1e-3) / 1e12
    rows_total = d["batch"] * d["M"]
    nrows = ORACLE_ROWS[kind]
    cb, sample = cpu_baseline(kind, r["host"], d, rows=rows_total if nrows is None else nrows)
    peak = PEAK["f32" if kind in ("f32", "c1", "c2odd", "c4") else "bf16"]
    line = {"config": d, "value": round(v, 2), "unit": "TFLOP/s", "pct_of_peak": round(100 * v / peak, 2),
            "ms_per_step": round(r["total_ms"] / steps, 4),
            "median_launch_ms": round(r["per_ms"][len(r["per_ms"]) // 2], 4),
            "parity_spot_check": spot_check(kind, r, sample, r["host"]), "cpu_baseline": cb}
    if kind == "c1":
        line["us_per_launch"] = round(1e3 * r["total_ms"] / steps, 2)
        line["note"] = "launch-latency bound (0.2 us of MFMA work at peak); no roofline target"
    line["roofline"] = roofline(kind, r)
    return line


def summarize_trace_groups(path: str, kernel: str, skip_frac: float = 0.5) -> dict:
    """Per (kernel, grid) durations from a rocprofv3 kernel trace of a run
    that launches several GEMMs per step (the MLP step): each group's
    dispatches after the first `skip_frac` of them (the warm-up), median and
    average."""
    import csv
    from collections import defaultdict
    groups = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if kernel in r["Kernel_Name"]:
            nm = r["Kernel_Name"]
            nm = (nm[:nm.rfind("(")] if nm.endswith(")") else nm).replace("void ", "").replace("oxm::", "").replace(
                "(anonymous namespace)::", "")
            groups[(nm, int(r["Grid_Size_X"]))].append(
                (int(r["Dispatch_Id"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    out = []
    for (name, grid), v in sorted(groups.items()):
        v.sort()
        d = np.array([x[1] for x in v[int(len(v) * skip_frac):]], dtype=np.float64) / 1e6
        out.append({"kernel": name, "grid_threads": grid, "dispatches": len(v), "used": len(d),
                    "median_ms": round(float(np.median(d)), 5), "avg_ms": round(float(d.mean()), 5)})
    return {"groups": out}


def summarize_trace(path: str, kernel: str, timed: int, after: int) -> dict:
    """Durations of the launches bench.py timed, from a rocprofv3 kernel trace
    of the same command: the dispatches of the kernel (name containing
    `kernel`) in dispatch order, minus the `after` individually timed ones at
    the end, last `timed` of the rest.  Their average is what the HIP-event
    figure (ms_per_step) measures, without the warm-up launches."""
    import csv
    rows = [r for r in csv.DictReader(open(path)) if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    if len(rows) < timed + after:
        raise SystemExit(f"{len(rows)} dispatches of {kernel!r}, fewer than {timed} + {after}")
    win = rows[len(rows) - after - timed:len(rows) - after]
    d = np.array([int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in win], dtype=np.float64) / 1e6
    names = sorted({r["Kernel_Name"] for r in win})
    return {"kernel": names, "dispatches_total": len(rows), "window": [len(rows) - after - timed, len(rows) - after],
            "avg_ms": round(float(d.mean()), 5), "median_ms": round(float(np.median(d)), 5),
            "min_ms": round(float(d.min()), 5), "max_ms": round(float(d.max()), 5),
            "span_ms": round((int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e6 / timed, 5)}


def summarize_pmc(paths: list, copy_bytes: float | None = None) -> dict:
    """Per-kernel means over the dispatches in rocprofv3 --pmc
    counter_collection.csv files (one counter pass per file), grouped by
    kernel name and grid size, with the derived figures the profiles quote:
    MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024
    SIMDs); LDS bank-conflict share = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE;
    L2 hit rate = TCC_HIT / (TCC_HIT + TCC_MISS); FETCH_SIZE / WRITE_SIZE
    (KiB per dispatch) in bytes, FETCH scaled x2 and WRITE x1 -- the factors
    a plain device copy of known size reads as (bench.py --copy-calibration)."""
    import csv
    from collections import defaultdict
    acc = defaultdict(lambda: defaultdict(list))
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            if "oxm::" not in name and "Cijk" not in name:
                continue
            short = (name[:name.rfind("(")] if name.endswith(")") else name).replace("void ", "").replace(
                "oxm::", "").replace("(anonymous namespace)::", "")
            acc[(short, int(r["Grid_Size"]))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    out = []
    for (name, grid), cs in sorted(acc.items()):
        m = {c: sum(v) / len(v) for c, v in cs.items()}
        d = {"kernel": name, "grid_threads": grid, "dispatches": max(len(v) for v in cs.values()), "mean": m}
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and "GRBM_GUI_ACTIVE" in m:
            d["mfma_busy"] = round(m["SQ_VALU_MFMA_BUSY_CYCLES"] / (m["GRBM_GUI_ACTIVE"] / 8 * 1024), 4)
        if "SQ_LDS_BANK_CONFLICT" in m and m.get("SQ_LDS_IDX_ACTIVE"):
            d["lds_bank_conflict_share"] = round(m["SQ_LDS_BANK_CONFLICT"] / m["SQ_LDS_IDX_ACTIVE"], 4)
        if "TCC_HIT_sum" in m and "TCC_MISS_sum" in m:
            d["l2_hit_rate"] = round(m["TCC_HIT_sum"] / (m["TCC_HIT_sum"] + m["TCC_MISS_sum"]), 4)
        if "FETCH_SIZE" in m:
            d["fetch_bytes"] = m["FETCH_SIZE"] * 1024 * 2.0
        if "WRITE_SIZE" in m:
            d["write_bytes"] = m["WRITE_SIZE"] * 1024 * 1.0
        out.append(d)
    return {"kernels": out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=["f32", "bf16", "f16", "mlp", "ops", "c1", "c2odd", "c4"], default="f32",
                    help="f32 / bf16 (the headline configurations) or f16 / c1 / c2odd / c4 time one GEMM; mlp "
                         "times the MLP step alone (for profiling)")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="summarize a rocprofv3 kernel_trace.csv of a bench run instead of running: the timed "
                         "window (--timed launches of --kernel, followed by --after per-launch timings)")
    ap.add_argument("--kernel", default="gemm_kernel", help="substring of the kernel name (--summarize-trace)")
    ap.add_argument("--timed", type=int, default=50, help="launches in the timed window (--summarize-trace)")
    ap.add_argument("--after", type=int, default=20, help="launches after the timed window (--summarize-trace)")
    ap.add_argument("--group", action="store_true",
                    help="with --summarize-trace: per (kernel, grid) medians over the second half of the run")
    ap.add_argument("--summarize-pmc", metavar="CSV", nargs="+",
                    help="summarize rocprofv3 --pmc counter_collection.csv files (one per counter pass) per kernel")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and the extra workload")
    ap.add_argument("--vendor", action="store_true",
                    help="time torch.matmul (the vendor library, hipBLASLt, run as a black box) on the same "
                         "operands and layout instead of this backend: a reference ceiling, not the metric")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (10x), the reference for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE scaling")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(args.summarize_pmc)), flush=True)
        return
    if args.summarize_trace:
        if args.group:
            print(json.dumps(summarize_trace_groups(args.summarize_trace, args.kernel)), flush=True)
        else:
            print(json.dumps(summarize_trace(args.summarize_trace, args.kernel, args.timed, args.after)), flush=True)
        return
    if args.copy_calibration:
        import torch
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0").normal_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "launches": 10}), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the GEMM would shard by rows "
              "of A and C, each GPU running the same kernel on its share); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "mlp":
        print(json.dumps({"mlp": time_mlp(args.steps, args.warmup)}), flush=True)
        return
    if args.workload == "ops":
        print(json.dumps({"ops": time_ops(args.steps)}), flush=True)
        return
    if args.vendor:
        print(json.dumps(time_vendor(args.workload, args.steps, args.warmup)), flush=True)
        return
    main_kind = args.workload
    res = time_gpu(main_kind, args.steps, args.warmup)
    res["steps"] = args.steps
    value = res["flops"] * args.steps / (res["total_ms"] * 1e-3) / 1e12
    line = {
        "metric": "GEMM TFLOP/s + % of MI355X dense MFMA peak (f32 4096³, bf16 8192³)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["total_ms"] / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": main_kind if main_kind in ("bf16", "f16") else "f32",
        "data": "synthetic",
        "config": res["desc"],
        "pct_of_peak": round(100 * value / PEAK["bf16" if main_kind in ("bf16", "f16") else "f32"], 2),
        "median_launch_ms": round(res["per_ms"][len(res["per_ms"]) // 2], 4),
        "roofline": roofline(main_kind, res),
    }
    if not args.no_cpu:
        nrows = ORACLE_ROWS.get(main_kind)
        rows_total = res["desc"]["batch"] * res["desc"]["M"]
        cb, sample = cpu_baseline(main_kind, res["host"], res["desc"], rows=rows_total if nrows is None else nrows)
        line["cpu_baseline"] = cb
        line["parity_spot_check"] = spot_check(main_kind, res, sample, res["host"])
        del res
        line["extra"] = {}
        others = [k for k in ("bf16", "f32") if k != main_kind] + ["f16", "c1", "c2odd", "c4"]
        for other in others:
            line["extra"][other] = extra_line(other, args.steps, args.warmup)
        line["extra"]["mlp"] = time_mlp(max(3, args.steps // 10), 2)
        line["extra"]["mlp"]["cpu_baseline"] = mlp_cpu_baseline()
        line["extra"]["ops"] = time_ops()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
