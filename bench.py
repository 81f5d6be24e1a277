"""Benchmark of the MI355X GEMM backend (one JSON line on stdout).

Metric: GEMM TFLOP/s and % of MI355X dense MFMA peak.
A "step" is one GEMM launch over inputs already resident in HBM.

  default workload  configs[1]: f32 C = A.B, 4096 x 4096 x 4096, row-major,
                    A, B ~ N(0,1) from a seed                    -> "value"
  second line item  configs[2]: bf16 in / f32 out, 8192^3, A row-major,
                    B a transposed strided view (strides [1, 8192]),
                    N(0, 0.02)                                  -> "extra"

Timing: W untimed warm-up launches, then K launches bracketed by HIP events
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


def make_inputs(kind: str):
    import oxmera_amd as ox
    dev = ox.Device.rocm(0)
    if kind == "f32":
        m = k = n = 4096
        rng = np.random.default_rng(12345)
        a_h = rng.standard_normal((m, k), dtype=np.float32)
        b_h = rng.standard_normal((k, n), dtype=np.float32)
        a = ox.Tensor.from_numpy(a_h, dev, ox.DType.F32)
        b = ox.Tensor.from_numpy(b_h, dev, ox.DType.F32)
        host = (a_h, b_h)
        desc = {"workload": "f32 matmul 4096x4096x4096, A and B contiguous row-major (BASELINE configs[1])",
                "M": m, "N": n, "K": k, "a_strides": [k, 1], "b_strides": [n, 1], "seed": 12345}
    else:
        m = k = n = 8192
        rng = np.random.default_rng(54321)
        a_h = ox.f32_to_bf16_bits(rng.normal(0, 0.02, (m, k)).astype(np.float32))
        bbuf = ox.f32_to_bf16_bits(rng.normal(0, 0.02, (n, k)).astype(np.float32))
        a = ox.Tensor.from_numpy(a_h, dev, ox.DType.BF16)
        b = ox.Tensor.from_numpy(bbuf, dev, ox.DType.BF16).permute([1, 0])  # [K, N], strides [1, K]
        host = (a_h, bbuf)
        desc = {"workload": "bf16-in f32-out matmul 8192^3, A row-major, B transposed view strides [1,8192] "
                            "(BASELINE configs[2])",
                "M": m, "N": n, "K": k, "a_strides": [k, 1], "b_strides": [1, k], "seed": 54321}
    out = ox.Tensor.empty((m, n), ox.DType.F32, dev)
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
        for _ in range(warmup):
            be.matmul(a, b, out=out, stream=stream)
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
    flops = 2.0 * desc["M"] * desc["N"] * desc["K"]
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
            for _ in range(warmup):
                model.train_step(x, t)
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


def cpu_baseline(kind: str, host, desc, budget_s: float = 12.0):
    """The naive oracle on a bounded sample of output rows, all host threads."""
    from oracle import oracle as O
    threads = min(os.cpu_count() or 1, 16)
    a_h, b_h = host
    M, N, K = desc["M"], desc["N"], desc["K"]
    if kind == "f32":
        av = O.StridedView.contiguous(a_h)
        bv = O.StridedView.contiguous(b_h)
    else:
        av = O.StridedView(a_h.reshape(-1), O.BF16, (M, K), (K, 1), 0)
        bv = O.StridedView(b_h.reshape(-1), O.BF16, (K, N), (1, K), 0)
    rows = threads
    while True:
        sel = np.random.default_rng(7).choice(M, size=rows, replace=False).astype(np.int64)
        t0 = time.perf_counter()
        res = O.matmul(av, bv, rows=sel, nthreads=threads)
        dt = time.perf_counter() - t0
        if dt >= budget_s / 4 or rows >= M:
            break
        rows = min(M, rows * max(2, int(budget_s / 4 / max(dt, 1e-3))))
    tflops = 2.0 * rows * N * K / dt / 1e12
    return {"value": tflops, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {M} output rows ({rows * N} outputs, K={K}) in {dt:.2f} s by the naive "
                      f"oxmera-cpu-style oracle (oracle/oxm_oracle.c, -O2, f32 ascending-k), "
                      f"extrapolated full time {dt * M / rows:.0f} s"}, (sel, res)


def kernel_name(kind: str) -> str:
    return ("gemm_kernel<float,256,256,2,4,Ld::K,Ld::MN> (register-staged LDS double buffer, 8 waves)" if kind == "f32"
            else "gemm_kernel_dl<bf16_t,256,256,2,4,2,64> (direct-to-LDS, 2 stages of 64 k, 8 waves)")


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
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK[kind], "unit": "TFLOP/s",
            "frac": round(achieved / PEAK[kind], 4), "traffic": traffic_for(kind),
            "kernel": kernel_name(kind), "avg_launch_ms": round(avg_ms, 4)}


def spot_check(kind: str, res, sample):
    """Parity of the timed output on the CPU-baseline rows."""
    sel, ref = sample
    got = res["out"].to_numpy()[sel].astype(np.float64)
    ref = ref.astype(np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) or 1e-30
    tol = 1e-5 * np.sqrt(res["desc"]["K"]) if kind == "f32" else 1e-2
    worst = float(np.max(np.abs(got - ref) / (tol * np.maximum(np.abs(ref), rms))))
    return {"rows": int(len(sel)), "max_err_over_tol": round(worst, 4), "pass": worst <= 1.0}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=["f32", "bf16", "mlp"], default="f32",
                    help="f32 / bf16 time one GEMM; mlp times the MLP step alone (for profiling)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and the extra workload")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (10x), the reference for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE scaling")
    args = ap.parse_args()
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
              "of A/C, see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "mlp":
        print(json.dumps({"mlp": time_mlp(args.steps, args.warmup)}), flush=True)
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
        "dtype": "f32" if main_kind == "f32" else "bf16",
        "data": "synthetic",
        "config": res["desc"],
        "pct_of_peak": round(100 * value / PEAK[main_kind], 2),
        "median_launch_ms": round(res["per_ms"][len(res["per_ms"]) // 2], 4),
        "roofline": roofline(main_kind, res),
    }
    if not args.no_cpu:
        cb, sample = cpu_baseline(main_kind, res["host"], res["desc"])
        line["cpu_baseline"] = cb
        line["parity_spot_check"] = spot_check(main_kind, res, sample)
        other = "bf16" if main_kind == "f32" else "f32"
        del res
        r2 = time_gpu(other, max(10, args.steps // 2), args.warmup)
        r2["steps"] = max(10, args.steps // 2)
        v2 = r2["flops"] * r2["steps"] / (r2["total_ms"] * 1e-3) / 1e12
        line["extra"] = {other: {"config": r2["desc"], "value": round(v2, 2), "unit": "TFLOP/s",
                                 "pct_of_peak": round(100 * v2 / PEAK[other], 2),
                                 "ms_per_step": round(r2["total_ms"] / r2["steps"], 4),
                                 "median_launch_ms": round(r2["per_ms"][len(r2["per_ms"]) // 2], 4),
                                 "roofline": roofline(other, r2)}}
        del r2
        line["extra"]["mlp"] = time_mlp(max(3, args.steps // 10), 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
