"""Benchmark of the hot path on one MI355X.

Workload: the ternary decode GEMV, W[4096 x 4096]
with trits {-1,0,+1} at p = {.25,.5,.25} packed 2 bits/weight row-major, one
fp32 per-tensor scale, x[4096] f32 ~ N(0,1) quantised to int8 by per-token
absmax, int32 accumulation, fp32 rescale, batch 1.  A step is one pass of
the path: pack-act-rows(x) then the GEMV, on the next of 128 distinct weight
copies (512 MiB, twice the 256 MB Infinity Cache, so weights stream from HBM).

value = algorithmic bytes of a step (4,227,076 B: packed W, f32 x, beta, f32 y)
      / measured step time, in GB/s.  The roofline object is for the GEMV
kernel alone (4,214,792 B per launch: W, int8 x, gamma, beta, y) over its
average launch duration, measured with HIP events on the stream the kernels
run on.  cpu_baseline is the CPU restatement (oracle/) of the same step on
the host cores.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nelisp-gpu_amd"))

HBM_PEAK_GBS = 8000.0
OUT, COLS = 4096, 4096
COPIES = 128
STEP_BYTES = OUT * COLS // 4 + COLS * 4 + 4 + OUT * 4          # 4,227,076
GEMV_BYTES = OUT * COLS // 4 + COLS + 4 + 4 + OUT * 4          # 4,214,792
METRIC = "ternary GEMV GB/s (% HBM peak) at 4096²; decode tok/s, 2B ternary model, batch 1"


def gpu_bench(steps: int, warmup: int):
    import nlgpu

    nlgpu.init()
    seed = 20260921 + 1
    t = nlgpu.trits(seed, (OUT, COLS))
    w_one = nlgpu.pack_ternary(t)
    wbytes = w_one.nbytes
    # 128 distinct copies: each row set is the same trits rotated by copy index
    # (different bytes per copy, same statistics)
    dW = nlgpu.DeviceArray(wbytes * COPIES)
    for c in range(COPIES):
        dW.upload(np.roll(w_one, c, axis=0), offset=c * wbytes)
    x = nlgpu.normal(seed + 100, COLS)
    beta = np.array([1.0], np.float32)
    dx, dbeta = nlgpu.to_device(x), nlgpu.to_device(beta)
    dxq = nlgpu.DeviceArray(COLS)
    dg = nlgpu.DeviceArray(4)
    dy = nlgpu.DeviceArray(OUT * 4)
    L = nlgpu.lib()
    stream = L.nlg_default_stream()

    def w_ptr(i):
        return dW.ptr + (i % COPIES) * wbytes

    def step(i):
        L.nlg_pack_act_rows(dx.ptr, dxq.ptr, dg.ptr, 1, COLS, stream)
        L.nlg_ternary_linear_i8(dxq.ptr, dg.ptr, w_ptr(i), None, dbeta.ptr, 0, dy.ptr, 1, OUT, COLS, stream)

    for i in range(warmup):
        step(i)
    nlgpu.sync()
    e0, e1 = nlgpu.Event(), nlgpu.Event()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    step_ms = e0.elapsed_ms(e1) / steps

    # the GEMV kernel alone: back-to-back launches over the rotating copies
    nlgpu.sync()
    g0, g1 = nlgpu.Event(), nlgpu.Event()
    g0.record(stream)
    for i in range(steps):
        L.nlg_ternary_linear_i8(dxq.ptr, dg.ptr, w_ptr(i), None, dbeta.ptr, 0, dy.ptr, 1, OUT, COLS, stream)
    g1.record(stream)
    gemv_ms = g0.elapsed_ms(g1) / steps
    nlgpu.sync()
    return dict(step_ms=step_ms, gemv_ms=gemv_ms, device=nlgpu.device_name(), x=x, w_one=w_one)


def cpu_baseline(x, w_one, seconds: float):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import nlg_oracle as orc

    beta = np.array([1.0], np.float32)
    n, t0 = 0, time.perf_counter()
    while True:
        xq, g = orc.pack_act_rows(x, 1, COLS)
        orc.ternary_linear_i8(xq, g, w_one, None, beta, 1, OUT, COLS)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    return dict(value=round(STEP_BYTES * n / dt / 1e9, 3), unit="GB/s", cores=orc.threads(), kind="port",
                sample=f"{n} steps of the 4096x4096 config-2 step (pack-act-rows + ternary GEMV, "
                       f"C restatement, OpenMP over output rows) in {dt:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the decode path is not sharded); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    r = gpu_bench(args.steps, args.warmup)
    value = STEP_BYTES / (r["step_ms"] * 1e-3) / 1e9
    achieved = GEMV_BYTES / (r["gemv_ms"] * 1e-3) / 1e9
    cpu = cpu_baseline(r["x"], r["w_one"], args.cpu_seconds)
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "ternary decode GEMV W[4096x4096] 2-bit, x f32 -> int8 absmax, batch 1, "
                               "128 rotated weight copies (512 MiB)",
                   "out": OUT, "cols": COLS, "batch": 1, "weight_copies": COPIES,
                   "step": "pack-act-rows + ternary GEMV"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_tern_i8_fast<4,1>", "bytes_per_launch": GEMV_BYTES,
                     "us_per_launch": round(r["gemv_ms"] * 1e3, 3)},
        "cpu_baseline": cpu,
        "device": r["device"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
