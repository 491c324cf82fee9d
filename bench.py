"""Benchmark of the hot path on one MI355X.

Workload: the ternary decode GEMV, W[4096 x 4096]
with trits {-1,0,+1} at p = {.25,.5,.25} packed 2 bits/weight row-major, one
fp32 per-tensor scale, x[4096] f32 ~ N(0,1) quantised to int8 by per-token
absmax, int32 accumulation, fp32 rescale, batch 1.  A step is one pass of
the path -- quantise x, then the GEMV -- on the next of 128 distinct weight
copies (512 MiB, twice the 256 MB Infinity Cache, so weights come from HBM).
The step is one kernel launch (nlg_ternary_linear: quantisation fused into
the GEMV).

value    = algorithmic bytes of a step (4,227,076 B: packed W 4 MiB, f32 x,
           beta, f32 y) / measured step time, GB/s.
roofline = the same kernel (the only one in the step): those bytes over its
           average launch duration from HIP events on the stream it runs on.
roofline.traffic is the HBM bytes per launch of the PMC traffic summary in
profiles/ (read, not measured here); roofline.ceiling_us is what one dependent
launch can reach on this part: the measured empty-launch floor plus the
bytes at the kernel's own streaming rate (the 128-matrix launch).
device_timing: the same step with every wave's start and end read from the
device's 100 MHz wall clock in a replayed graph (kernel duration and the idle
gap to the next launch), no profiler attached.
Extra fields: the GEMV alone on pre-quantised int8 x (4,214,792 B/launch),
the same GEMV kernel over all 128 copies stacked into one [524288 x 4096]
launch (launch cost amortised: the kernel's streaming rate), and the
measured launch floor (an empty kernel, back to back).
cpu_baseline: the CPU restatement (oracle/) of the same step on host cores.
matmul_config1 / softmax_config3 / swiglu_ffn_config4: configs 1, 3 and 4 at
their full sizes.
decode: config 5, the 30-layer ternary decoder stack at batch 1 and 32 --
tokens/s over 256 greedy steps after a 512-token prompt, the step's
algorithmic bytes (every weight, the LM head, K/V of the cached positions)
over its time, and each kernel of a step timed alone at the last position.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep]
"""
import argparse
import ctypes
import ctypes as C
import json
import os
import re
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
# HBM bytes per step: the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary of
# this kernel (read from the committed profile, not measured by this run)
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "ternary_gemv_4096_decode_pmc_traffic.md")
WALL_CLOCK_MHZ = 100.0  # s_memrealtime's constant clock on this part


def step_traffic():
    """(bytes per step, FETCH_SIZE calibration factor) from the traffic
    summary in profiles/, or (None, None) when it is not there."""
    try:
        txt = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None, None
    m = re.search(r"\*\*traffic = ([\d,]+) B\*\*", txt)
    f = re.search(r"factor \*\*([\d.]+)\*\*", txt)
    return (int(m.group(1).replace(",", "")) if m else None), (f.group(1) if f else None)
METRIC = "ternary GEMV GB/s (% HBM peak) at 4096²; decode tok/s, 2B ternary model, batch 1"


def timed(fn, n, stream, stats=None):
    """Average ms per call of fn(i) over at least max(n, 200) calls.  The
    calls are captured into a HIP graph of COPIES launches (one pass over the
    rotating weight copies) replayed R = max(16, ceil(max(n, 200) / COPIES))
    times, each replay between its own pair of events on the launch stream,
    so host-side launch overhead (Python, ctypes, hipLaunchKernel) is not
    what gets measured.  Returns the mean over all R * COPIES launches; when
    `stats` is a dict it also receives the launch count and the median / p10
    / p90 of the per-launch time across the replays."""
    import nlgpu
    nlgpu.graph_begin(stream)
    for i in range(COPIES):
        fn(i)
    g = nlgpu.graph_end(stream)
    reps = max(16, -(-max(n, 200) // COPIES))
    nlgpu.graph_launch(g, stream)  # warm replay
    ev = [nlgpu.Event() for _ in range(reps + 1)]
    ev[0].record(stream)
    for r in range(reps):
        nlgpu.graph_launch(g, stream)
        ev[r + 1].record(stream)
    per = np.array([ev[r].elapsed_ms(ev[r + 1]) / COPIES for r in range(reps)])
    ms = ev[0].elapsed_ms(ev[reps]) / (reps * COPIES)
    nlgpu.graph_destroy(g)
    if stats is not None:
        stats.update(launches=reps * COPIES, replays=reps, mean_us=round(ms * 1e3, 4),
                     median_us=round(float(np.median(per)) * 1e3, 4),
                     p10_us=round(float(np.percentile(per, 10)) * 1e3, 4),
                     p90_us=round(float(np.percentile(per, 90)) * 1e3, 4))
    return ms


def copy_peak_gbs(stream, nbytes=1 << 30, reps=10):
    """Device-to-device copy rate (bytes read + written per second) of a
    1 GiB buffer, the measured ceiling next to the 8 TB/s spec peak."""
    import nlgpu
    a, b = nlgpu.DeviceArray(nbytes), nlgpu.DeviceArray(nbytes)
    L = nlgpu.lib()
    L.nlg_copy_d2d(b.ptr, a.ptr, nbytes, stream)
    e0, e1 = nlgpu.Event(), nlgpu.Event()
    e0.record(stream)
    for _ in range(reps):
        L.nlg_copy_d2d(b.ptr, a.ptr, nbytes, stream)
    e1.record(stream)
    gbs = 2 * nbytes * reps / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    a.free()
    b.free()
    return gbs


def gpu_bench(steps: int, warmup: int, sweep: bool):
    import nlgpu

    nlgpu.init()
    seed = 20260921 + 1
    t = nlgpu.trits(seed, (OUT, COLS))
    w_one = nlgpu.pack_ternary(t)
    wbytes = w_one.nbytes
    # 128 distinct copies: the same trits with rows rotated per copy
    dW = nlgpu.DeviceArray(wbytes * COPIES)
    for c in range(COPIES):
        dW.upload(np.roll(w_one, c, axis=0), offset=c * wbytes)
    x = nlgpu.normal(seed + 100, COLS)
    beta = np.array([1.0], np.float32)
    dx, dbeta = nlgpu.to_device(x), nlgpu.to_device(beta)
    dxq = nlgpu.DeviceArray(COLS)
    dg = nlgpu.DeviceArray(4)
    dy = nlgpu.DeviceArray(OUT * 4)
    dY = nlgpu.DeviceArray(OUT * COPIES * 4)
    L = nlgpu.lib()
    stream = L.nlg_default_stream()
    res = dict(device=nlgpu.device_name(), x=x, w_one=w_one)

    def w_ptr(i):
        return dW.ptr + (i % COPIES) * wbytes

    def step(i, rpw=0):
        rc = L.nlg_ternary_linear_cfg(dx.ptr, w_ptr(i), None, dbeta.ptr, 0, dy.ptr, None, 1, OUT, COLS,
                                      rpw, None, 0, stream)
        if rc:
            raise nlgpu.NlgError(nlgpu.last_error())

    def gemv(i, rpw=4, wpb=4):
        L.nlg_ternary_linear_i8_cfg(dxq.ptr, dg.ptr, w_ptr(i), None, dbeta.ptr, 0, dy.ptr, 1, OUT, COLS,
                                    rpw, wpb, stream)

    L.nlg_pack_act_rows(dx.ptr, dxq.ptr, dg.ptr, 1, COLS, stream)
    for i in range(warmup):
        step(i)
    nlgpu.sync()
    res["step_stats"] = {}
    res["step_ms"] = timed(step, steps, stream, res["step_stats"])
    nlgpu.sync()
    # the same step with each wave's start and end on the device's wall
    # clock (nlg_ternary_linear_timed): per launch of the last replay, the
    # first wave's start to the last wave's end, and the idle gap to the
    # next launch's first wave
    nst = int(L.nlg_ternary_linear_timed_stamps(OUT))
    dts = nlgpu.DeviceArray(nst * COPIES)

    def tstep(i):
        rc = L.nlg_ternary_linear_timed(dx.ptr, w_ptr(i), dbeta.ptr, dy.ptr, OUT, COLS,
                                        dts.ptr + (i % COPIES) * nst, nst, stream)
        if rc:
            raise nlgpu.NlgError(nlgpu.last_error())

    for i in range(warmup):
        tstep(i)
    res["timed_ms"] = timed(tstep, steps, stream)
    st = dts.download(np.uint64, nst * COPIES // 8).reshape(COPIES, -1, 2).astype(np.int64)
    t0, t1 = st[:, :, 0].min(axis=1), st[:, :, 1].max(axis=1)
    res["device_us"] = (t1 - t0) / WALL_CLOCK_MHZ
    res["gap_us"] = (t0[1:] - t1[:-1]) / WALL_CLOCK_MHZ
    res["replay_span_us"] = (t1[-1] - t0[0]) / WALL_CLOCK_MHZ
    dts.free()
    nlgpu.sync()
    for i in range(warmup):
        gemv(i)
    res["gemv_ms"] = timed(gemv, steps, stream)
    nlgpu.sync()
    # one launch over all copies stacked: [COPIES*OUT x COLS]
    stacked = lambda i: L.nlg_ternary_linear_i8_cfg(dxq.ptr, dg.ptr, dW.ptr, None, dbeta.ptr, 0, dY.ptr, 1,
                                                    OUT * COPIES, COLS, 4, 4, stream)
    stacked(0)
    nlgpu.sync()
    e0, e1 = nlgpu.Event(), nlgpu.Event()
    e0.record(stream)
    for i in range(20):
        stacked(i)
    e1.record(stream)
    res["stacked_ms"] = e0.elapsed_ms(e1) / 20
    nlgpu.sync()
    # launch floor: an empty fill of 16 bytes, back to back
    res["floor_ms"] = timed(lambda i: L.nlg_zero(dg.ptr, 4, stream), steps, stream)
    nlgpu.sync()
    res["copy_gbs"] = copy_peak_gbs(stream)
    nlgpu.sync()
    if sweep:
        sw = {}
        for rpw in (1, 2, 4, 8):
            for i in range(warmup):
                step(i, rpw)
            sw[f"fused rpw={rpw}"] = round(timed(lambda i: step(i, rpw), steps, stream) * 1e3, 3)
        for rpw in (1, 2, 4, 8):
            for wpb in (1, 2, 4):
                f = lambda i: gemv(i, rpw, wpb)
                for i in range(warmup):
                    f(i)
                sw[f"i8 rpw={rpw} wpb={wpb}"] = round(timed(f, steps, stream) * 1e3, 3)
        res["sweep_us"] = sw
    nlgpu.sync()
    return res


# ---------------------------------------------------------------- config 5

STACK = dict(layers=30, d_model=2560, heads=20, kv_heads=5, head_dim=128, d_ff=6912, vocab=128256)
PROMPT, DECODE = 512, 256


class _Ptr:
    """A device pointer from the stack, shaped like nlgpu.DeviceArray."""

    def __init__(self, ptr, nbytes):
        self.ptr, self.nbytes = ptr, nbytes

    def as_buffer(self, nfloats=None):
        import nlgpu
        return nlgpu.Buffer(self.ptr, self.nbytes // 4 if nfloats is None else int(nfloats))


def _tensor(s, name, layer=-1):
    import ctypes as C
    import nlgpu
    p, n = C.c_void_p(), C.c_size_t(0)
    if nlgpu.lib().nlg_stack_tensor(s.h, name.encode(), layer, C.byref(p), C.byref(n)):
        raise nlgpu.NlgError(nlgpu.last_error())
    return _Ptr(p.value, n.value)


def _per_launch_us(fn, n, stream):
    """us per launch of fn(i), i = 0..n-1, captured in one graph."""
    import nlgpu
    nlgpu.graph_begin(stream)
    for i in range(n):
        fn(i)
    g = nlgpu.graph_end(stream)
    nlgpu.graph_launch(g, stream)
    e0, e1 = nlgpu.Event(), nlgpu.Event()
    e0.record(stream)
    for _ in range(3):
        nlgpu.graph_launch(g, stream)
    e1.record(stream)
    us = e0.elapsed_ms(e1) * 1e3 / (3 * n)
    nlgpu.graph_destroy(g)
    return us


def _decode_kernels(s, batch, stream):
    """The five kernels of one decoder layer at the last cache position
    (767), each a function of the launch index i that rotates over the 30
    layers' weights, with its algorithmic bytes per launch."""
    import nlgpu
    c = STACK
    max_seq = PROMPT + DECODE
    L, d, f = c["layers"], c["d_model"], c["d_ff"]
    nq, nkv = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    T = lambda n, l=-1: _tensor(s, n, l)
    x, co, si = T("x"), T("rope_cos"), T("rope_sin")
    pos = nlgpu.to_device(np.array([max_seq - 1], np.int32))
    q = nlgpu.DeviceArray(batch * nq * 4)
    h = nlgpu.DeviceArray(batch * f * 4)
    ws = nlgpu.DeviceArray(nlgpu.decode_attn_f16_workspace(batch, c["heads"], c["kv_heads"], c["head_dim"], max_seq))
    ly = [{k: T(k, l) for k in ("wqkv", "bqkv", "wo", "bo", "wgu", "bgu", "wd", "bd", "gattn", "gffn", "kc", "vc")}
          for l in range(L)]
    eps = 1e-5
    n = 4 * L
    kv_bytes = batch * max_seq * nkv * 2 * 2  # K and V, fp16, every cached position
    kern = {
        "qkv_rope_append": (lambda i: nlgpu.rms_ternary_qkv_rope(
            x, ly[i % L]["gattn"], eps, ly[i % L]["wqkv"], ly[i % L]["bqkv"], q, ly[i % L]["kc"], ly[i % L]["vc"],
            co, si, pos, batch, c["heads"], c["kv_heads"], c["head_dim"], max_seq, d, stream=stream),
            (nq + 2 * nkv) * d // 4 + batch * (d * 4 + nq * 4 + 2 * nkv * 2)),
        "attention_chunks": (lambda i: nlgpu.decode_attn_f16_chunks(
            q, ly[i % L]["kc"], ly[i % L]["vc"], pos, batch, c["heads"], c["kv_heads"], c["head_dim"], max_seq, ws,
            stream=stream), kv_bytes + batch * nq * 4),
        "attn_merge_o_proj_residual": (lambda i: nlgpu.attn_ternary_linear_residual(
            ws, batch, c["heads"], c["kv_heads"], c["head_dim"], max_seq, ly[i % L]["wo"], None, ly[i % L]["bo"],
            x, x, d, stream=stream), d * nq // 4 + batch * d * 8),
        "rms_gate_up_swiglu": (lambda i: nlgpu.rms_ternary_swiglu(
            x, ly[i % L]["gffn"], eps, ly[i % L]["wgu"], ly[i % L]["bgu"], h, batch, f, d, stream=stream),
            2 * f * d // 4 + batch * (d * 4 + f * 4)),
        "down_proj_residual": (lambda i: nlgpu.ternary_linear_residual(
            h, ly[i % L]["wd"], None, ly[i % L]["bd"], x, x, batch, d, f, stream=stream),
            d * f // 4 + batch * (f * 4 + d * 8)),
    }
    return kern, L


def decode_bench(batch: int, stream):
    """Config 5: prefill 512 random ids (teacher-forced token steps), then 256
    greedy steps, one captured graph per step; then each kernel of a step
    timed on its own over the 30 layers' weights."""
    import nlgpu
    c = STACK
    max_seq = PROMPT + DECODE
    s = nlgpu.Stack(**c, max_seq=max_seq, batch=batch, seed=20260921 + 5)
    ids = (nlgpu.uniform(20260921 + 55, batch * PROMPT) * c["vocab"]).astype(np.int32).reshape(batch, PROMPT)
    e0, e1, e2 = nlgpu.Event(), nlgpu.Event(), nlgpu.Event()
    s.prefill(ids)  # warm: allocates the prefill rows and scratch
    e0.record(stream)
    s.prefill(ids)  # all 512 prompt tokens at once, then the first greedy token
    e1.record(stream)
    prefill_ms = e0.elapsed_ms(e1)
    s.step(1)  # first decode step: captures the step graph
    e1.record(stream)
    s.step(DECODE - 1)
    e2.record(stream)
    decode_ms = e1.elapsed_ms(e2) * DECODE / (DECODE - 1)
    toks, _ = s.tokens()
    assert (toks[:, :max_seq] >= 0).all()
    # per-kernel, at the last position (768 cached), rotating over the layers
    kern, L = _decode_kernels(s, batch, stream)
    n = 4 * L
    d, f = c["d_model"], c["d_ff"]
    nq, nkv = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    per = {}
    for name, (fn, nbytes) in kern.items():
        us = _per_launch_us(fn, n, stream)
        per[name] = {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
    lm_bytes = c["vocab"] * d // 4 + batch * (d * 4 + c["vocab"] * 4)
    ms_tok = decode_ms / DECODE
    layer_bytes = (nq + 2 * nkv) * d // 4 + d * nq // 4 + 2 * f * d // 4 + d * f // 4
    # per step: every weight once, the LM head, and K/V of the cached positions
    mean_len = PROMPT + (DECODE + 1) / 2.0
    step_bytes = L * layer_bytes + c["vocab"] * d // 4 + L * batch * mean_len * nkv * 2 * 2
    s.close()
    return {"batch": batch, "tok_s": round(batch * DECODE / (decode_ms * 1e-3), 1),
            "ms_per_step": round(ms_tok, 4), "prefill_ms": round(prefill_ms, 2),
            "prefill": "batch x 512 prompt rows at once: batched int8 MFMA linears + causal attention, "
                       "then the LM head on the last row",
            "prefill_tok_s": round(batch * PROMPT / (prefill_ms * 1e-3), 1),
            "step_bytes": int(step_bytes), "step_gbs": round(step_bytes / (ms_tok * 1e-3) / 1e9, 1),
            "step_frac": round(step_bytes / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            # per layer: 5 launches, or 9 when the linears take the batched (quantise + GEMM) form
            "launches_per_step": L * (9 if batch >= 4 else 5) + (2 if batch >= 4 else 1) + (2 if batch > 1 else 1),
            "lm_head_bytes": int(lm_bytes), "per_kernel": per}


# ---------------------------------------------------------------- config 1

def matmul_bench(stream):
    """Config 1: f32 C[256x256] = A[256x256] B[256x256], A, B ~ U[-1,1] from
    a seed, through the by-name kernels (the vkmatmul path), each variant
    graph-timed; checked against a float64 product."""
    import nlgpu
    M = K = N = 256
    a = (nlgpu.uniform(20260921 + 10, M * K) * 2 - 1).astype(np.float32)
    b = (nlgpu.uniform(20260921 + 11, K * N) * 2 - 1).astype(np.float32)
    da, db, dc = nlgpu.to_device(a), nlgpu.to_device(b), nlgpu.DeviceArray(M * N * 4)
    want = a.reshape(M, K).astype(np.float64) @ b.reshape(K, N).astype(np.float64)
    flops = 2 * M * K * N
    out = {}
    for name, groups in (("matmul", (M * N + 63) // 64), ("matmul-tiled", (M // 16) * (N // 16)),
                         ("matmul-reg", ((M // 4) * (N // 4) + 63) // 64)):
        fn = lambda i: nlgpu.dispatch(name, [da, db, dc], [M, K, N], groups, stream=stream)
        fn(0)
        nlgpu.sync()
        err = float(np.abs(dc.download(np.float32, M * N).reshape(M, N) - want).max() / np.abs(want).max())
        us = _per_launch_us(fn, 128, stream)
        out[name] = {"us": round(us, 3), "gflops": round(flops / us / 1e3, 1), "max_rel_err": err}
    best = min(out, key=lambda k: out[k]["us"])
    out["flops"] = flops
    out["best"] = best
    out["frac_fp32_peak"] = round(out[best]["gflops"] / 157300.0, 5)
    out["note"] = ("33.5 MFLOP: launch/latency-bound (0.2 us of fp32 peak); every output is the reference's "
                   "own chain of 256 dependent f32 adds (bit-identical), one 16x16 tile per CU")
    return out


# ---------------------------------------------------------------- config 3

SM_HEADS, SM_N = 32, 4096
SM_BYTES = 2 * 4 * SM_HEADS * SM_N * SM_N  # read + write of every f32, 4,294,967,296


def softmax_bench(stream):
    """Config 3: row softmax in place over [32 x 4096 x 4096] f32 scores,
    N(0, 3^2) with -inf above each head's diagonal (drawn on the device)."""
    import nlgpu
    n = SM_HEADS * SM_N * SM_N
    a = nlgpu.DeviceArray(n * 4)
    nlgpu.fill_normal(a, n, 20260921 + 3, 3.0, SM_N, stream=stream)
    rows = SM_HEADS * SM_N
    nlgpu.softmax_rows(a, a, rows, SM_N, stream=stream)  # warm
    e0, e1 = nlgpu.Event(), nlgpu.Event()
    reps = 5
    e0.record(stream)
    for _ in range(reps):
        nlgpu.softmax_rows(a, a, rows, SM_N, stream=stream)
    e1.record(stream)
    ms = e0.elapsed_ms(e1) / reps
    a.free()
    gbs = SM_BYTES / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "bytes": SM_BYTES, "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "shape": [SM_HEADS, SM_N, SM_N], "kernel": "k_softmax_reg (one workgroup per row, in place)"}


# ---------------------------------------------------------------- config 4

FFN_D, FFN_F, FFN_COPIES = 2560, 6912, 40
INT8_PEAK_TOPS = 5000.0


def ffn_bench(stream):
    """Config 4: h = silu(x Wg) * (x Wu), y = h Wd, all ternary 2-bit with
    per-tensor scales and int8 absmax activations, at 1, 16 and 512 tokens;
    40 distinct FFN weight copies (531 MB) rotated so weights stream from HBM.
    Tiled copies of the weights are registered once before timing (as a
    model would at load); the matrix-core GEMMs (16 and 512 tokens) read them."""
    import nlgpu
    seed = 20260921 + 4
    tg = nlgpu.trits(seed, (FFN_F, FFN_D))
    tu = nlgpu.trits(seed + 1, (FFN_F, FFN_D))
    td = nlgpu.trits(seed + 2, (FFN_D, FFN_F))
    gu = np.empty((2 * FFN_F, FFN_D // 16), np.uint32)
    gu[0::2], gu[1::2] = nlgpu.pack_ternary(tg), nlgpu.pack_ternary(tu)
    wd = nlgpu.pack_ternary(td)
    dgu = nlgpu.DeviceArray(gu.nbytes * FFN_COPIES)
    dwd = nlgpu.DeviceArray(wd.nbytes * FFN_COPIES)
    for c in range(FFN_COPIES):
        dgu.upload(np.roll(gu, 2 * c, axis=0), offset=c * gu.nbytes)
        dwd.upload(np.roll(wd, c, axis=0), offset=c * wd.nbytes)
    bgu = nlgpu.to_device(np.full(2 * FFN_F, 1.0 / np.sqrt(FFN_D / 2), np.float32))
    bd = nlgpu.to_device(np.array([1.0 / np.sqrt(FFN_F / 2)], np.float32))
    wbytes = gu.nbytes + wd.nbytes
    out = {}
    gu_c = [_Ptr(dgu.ptr + c * gu.nbytes, gu.nbytes) for c in range(FFN_COPIES)]
    wd_c = [_Ptr(dwd.ptr + c * wd.nbytes, wd.nbytes) for c in range(FFN_COPIES)]
    for c in range(FFN_COPIES):
        nlgpu.ternary_tiled_register(gu_c[c], 2 * FFN_F, FFN_D)
        nlgpu.ternary_tiled_register(wd_c[c], FFN_D, FFN_F)
    for B in (1, 16, 512):
        x = nlgpu.to_device(nlgpu.normal(seed + 10 + B, B * FFN_D))
        h = nlgpu.DeviceArray(B * FFN_F * 4)
        y = nlgpu.DeviceArray(B * FFN_D * 4)

        def ffn(i):
            c = i % FFN_COPIES
            nlgpu.rms_ternary_swiglu(x, None, 0.0, gu_c[c], bgu, h, B, FFN_F, FFN_D, stream=stream)
            nlgpu.ternary_linear(h, wd_c[c], None, bd, y, B, FFN_D, FFN_F, stream=stream)
        ffn(0)  # reserves the batched scratch outside the capture
        us = _per_launch_us(ffn, FFN_COPIES, stream)
        nbytes = wbytes + 2 * B * FFN_D * 4
        ops = 2 * B * (2 * FFN_F * FFN_D + FFN_D * FFN_F)
        r = {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
             "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "tops": round(ops / us / 1e6, 2),
             "frac_int8_mfma": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
             "path": "fused GEMV (2 launches)" if B < 4 else "per-token quantise + int8 MFMA GEMM (4 launches)"
             + (", tiled weight copies" if B >= 4 else "")}
        out[f"B{B}"] = r
    for c in range(FFN_COPIES):
        nlgpu.ternary_tiled_unregister(gu_c[c])
        nlgpu.ternary_tiled_unregister(wd_c[c])
    dgu.free()
    dwd.free()
    return out


def repack_bench(stream):
    """Weight ingest: the config-5 gate|up matrix (13,824 x 2,560 trits) repacked
    into the 2-bit layout from int8 lanes and from base-4 codes (pk 12), 8
    rotated input copies each; algorithmic bytes = input + output words."""
    import nlgpu
    out, cols, pk, ncp = 2 * FFN_F, FFN_D, 12, 8
    t = nlgpu.trits(20260921 + 6, (out, cols)).astype(np.int64)
    ng, wng, fcount = (cols + 3) // 4, (cols + 15) // 16, (cols + pk - 1) // pk
    lanes = t.astype(np.int8).view(np.uint8).reshape(out, cols)
    wp = np.zeros((out, 4 * ng), np.uint8)
    wp[:, :cols] = lanes
    wp = wp.view("<u4").reshape(out, ng)
    codes = np.zeros((out, fcount * pk), np.int64)
    codes[:, :cols] = t + 1
    wpk = (codes.reshape(out, fcount, pk) * (4 ** np.arange(pk))).sum(axis=2).astype(np.float32)
    w2 = nlgpu.DeviceArray(out * wng * 4)
    res = {}
    for name, host, fn in (
            ("int8_lanes", wp, lambda src: nlgpu.repack_i8_to_2bit(src, out, cols, w2, stream=stream)),
            ("base4_pk12", wpk, lambda src: nlgpu.repack_packed_to_2bit(src, out, cols, pk, fcount, w2,
                                                                         stream=stream))):
        dsrc = nlgpu.DeviceArray(host.nbytes * ncp)
        for c in range(ncp):
            dsrc.upload(host, offset=c * host.nbytes)
        us = _per_launch_us(lambda i: fn(_Ptr(dsrc.ptr + (i % ncp) * host.nbytes, host.nbytes)), 4 * ncp, stream)
        nbytes = host.nbytes + out * wng * 4
        res[name] = {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        dsrc.free()
    w2.free()
    return res


def tlinear_bench(stream):
    """The transposed linear ternary-rows-t (input gradient X = W'(BETA*G)) at
    the down projection's shape, W [2560 x 6912] 2-bit, one position, 64
    rotated weight copies; bytes = weights + block scales + G + X."""
    import nlgpu
    out, cols, seq, ncp = FFN_D, FFN_F, 1, 64
    wng, nblk = (cols + 15) // 16, (cols + 127) // 128
    w = nlgpu.pack_ternary(nlgpu.trits(20260921 + 7, (out, cols)))
    dw = nlgpu.DeviceArray(w.nbytes * ncp)
    for c in range(ncp):
        dw.upload(w, offset=c * w.nbytes)
    beta = nlgpu.to_device(np.full(out * nblk, 0.05, np.float32))
    g = nlgpu.to_device(nlgpu.normal(20260921 + 8, seq * out))
    x = nlgpu.DeviceArray(seq * cols * 4)
    groups = (seq * cols + 63) // 64

    def fn(i):
        nlgpu.dispatch("ternary-rows-t", [(_Ptr(dw.ptr + (i % ncp) * w.nbytes, w.nbytes), out * wng),
                                          (beta, out * nblk), (g, seq * out), (x, seq * cols)],
                       [out, cols, nblk, wng, seq], groups, stream=stream)
    us = _per_launch_us(fn, 2 * ncp, stream)
    nbytes = w.nbytes + out * nblk * 4 + seq * (out + cols) * 4
    dw.free()
    return {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "shape": [out, cols, seq],
            "note": "each column summed over the 2560 rows in order (bit-identical to the reference's sum)"}


def paged_bench(stream):
    """PagedAttention over fp16 pools at the config-5 decode shape (20/5 heads
    x 128, every sequence at position 767, blocks of 16 positions in a random
    order), B = 1 and 32, 8 rotated pools; bytes = K and V of the attended
    positions + q + out (+ the block table)."""
    import nlgpu
    heads, kvh, hd, bs, mbps, ncp = 20, 5, 128, 16, 48, 8
    kvdim = kvh * hd
    res = {}
    for B in (1, 32):
        npool = B * mbps
        rng = np.random.default_rng(B)
        table = rng.permutation(npool).reshape(B, mbps).astype(np.int32)
        lens = np.full(B, bs * mbps - 1, np.int32)
        pool_bytes = npool * bs * kvdim * 2
        kp, vp = nlgpu.DeviceArray(pool_bytes * ncp), nlgpu.DeviceArray(pool_bytes * ncp)
        nlgpu.lib().nlg_fill_normal(C.c_void_p(kp.ptr), pool_bytes * ncp // 4, 1, C.c_float(1.0), 0, stream)
        nlgpu.lib().nlg_fill_normal(C.c_void_p(vp.ptr), pool_bytes * ncp // 4, 2, C.c_float(1.0), 0, stream)
        q = nlgpu.to_device(nlgpu.normal(3, B * heads * hd))
        out = nlgpu.DeviceArray(B * heads * hd * 4)
        ws = nlgpu.DeviceArray(nlgpu.decode_attn_paged_f16_workspace(B, heads, kvh, hd, bs, mbps))
        dl, dt = nlgpu.to_device(lens), nlgpu.to_device(table)

        def fn(i):
            c = i % ncp
            nlgpu.decode_attn_paged_f16(q, _Ptr(kp.ptr + c * pool_bytes, pool_bytes),
                                        _Ptr(vp.ptr + c * pool_bytes, pool_bytes), dl, dt, npool, out, B, heads,
                                        kvh, hd, bs, mbps, ws, stream=stream)
        us = _per_launch_us(fn, 4 * ncp, stream)
        nbytes = B * bs * mbps * kvdim * 2 * 2 + B * heads * hd * 8 + table.nbytes
        res[f"B{B}"] = {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
                        "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "launches": 2}
        kp.free(); vp.free()
    return res


def ring_bench(stream):
    """StreamingLLM decode attention over fp16 ring caches at the config-5
    decode shape (20/5 heads x 128), 4 sink slots + a 2044-slot window, every
    sequence wrapped (stream positions 10000 + b), B = 1 and 32, 8 rotated
    cache copies; bytes = K and V of the 2048 attended slots + q + out + the
    two rotation tables (2048 rows x 64 floats each)."""
    import nlgpu
    heads, kvh, hd, nsink, win, ncp = 20, 5, 128, 4, 2044, 8
    cap = nsink + win
    ang = np.outer(np.arange(cap), 1.0 / 500000.0 ** (np.arange(hd // 2) * 2.0 / hd))
    co, si = nlgpu.to_device(np.cos(ang).astype(np.float32)), nlgpu.to_device(np.sin(ang).astype(np.float32))
    res = {}
    for B in (1, 32):
        cache_bytes = B * kvh * cap * hd * 2
        kc, vc = nlgpu.DeviceArray(cache_bytes * ncp), nlgpu.DeviceArray(cache_bytes * ncp)
        nlgpu.lib().nlg_fill_normal(C.c_void_p(kc.ptr), cache_bytes * ncp // 4, 1, C.c_float(1.0), 0, stream)
        nlgpu.lib().nlg_fill_normal(C.c_void_p(vc.ptr), cache_bytes * ncp // 4, 2, C.c_float(1.0), 0, stream)
        q = nlgpu.to_device(nlgpu.normal(3, B * heads * hd))
        out = nlgpu.DeviceArray(B * heads * hd * 4)
        ws = nlgpu.DeviceArray(nlgpu.decode_attn_stream_f16_workspace(B, heads, kvh, hd, nsink, win))
        dpos = nlgpu.to_device(10000 + np.arange(B, dtype=np.int32))

        def fn(i):
            c = i % ncp
            nlgpu.decode_attn_stream_f16(q, _Ptr(kc.ptr + c * cache_bytes, cache_bytes),
                                         _Ptr(vc.ptr + c * cache_bytes, cache_bytes), dpos, co, si, out, B, heads,
                                         kvh, hd, nsink, win, ws, stream=stream)
        us = _per_launch_us(fn, 4 * ncp, stream)
        nbytes = 2 * cache_bytes + B * heads * hd * 8 + 2 * cap * (hd // 2) * 4
        res[f"B{B}"] = {"us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
                        "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "launches": 2}
        kc.free(); vc.free()
    return res


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _lavapipe_probe():
    """Whether the reference's own kernels could run through Vulkan on Mesa
    lavapipe here: that needs Emacs (the kernels are an Elisp DSL compiled to
    SPIR-V by Elisp), a Vulkan loader, the lavapipe ICD and the reference
    sources, which never reach the GPU box."""
    import ctypes.util
    import glob
    import shutil
    missing = []
    if not shutil.which("emacs"):
        missing.append("emacs")
    if not ctypes.util.find_library("vulkan"):
        missing.append("libvulkan")
    if not glob.glob("/usr/share/vulkan/icd.d/lvp_icd*.json") + glob.glob("/etc/vulkan/icd.d/lvp_icd*.json"):
        missing.append("lavapipe ICD (lvp_icd*.json)")
    missing.append("the reference sources (only this repository is on the GPU box)")
    return "not run: missing " + ", ".join(missing)


def _cpu_trits2(rng, out, cols):
    """Random 2-bit ternary rows for the CPU samples: field = 00 (p 1/2),
    01 or 11 (p 1/4 each), the trit distribution of the configs."""
    wng = (cols + 15) // 16
    lo = rng.integers(0, 1 << 32, (out, wng), dtype=np.uint64).astype(np.uint32) & np.uint32(0x55555555)
    r = rng.integers(0, 1 << 32, (out, wng), dtype=np.uint64).astype(np.uint32) & np.uint32(0x55555555)
    return lo | ((lo & r) << np.uint32(1))


def _time_loop(fn, seconds):
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return n, dt


def cpu_baseline(x, w_one, seconds: float):
    """The C restatement of the reference kernels (oracle/, OpenMP over
    invocations, -O2 -ffp-contract=off) on the host cores: config 2 for
    `seconds`, then bounded samples of configs 3, 4 and 5."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import nlg_oracle as orc

    beta = np.array([1.0], np.float32)

    def step():
        xq, g = orc.pack_act_rows(x, 1, COLS)
        orc.ternary_linear_i8(xq, g, w_one, None, beta, 1, OUT, COLS)

    n, dt = _time_loop(step, seconds)
    res = dict(value=round(STEP_BYTES * n / dt / 1e9, 3), unit="GB/s", cores=orc.threads(), kind="port",
               sample=f"{n} steps of the 4096x4096 config-2 step (pack-act-rows + ternary GEMV, C "
                      f"restatement of the reference kernels, OpenMP over output rows) in {dt:.1f} s",
               cpu_model=_cpu_model(), threads=orc.threads(), lavapipe=_lavapipe_probe())
    rng = np.random.default_rng(20260921)
    part = max(1.0, seconds / 3)
    other = {}
    # config 3: softmax rows of one causal 4096-wide head tile (rows 2048..2559)
    rows = 512
    a = (rng.standard_normal((rows, SM_N)) * 3.0).astype(np.float32)
    a[np.arange(SM_N)[None, :] > (2048 + np.arange(rows))[:, None]] = -np.inf
    n, dt = _time_loop(lambda: orc.softmax_rows(a, rows, SM_N), part)
    other["softmax_config3"] = {"gbs": round(2 * 4 * rows * SM_N * n / dt / 1e9, 3),
                                "sample": f"{n} x {rows} causal rows of 4096 in {dt:.1f} s (bytes = read + write)"}
    # config 4: the SwiGLU FFN at B = 1 (gate|up linear, silu-mul, down linear)
    wgu, wd = _cpu_trits2(rng, 2 * FFN_F, FFN_D), _cpu_trits2(rng, FFN_D, FFN_F)
    xf = rng.standard_normal(FFN_D).astype(np.float32)
    bgu = np.full(2 * FFN_F, 1.0 / np.sqrt(FFN_D / 2), np.float32)
    bdn = np.array([1.0 / np.sqrt(FFN_F / 2)], np.float32)

    def ffn():
        xq, g = orc.pack_act_rows(xf, 1, FFN_D)
        gu = orc.ternary_linear_i8(xq, g, wgu, None, bgu, 1, 2 * FFN_F, FFN_D, beta_per_row=True)
        h = np.zeros(FFN_F, np.float32)
        orc.dispatch("silu-mul", [np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]), h], [FFN_F],
                     (FFN_F + 63) // 64)
        hq, hg = orc.pack_act_rows(h, 1, FFN_F)
        orc.ternary_linear_i8(hq, hg, wd, None, bdn, 1, FFN_D, FFN_F)

    n, dt = _time_loop(ffn, part)
    ffn_bytes = wgu.nbytes + wd.nbytes + 2 * FFN_D * 4
    other["swiglu_ffn_config4_B1"] = {"us": round(dt / n * 1e6, 1), "gbs": round(ffn_bytes * n / dt / 1e9, 3),
                                      "sample": f"{n} FFNs at one token in {dt:.1f} s"}
    # config 5 at B = 1: one decoder layer at position 640 (the mean attended
    # length), extrapolated to 30 layers, plus the LM head timed on a slice
    c = STACK
    d, f, hd = c["d_model"], c["d_ff"], c["head_dim"]
    nq, nkv, ms = c["heads"] * hd, c["kv_heads"] * hd, PROMPT + DECODE
    wqkv, wo = _cpu_trits2(rng, nq + 2 * nkv, d), _cpu_trits2(rng, d, nq)
    bq = np.full(nq + 2 * nkv, 1.0 / np.sqrt(d / 2), np.float32)
    bo = np.array([1.0 / np.sqrt(nq / 2)], np.float32)
    gain = np.ones(d, np.float32)
    kc = rng.standard_normal(c["kv_heads"] * ms * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(c["kv_heads"] * ms * hd).astype(np.float16).view(np.uint16)
    xs = rng.standard_normal(d).astype(np.float32)
    ang = np.outer(np.arange(ms), 1.0 / c.get("rope_theta", 500000.0) ** (np.arange(hd // 2) * 2.0 / hd))
    co, si = np.cos(ang).astype(np.float32).ravel(), np.sin(ang).astype(np.float32).ravel()
    pos = 640

    def lin(v, w, b, out, cols, per_row=False):
        vq, vg = orc.pack_act_rows(np.ascontiguousarray(v, np.float32), 1, cols)
        return orc.ternary_linear_i8(vq, vg, w, None, b, 1, out, cols, beta_per_row=per_row)

    def rope(v, cols, heads):
        o = np.zeros(cols, np.float32)
        orc.dispatch("decode-rope-b", [np.ascontiguousarray(v, np.float32), co, si, np.array([1.0], np.float32),
                                       np.array([float(pos)], np.float32), o], [1, cols, heads], (cols // 2 + 63) // 64)
        return o

    def layer():
        xn = orc.rmsnorm_rows(xs, gain, 1e-5, 1, d)
        qkv = lin(xn, wqkv, bq, nq + 2 * nkv, d, True)
        q = rope(qkv[:nq], nq, c["heads"])
        rope(qkv[nq:nq + nkv], nkv, c["kv_heads"])
        att = orc.decode_attn_f16(q, kc, vc, pos, 1, c["heads"], c["kv_heads"], hd, ms)
        x1 = (xs + lin(att, wo, bo, d, nq)).astype(np.float32)
        xn = orc.rmsnorm_rows(x1, gain, 1e-5, 1, d)
        gu = lin(xn, wgu, bgu, 2 * f, d, True)
        h = np.zeros(f, np.float32)
        orc.dispatch("silu-mul", [np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]), h], [f],
                     (f + 63) // 64)
        return (x1 + lin(h, wd, bdn, d, f)).astype(np.float32)

    n, dt = _time_loop(layer, part)
    t_layer = dt / n
    head_rows = 16384
    wlm = _cpu_trits2(rng, head_rows, d)
    nh, dth = _time_loop(lambda: lin(xs, wlm, bo, head_rows, d), 0.5)
    t_head = dth / nh * c["vocab"] / head_rows
    t_tok = c["layers"] * t_layer + t_head
    other["decode_config5_B1"] = {"tok_s": round(1.0 / t_tok, 3), "ms_per_token": round(t_tok * 1e3, 1),
                                  "sample": f"{n} decoder layers at position {pos} in {dt:.1f} s (x30), plus the "
                                            f"LM head timed on {head_rows} of its {c['vocab']} rows "
                                            f"({nh} passes, scaled by rows)"}
    res["other_configs"] = other
    return res


def pmc_probe():
    """Eager launches for rocprofv3 --pmc and --kernel-trace runs, in this
    order: 64 config-2 steps (rotating weight copies), 4 launches of the
    same GEMV kernel over all 128 copies stacked (long dispatches that
    calibrate GRBM_GUI_ACTIVE's clock), 4 device-to-device copies of 64 MiB
    (calibrating FETCH_SIZE / WRITE_SIZE), then the five decoder-layer
    kernels at batch 1 and at batch 32 (30 launches each, one per layer, at
    cache position 767) and one full-size config-3 softmax."""
    import nlgpu
    nlgpu.init()
    seed = 20260921 + 1
    w_one = nlgpu.pack_ternary(nlgpu.trits(seed, (OUT, COLS)))
    wbytes = w_one.nbytes
    dW = nlgpu.DeviceArray(wbytes * COPIES)
    for c in range(COPIES):
        dW.upload(np.roll(w_one, c, axis=0), offset=c * wbytes)
    dx = nlgpu.to_device(nlgpu.normal(seed + 100, COLS))
    dbeta = nlgpu.to_device(np.array([1.0], np.float32))
    dy = nlgpu.DeviceArray(OUT * 4)
    L = nlgpu.lib()
    for i in range(64):
        L.nlg_ternary_linear_cfg(dx.ptr, dW.ptr + (i % COPIES) * wbytes, None, dbeta.ptr, 0, dy.ptr, None, 1,
                                 OUT, COLS, 0, None, 0, None)
    nlgpu.sync()
    dxq, dg, dY = nlgpu.DeviceArray(COLS), nlgpu.DeviceArray(4), nlgpu.DeviceArray(OUT * COPIES * 4)
    L.nlg_pack_act_rows(dx.ptr, dxq.ptr, dg.ptr, 1, COLS, None)
    for _ in range(4):
        L.nlg_ternary_linear_i8_cfg(dxq.ptr, dg.ptr, dW.ptr, None, dbeta.ptr, 0, dY.ptr, 1, OUT * COPIES, COLS, 4, 4,
                                    None)
    nlgpu.sync()
    a, b = nlgpu.DeviceArray(64 << 20), nlgpu.DeviceArray(64 << 20)
    for _ in range(4):
        L.nlg_copy_d2d(b.ptr, a.ptr, 64 << 20, None)
    nlgpu.sync()
    print("pmc probe: 64 config-2 steps, 4 stacked GEMVs, 4 copies of 64 MiB", flush=True)
    del dW, dY, a, b
    stream = L.nlg_default_stream()
    for batch in (1, 32):
        st = nlgpu.Stack(**STACK, max_seq=PROMPT + DECODE, batch=batch, seed=20260921 + 5)
        kern, nl = _decode_kernels(st, batch, stream)
        for name, (fn, _) in kern.items():
            for i in range(nl):
                fn(i)
            nlgpu.sync()
        st.close()
        print(f"pmc probe: decoder-layer kernels at batch {batch}, {nl} launches each", flush=True)
    n = SM_HEADS * SM_N * SM_N
    sm = nlgpu.DeviceArray(n * 4)
    nlgpu.fill_normal(sm, n, 20260921 + 3, 3.0, SM_N)
    nlgpu.softmax_rows(sm, sm, SM_HEADS * SM_N, SM_N)
    nlgpu.sync()
    print("pmc probe: one config-3 softmax", flush=True)


def profile_eager(stack=True):
    """Launch, without graphs (rocprofv3's kernel trace follows eager launches
    only), what the rocprof summaries cover: the config-5 decoder stack at
    batch 1 and 32 (512-row prefill, then 16 decode steps; left out when
    `stack` is false) and the config-4 FFN at 512 and 16384 tokens (10 passes
    each).  Prints one line per phase."""
    import nlgpu
    nlgpu.init()
    c = STACK
    for batch in ((1, 32) if stack else ()):
        s = nlgpu.Stack(**c, max_seq=PROMPT + DECODE, batch=batch, seed=20260921 + 5)
        ids = (nlgpu.uniform(20260921 + 55, batch * PROMPT) * c["vocab"]).astype(np.int32).reshape(batch, PROMPT)
        s.prefill(ids)
        s.step(16, graph=False)
        nlgpu.sync()
        s.close()
        print(f"profile: stack batch {batch}: prefill {PROMPT} rows + 16 eager decode steps", flush=True)
    seed = 20260921 + 4
    gu = np.empty((2 * FFN_F, FFN_D // 16), np.uint32)
    gu[0::2] = nlgpu.pack_ternary(nlgpu.trits(seed, (FFN_F, FFN_D)))
    gu[1::2] = nlgpu.pack_ternary(nlgpu.trits(seed + 1, (FFN_F, FFN_D)))
    dgu, dwd = nlgpu.to_device(gu), nlgpu.to_device(nlgpu.pack_ternary(nlgpu.trits(seed + 2, (FFN_D, FFN_F))))
    bgu = nlgpu.to_device(np.full(2 * FFN_F, 1.0 / np.sqrt(FFN_D / 2), np.float32))
    bd = nlgpu.to_device(np.array([1.0 / np.sqrt(FFN_F / 2)], np.float32))
    nlgpu.ternary_tiled_register(dgu, 2 * FFN_F, FFN_D)
    nlgpu.ternary_tiled_register(dwd, FFN_D, FFN_F)
    for B in (512, 16384):
        x = nlgpu.to_device(nlgpu.normal(seed + 10 + B, B * FFN_D))
        h, y = nlgpu.DeviceArray(B * FFN_F * 4), nlgpu.DeviceArray(B * FFN_D * 4)
        for _ in range(10):
            nlgpu.rms_ternary_swiglu(x, None, 0.0, dgu, bgu, h, B, FFN_F, FFN_D)
            nlgpu.ternary_linear(h, dwd, None, bd, y, B, FFN_D, FFN_F)
        nlgpu.sync()
        print(f"profile: FFN {FFN_D}x{FFN_F} at {B} tokens, 10 passes", flush=True)
        del x, h, y
    nlgpu.ternary_tiled_unregister(dgu)
    nlgpu.ternary_tiled_unregister(dwd)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decoder stack")
    ap.add_argument("--pmc-probe", action="store_true", help="only the launches the PMC profiles count")
    ap.add_argument("--profile-eager", action="store_true",
                    help="only the eager stack and FFN launches the rocprof kernel summaries cover")
    ap.add_argument("--profile-ffn", action="store_true",
                    help="only the eager FFN launches (the MFMA counter summary)")
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.profile_eager or args.profile_ffn:
        profile_eager(stack=not args.profile_ffn)
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the decode path is not sharded); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    r = gpu_bench(args.steps, args.warmup, args.sweep)
    decode = {}
    if not args.no_decode:
        import nlgpu
        stream = nlgpu.lib().nlg_default_stream()
        for b in (1, 32):
            decode[f"batch{b}"] = decode_bench(b, stream)
    extra = {}
    if not args.no_decode:
        import nlgpu
        stream = nlgpu.lib().nlg_default_stream()
        extra["matmul_config1"] = matmul_bench(stream)
        extra["softmax_config3"] = softmax_bench(stream)
        extra["swiglu_ffn_config4"] = ffn_bench(stream)
        extra["weight_ingest_repack"] = repack_bench(stream)
        extra["transposed_linear"] = tlinear_bench(stream)
        extra["paged_attention_f16"] = paged_bench(stream)
        extra["ring_attention_f16"] = ring_bench(stream)
    value = STEP_BYTES / (r["step_ms"] * 1e-3) / 1e9
    gemv_gbs = GEMV_BYTES / (r["gemv_ms"] * 1e-3) / 1e9
    stacked_gbs = GEMV_BYTES * COPIES / (r["stacked_ms"] * 1e-3) / 1e9
    ceiling_us = r["floor_ms"] * 1e3 + STEP_BYTES / (stacked_gbs * 1e3)
    traffic, tfac = step_traffic()
    cpu = cpu_baseline(r["x"], r["w_one"], args.cpu_seconds)
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["step_stats"]["launches"],
        "steps_requested": args.steps,
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
                   "step": "one launch: pack-act-rows quantisation fused into the ternary GEMV"},
        "timing": dict(r["step_stats"], how="HIP events around each replay of a 128-launch graph on the "
                                             "kernel's stream; value uses the mean over every launch"),
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "copy_peak_gbs": round(r["copy_gbs"], 1),
                     "frac_of_copy_peak": round(value / r["copy_gbs"], 4),
                     "traffic_source": ("profiles/ternary_gemv_4096_decode_pmc_traffic.md (FETCH_SIZE x "
                                        f"{tfac} + WRITE_SIZE, calibrated on a 64 MiB copy)") if traffic else
                                       "profile absent",
                     "kernel": "k_tern_fused", "bytes_per_launch": STEP_BYTES,
                     "us_per_launch": round(r["step_ms"] * 1e3, 3),
                     # what one dependent launch can reach on this part: the
                     # empty-launch floor plus the bytes at the kernel's own
                     # streaming rate (the 128-matrix launch)
                     "ceiling_us": round(ceiling_us, 3),
                     "frac_of_ceiling": round(ceiling_us / (r["step_ms"] * 1e3), 4)},
        "device_timing": {"kernel_us": round(float(np.mean(r["device_us"])), 3),
                          "kernel_us_p10_p90": [round(float(np.percentile(r["device_us"], q)), 3) for q in (10, 90)],
                          "gap_to_next_us": round(float(np.mean(r["gap_us"])), 3),
                          "kernel_plus_gap_us": round(float(np.mean(r["device_us"][:-1] + r["gap_us"])), 3),
                          "event_us_per_launch": round(r["timed_ms"] * 1e3, 3),
                          "how": "nlg_ternary_linear_timed: the same step with every wave's start and end read "
                                 "from the 100 MHz wall clock (s_memrealtime) in a replayed 128-launch graph; "
                                 "kernel = first wave's start to last wave's end of a launch, gap = idle time "
                                 "to the next launch's first wave; no profiler attached"},
        "gemv_prequantised": {"gbs": round(gemv_gbs, 2), "us_per_launch": round(r["gemv_ms"] * 1e3, 3),
                              "bytes_per_launch": GEMV_BYTES, "kernel": "k_tern_i8_dec"},
        "gemv_stacked_one_launch": {"gbs": round(stacked_gbs, 2), "frac": round(stacked_gbs / HBM_PEAK_GBS, 4),
                                    "rows": OUT * COPIES, "ms": round(r["stacked_ms"], 4)},
        "launch_floor_us": round(r["floor_ms"] * 1e3, 3),
        "cpu_baseline": cpu,
        "device": r["device"],
    }
    if decode:
        out["decode"] = dict(decode, model="30-layer ternary decoder, d 2560, 20/5 heads x 128, d_ff 6912, "
                                           "vocab 128256 (ternary LM head), fp16 KV, random-init seeded weights, "
                                           "prompt 512 random ids then 256 greedy tokens")
    out.update(extra)
    if "sweep_us" in r:
        out["sweep_us"] = r["sweep_us"]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
