#!/usr/bin/env python3
"""Benchmark of the NVFP4 matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]
                    [--calibrate]

A step is one launch of the hot-path kernel over one batch of synthetic input with
every operand already resident in HBM.  The headline workload is the decode fused
GeGLU at batch 1: x bf16 [1,5376], gate/up NVFP4 [21504 x 5376], out bf16 [1,21504].
The weights are rotated over several copies (> 256 MB MALL) so every step streams
them from HBM.  Steps are timed with HIP events recorded on the launch stream.

Prints one JSON line: value = algorithmic bytes per step / average step time (GB/s).
The roofline object prices the same kernel against MI355X's 8 TB/s HBM peak, and its
"read_ceiling" times the fastest plain streaming read of the same bytes (rotated the
same way) for the rate any kernel moving them reaches on this GPU; the
cpu_baseline object times the reference's own CPU implementation of the op
(src/tests/cpu_ref.h matvecNvfp4Cpu + geluTanh, compiled from its sources), single-
threaded like the reference: the headline workload, and under "configs" every
workload of the path in its GPU record's unit (the two prefill workloads on stated
slices, extrapolated).

The "secondary" object carries the metric's second half and the other workloads of
the path, each timed the same way (HIP events around back-to-back steps; at least 10
launches and 20 ms of GPU time per record, the count in its "steps", after at least
60 ms of untimed warmup launches: the clocks ramp under sustained MFMA load):
  moe_prefill   MoE layer prefill: 4096 tokens, hidden 2816, 128 experts, top-8,
                intermediate 704, Zipf(1.1) routing -> TFLOP/s vs the 2.5 PFLOP/s
                dense bf16 MFMA peak (flops of the routed pairs only);
  gemm_prefill  dense prefill GEMM bf16 [2048,5376] x NVFP4 [21504x5376]^T -> TFLOP/s;
  geglu_prefill / matmul_prefill_f32  the same weight shape through the fused GeGLU
                (bf16 x) and the fp32 matmul (fp32 x, bf16 hi + lo split) -> TFLOP/s;
  dense_mlp_prefill_f32  the Gemma dense MLP block (hidden 2816, intermediate 2112) at
                512 tokens, fp32, RMSNorm folded in -> TFLOP/s;
  moe_decode    MoE decode: 16 tokens, same experts -> GB/s of the distinct experts'
                weights + activations (expert slots rotated over copies > MALL).
--calibrate runs, before the timed steps, one streaming read of 1 GiB and one 256 MiB
device copy, the known-size kernels the HBM counters (FETCH_SIZE / WRITE_SIZE) of a
rocprofv3 --pmc pass are scaled by.
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

from apex_amd import hip, synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def geglu_workload(rows=21504, K=5376, seed=0):
    x, gate, up = synth.geglu_case(seed=seed, rows=rows, K=K)
    w_bytes = 2 * (gate.codes.nbytes + gate.scales.nbytes)
    algo_bytes = w_bytes + x.nbytes + rows * 2
    flops = 2 * 2 * rows * K
    return x, gate, up, algo_bytes, flops


def touch_weights(sets, stream):
    """Read every weight copy once with the plain streaming-read probe, so that the
    operands are resident and mapped before any launch is timed: the first kernel to
    read a fresh allocation pays its page-table walks (measured: the launch that first
    met the sixth copy took ~30 us against ~22 us).  A decode loop reads the same
    weights every step, so its steady state has them mapped."""
    sink = hip.DeviceArray((hip.read_probe_sink_words(),), np.uint32)
    for s in sets:
        for arr in s:
            hip.read_probe(arr, sink, stream)
    stream.synchronize()


def time_geglu(steps: int, warmup: int, rows=21504, K=5376):
    x, gate, up, algo_bytes, flops = geglu_workload(rows, K)
    w_bytes = algo_bytes - x.nbytes - rows * 2
    copies = max(4, int(np.ceil(2.5 * MALL_BYTES / w_bytes)))
    dx = hip.DeviceArray.from_numpy(x)
    base = [hip.DeviceArray.from_numpy(a) for a in (gate.codes, gate.scales, up.codes, up.scales)]
    sets = [base]
    for _ in range(copies - 1):
        s = [hip.DeviceArray(a.shape, a.dtype) for a in base]
        for d, b in zip(s, base):
            d.copy_from(b)
        sets.append(s)
    out = hip.DeviceArray((1, rows), np.uint16)
    stream = hip.Stream()
    touch_weights(sets, stream)

    def step(i):
        gc, gs, uc, us = sets[i % copies]
        hip.nvfp4_geglu_bf16(dx, gc, gs, uc, us, out, 1, rows, K, stream=stream)

    for i in range(warmup):
        step(i)
    stream.synchronize()
    hip.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    e1.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    per_step_s = ms / 1e3 / steps
    stream.close()
    return {
        "algo_bytes": algo_bytes, "flops": flops, "per_step_s": per_step_s, "wall_s": wall,
        "copies": copies, "rows": rows, "K": K,
    }


def time_read_ceiling(nbytes: int, copies: int, steps: int, warmup: int):
    """The fastest plain streaming read of `nbytes` (the library's read probe, rotated
    over `copies` buffers like the headline's weights, so the MALL serves none of it):
    the rate a kernel moving these bytes can reach on this GPU, beside the spec peak."""
    bufs = [hip.DeviceArray((nbytes,), np.uint8) for _ in range(copies)]
    for b in bufs:
        b.fill_bytes(1)
    sink = hip.DeviceArray((hip.read_probe_sink_words(),), np.uint32)
    stream = hip.Stream()

    def step(i):
        hip.read_probe(bufs[i % copies], sink, stream=stream)

    sec, n = time_steps(step, steps, warmup, stream)
    stream.close()
    for b in bufs + [sink]:
        b.close()
    return {"value": round(nbytes / sec / 1e9, 2), "unit": "GB/s", "us_per_read": round(sec * 1e6, 3),
            "steps": n, "bytes": int(nbytes), "copies_rotated": copies}


# ---- CPU baseline: the reference's own CPU code on every workload ------------------

def _cpu_ops():
    """(kind, matvec, geglu, moe_ffn): the reference's matvecNvfp4Cpu / geluTanh compiled
    from its sources (src/tests/cpu_ref.h) where available ("reference"), else the
    oracle's restatement of the same arithmetic ("port").  Single-threaded, as the
    reference is (src/tests/cpu_ref.h:50-63)."""
    import oracle  # the oracle / reference CPU code is the checker and the baseline only

    if oracle.ref_available():
        return ("reference", oracle.ref_matvec,
                lambda g, u, x: oracle.ref_geglu(g, u, x),
                lambda slots, x, ids, w, E: oracle.ref_moe_ffn(slots, x, ids, w, E))
    return ("port", lambda c, s, x: oracle.matvec(c, s, x),
            lambda g, u, x: oracle.geglu(oracle.matvec(*g, x), oracle.matvec(*u, x)),
            lambda slots, x, ids, w, E: oracle.moe_ffn(slots, x, ids, w))


def _repeat(fn, budget_s):
    """Run fn() until budget_s has elapsed (at least once): (seconds per call, calls)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            return dt / n, n


def cpu_baselines(budget_s: float = 4.0):
    """The reference's CPU implementation timed on every workload of the path, on this
    host, one core, in the unit of the workload's GPU record.  Configurations 0-2 run
    whole; 3 (dense prefill GEMM) runs a slice of weight rows for all 2048 tokens and
    4 (MoE prefill) two slices of tokens: both products are linear in those rows /
    tokens, so the full-size time is extrapolated (for 4 along the line through the two
    slices, which keeps the per-expert row decodes a slice pays once out of the slope)."""
    import oracle
    kind, mv, geglu, moe = _cpu_ops()
    nproc = os.cpu_count()
    out = {}

    def rec(value, unit, sample):
        return {"value": value, "unit": unit, "cores": 1, "kind": kind,
                "sample": f"{sample}; single-threaded, host nproc={nproc}"}

    # GEMV 2048 x 2048, bf16 x (widened exactly), batch 1
    x, w = synth.gemv_case(seed=0)
    xf = synth.bf16_to_f32(x)
    algo = w.codes.nbytes + w.scales.nbytes + x.nbytes + w.rows * 2
    sec, n = _repeat(lambda: mv(w.codes, w.scales, xf), budget_s / 4)
    out["gemv_2048"] = rec(round(algo / sec / 1e9, 4), "GB/s",
                           f"whole workload: matvecNvfp4Cpu 2048x2048, batch 1, {n} calls, "
                           f"{sec * 1e3:.2f} ms each")

    # decode fused GeGLU 2 x [21504 x 5376], batch 1 (the headline workload)
    x, gate, up, algo, _ = geglu_workload()
    xf = synth.bf16_to_f32(x)
    sec, n = _repeat(lambda: geglu((gate.codes, gate.scales), (up.codes, up.scales), xf), budget_s)
    out["geglu_decode"] = rec(round(algo / sec / 1e9, 4), "GB/s",
                              f"whole workload: gate and up matvecNvfp4Cpu [21504x5376] + "
                              f"geluTanh(gate) * up, batch 1, {n} calls, {sec:.2f} s each")

    # MoE decode, 16 tokens
    x, logits, slots = _case("moe_decode")
    T, H, E, I = x.shape[0], x.shape[1], logits.shape[1], slots.I
    ids, wts = oracle.moe_route(synth.bf16_to_f32(logits), 8)
    U = len(np.unique(ids))
    algo = U * 3 * (I * H // 2 + I * H // 16) + x.nbytes + logits.nbytes + T * H * 2
    xf = synth.bf16_to_f32(x)
    sec, n = _repeat(lambda: moe(slots, xf, ids, wts, E), budget_s / 2)
    out["moe_decode"] = rec(round(algo / sec / 1e9, 4), "GB/s",
                            f"whole workload: 16 tokens x top-8 over {U} experts, per expert "
                            f"gate/up/down matvecNvfp4Cpu + geluTanh, weighted sum; {n} calls, "
                            f"{sec:.2f} s each")

    # prefill GEMM 2048 x 21504 x 5376 on a slice of W's rows
    A, w = _case("gemm")
    Af = synth.bf16_to_f32(A)
    M, N, K = A.shape[0], w.rows, w.K
    t = time.perf_counter()
    mv(w.codes[:4], w.scales[:4], Af)
    per_row = (time.perf_counter() - t) / 4
    rows = int(min(N, max(8, budget_s / per_row)))
    t = time.perf_counter()
    mv(w.codes[:rows], w.scales[:rows], Af)
    dt = time.perf_counter() - t
    full = dt * N / rows
    out["gemm_prefill"] = rec(round(2.0 * M * N * K / full / 1e12, 6), "TFLOP/s",
                              f"slice: rows 0..{rows - 1} of {N} x all {M} tokens "
                              f"(K={K}) in {dt:.2f} s, extrapolated x{N / rows:.1f} to "
                              f"{full:.0f} s for the whole GEMM")

    # MoE prefill, 4096 tokens, on two slices of tokens
    x, logits, slots = _case("moe_prefill")
    T, H, E, I = x.shape[0], x.shape[1], logits.shape[1], slots.I
    ids, wts = oracle.moe_route(synth.bf16_to_f32(logits), 8)
    xf = synth.bf16_to_f32(x)

    def slice_time(nt):
        t = time.perf_counter()
        moe(slots, xf[:nt], ids[:nt], wts[:nt], E)
        return time.perf_counter() - t

    t4 = slice_time(4)
    n1 = int(max(8, min(T // 4, budget_s / 4 / max(t4 / 4, 1e-6))))
    n2 = 3 * n1
    t1, t2 = slice_time(n1), slice_time(n2)
    slope = (t2 - t1) / (n2 - n1)
    full = t1 + slope * (T - n1)
    flops = 2.0 * T * 8 * 3 * H * I
    out["moe_prefill"] = rec(round(flops / full / 1e12, 6), "TFLOP/s",
                             f"slices: tokens 0..{n1 - 1} in {t1:.2f} s and 0..{n2 - 1} "
                             f"in {t2:.2f} s (experts grouped, gate/up/down matvecNvfp4Cpu + "
                             f"geluTanh), the line through both extrapolated to all {T} tokens: "
                             f"{full:.0f} s")
    return out


# ---- GPU timing -----------------------------------------------------------------------

# every secondary record times at least this many launches and this much GPU time, after
# at least this much GPU time of untimed warmup launches of the same step: the clocks
# ramp under sustained MFMA load (the dense prefill GEMM runs 476 -> 417 -> 400 -> 390 us
# over its first 60 launches, ~27 ms, and holds there), so a record timed right after a
# cold start would measure the ramp, not the kernel
MIN_TIMED_STEPS = 10
MIN_TIMED_MS = 20.0
MIN_WARMUP_MS = 60.0


def time_steps(step, steps, warmup, stream, min_steps=MIN_TIMED_STEPS, min_ms=MIN_TIMED_MS,
               min_warmup_ms=MIN_WARMUP_MS):
    """Seconds per step of `step(i)` launched back to back on `stream`, and the number of
    steps timed: max(warmup, 1) untimed steps -- more until min_warmup_ms of GPU time has
    run -- then max(steps, min_steps) timed steps, more if needed to cover min_ms."""
    warmup = max(1, warmup)
    stream.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(warmup):
        step(i)
    e1.record(stream)
    e1.synchronize()
    warm_ms = e0.elapsed_ms(e1)
    est_ms = warm_ms / warmup
    if est_ms > 0 and warm_ms < min_warmup_ms:
        more = int(np.ceil((min_warmup_ms - warm_ms) / est_ms))
        e0.record(stream)
        for i in range(more):
            step(warmup + i)
        e1.record(stream)
        e1.synchronize()
        est_ms = e0.elapsed_ms(e1) / more
    n = max(steps, min_steps)
    if est_ms > 0:
        n = max(n, int(np.ceil(min_ms / est_ms)))
    hip.synchronize()
    e0.record(stream)
    for i in range(n):
        step(i)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) / 1e3 / n, n


_CASE_CACHE = {}


def _case(name):
    """Seeded synthetic workloads shared by the GPU records and the CPU baselines."""
    if name not in _CASE_CACHE:
        _CASE_CACHE[name] = {"moe_decode": lambda: synth.moe_decode_case(seed=0),
                             "moe_prefill": lambda: synth.moe_prefill_case(seed=0),
                             "gemm": lambda: synth.gemm_case(seed=0)}[name]()
    return _CASE_CACHE[name]


def moe_setup(case, copies):
    x, logits, slots = case
    T, H = x.shape
    E = logits.shape[1]
    dx, dl = hip.DeviceArray.from_numpy(x), hip.DeviceArray.from_numpy(logits)
    base = hip.DeviceArray.from_numpy(slots.data)
    sl = [base]
    for _ in range(copies - 1):
        c = hip.DeviceArray(base.shape, base.dtype)
        c.copy_from(base)
        sl.append(c)
    y = hip.DeviceArray((T, H), np.uint16)
    ws = hip.DeviceArray((hip.moe_workspace_bytes(T, E, 8, H, slots.I),), np.uint8)
    ms = [hip.moe_slots(b, slots.stride, slots.offsets) for b in sl]
    return dx, dl, sl, ms, y, ws


def time_moe_decode(steps, warmup):
    case = _case("moe_decode")
    x, logits, slots = case
    T, H, E, I = x.shape[0], x.shape[1], logits.shape[1], slots.I
    # distinct experts the step streams: from the library's own router
    ids = hip.DeviceArray((T, 8), np.int32)
    wts = hip.DeviceArray((T, 8), np.float32)
    hip.moe_route_bf16(hip.DeviceArray.from_numpy(logits), ids, wts, T, E, 8)
    hip.synchronize()
    U = len(np.unique(ids.numpy()))
    piece_bytes = 3 * (I * H // 2 + I * H // 16)
    algo = U * piece_bytes + x.nbytes + logits.nbytes + T * H * 2
    copies = max(2, int(np.ceil(2.5 * MALL_BYTES / (U * piece_bytes))))
    dx, dl, sl, ms, y, ws = moe_setup(case, copies)
    stream = hip.Stream()

    def step(i):
        hip.moe_ffn_bf16(dx, dl, ms[i % copies], y, T, E, 8, H, I, ws, stream=stream)

    sec, nsteps = time_steps(step, steps, warmup, stream)
    stream.close()
    gbs = algo / sec / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": int(algo),
            "distinct_experts": int(U), "slot_copies_rotated": copies,
            "workload": "MoE decode: x bf16 [16,2816], logits bf16 [16,128], top-8, 128 "
                        "experts NVFP4 gate/up [704x2816], down [2816x704], y bf16 [16,2816]",
            "path": "grouped GEMV gate/up with routing and planning in every workgroup and "
                    "GeGLU, grouped GEMV down by token groups, fixed-order combine (3 launches)"}


def time_moe_prefill(steps, warmup):
    case = _case("moe_prefill")
    x, logits, slots = case
    T, H, E, I = x.shape[0], x.shape[1], logits.shape[1], slots.I
    flops = 2.0 * T * 8 * 3 * H * I
    dx, dl, sl, ms, y, ws = moe_setup(case, 1)
    stream = hip.Stream()

    def step(i):
        hip.moe_ffn_bf16(dx, dl, ms[0], y, T, E, 8, H, I, ws, stream=stream)

    sec, nsteps = time_steps(step, steps, warmup, stream)
    stream.close()
    tf = flops / sec / 1e12
    return {"value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
            "roofline_frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops": int(flops),
            "workload": "MoE prefill: x bf16 [4096,2816], Zipf(1.1) routing over 128 experts "
                        "(8 empty), top-8, NVFP4 gate/up [704x2816], down [2816x704], y bf16",
            "path": "route + per-block expert masks, column scan of the block counts, "
                    "placing (plan + positions), grouped MFMA GEMM gate/up with GeGLU "
                    "epilogue, grouped MFMA GEMM down, weighted combine (6 launches)"}


def time_gemm_prefill(steps, warmup, M=2048, N=21504, K=5376):
    A, w = _case("gemm") if (M, N, K) == (2048, 21504, 5376) else \
        synth.gemm_case(seed=0, M=M, N=N, K=K)
    dA = hip.DeviceArray.from_numpy(A)
    dc, ds = hip.DeviceArray.from_numpy(w.codes), hip.DeviceArray.from_numpy(w.scales)
    C = hip.DeviceArray((M, N), np.uint16)
    stream = hip.Stream()

    def step(i):
        hip.nvfp4_gemm_bf16(dA, dc, ds, C, M, N, K, stream=stream)

    sec, nsteps = time_steps(step, steps, warmup, stream)
    stream.close()
    for a in (dA, dc, ds, C):
        a.close()
    tf = 2.0 * M * N * K / sec / 1e12
    return {"value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
            "roofline_frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops": int(2 * M * N * K),
            "workload": f"prefill GEMM: A bf16 [{M},{K}] x NVFP4 W [{N}x{K}]^T -> C bf16 [{M},{N}]",
            "yardstick_vendor_bf16_gemm_tflops": vendor_bf16_gemm(M, N, K, max(steps, 60),
                                                                  max(warmup, 160))}


def time_dense_prefill(steps, warmup, T=2048, N=21504, K=5376):
    """Prefill through the reference-named dense ops at the headline weight shape:
    the fused GeGLU with bf16 activations (gate and up in one MFMA GEMM) and the fp32
    matmul (the reference's fp32 contract: x split into bf16 hi + lo, twice the MFMA
    work).  TFLOP/s count the useful products only, 2 T N K per matrix."""
    rng = np.random.default_rng(0)
    g, u = synth.nvfp4_weights(rng, N, K), synth.nvfp4_weights(rng, N, K)
    dw = [hip.DeviceArray.from_numpy(a) for a in (g.codes, g.scales, u.codes, u.scales)]
    xb = hip.DeviceArray.from_numpy(synth.normal_bf16(rng, (T, K)))
    xf = hip.DeviceArray.from_numpy(rng.standard_normal((T, K)).astype(np.float32))
    hb, yf = hip.DeviceArray((T, N), np.uint16), hip.DeviceArray((T, N), np.float32)
    stream = hip.Stream()
    out = {}
    for name, flops, fn, text in [
        ("geglu_prefill", 4.0 * T * N * K,
         lambda i: hip.nvfp4_geglu_bf16(xb, *dw, hb, T, N, K, stream=stream),
         f"prefill fused GeGLU: x bf16 [{T},{K}], gate/up NVFP4 [{N}x{K}] -> bf16 [{T},{N}]"),
        ("matmul_prefill_f32", 2.0 * T * N * K,
         lambda i: hip.nvfp4_matmul_f32(xf, dw[0], dw[1], yf, T, N, K, stream=stream),
         f"prefill matmul, fp32 contract: x fp32 [{T},{K}] x NVFP4 [{N}x{K}]^T -> fp32 "
         f"[{T},{N}] (bf16 hi + lo split, 2x MFMA work)")]:
        sec, nsteps = time_steps(fn, steps, warmup, stream)
        tf = flops / sec / 1e12
        out[name] = {"value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
                     "roofline_frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops": int(flops),
                     "workload": text}
    stream.close()
    for a in dw + [xb, xf, hb, yf]:
        a.close()
    out["dense_mlp_prefill_f32"] = time_dense_mlp_prefill(steps, warmup)
    return out


def time_dense_mlp_prefill(steps, warmup, T=512, H=2816, I=2112):
    """The Gemma dense MLP block at prefill, fp32 (the reference contract): RMSNorm
    folded into the fused GeGLU GEMM's split pass, then the down GEMM (split-K: this
    shape has few tiles).  FLOPs 2 T (2 I H + H I)."""
    h, nw, g, u, d = synth.dense_mlp_case(seed=0, tokens=T, H=H, I=I)
    arrs = [hip.DeviceArray.from_numpy(a) for a in (h, nw, g.codes, g.scales, u.codes, u.scales,
                                                    d.codes, d.scales)]
    dh, dnw, gc, gs, uc, us, dc, ds = arrs
    hh, y = hip.DeviceArray((T, I), np.float32), hip.DeviceArray((T, H), np.float32)
    stream = hip.Stream()

    def step(i):
        hip.nvfp4_geglu_rms_norm_f32(dh, dnw, 1e-6, gc, gs, uc, us, hh, T, I, H, stream=stream)
        hip.nvfp4_matmul_f32(hh, dc, ds, y, T, H, I, stream=stream)

    sec, nsteps = time_steps(step, steps, warmup, stream)
    stream.close()
    for a in arrs + [hh, y]:
        a.close()
    flops = 2.0 * T * (2 * I * H + H * I)
    tf = flops / sec / 1e12
    return {"value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
            "roofline_frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops": int(flops),
            "workload": f"dense MLP prefill, fp32: {T} tokens, RMSNorm [{H}] fused into GeGLU "
                        f"NVFP4 [{I}x{H}] x2, down NVFP4 [{H}x{I}] (GEMMs: split pass, split-K)"}


def time_norms(steps, warmup, T=4096, H=2816, heads=16, D=256):
    """The two normalisation kernels at prefill size: RMSNorm of x fp32 [4096, 2816]
    and per-head RMSNorm + RoPE of q fp32 [4096, 16, 256] (128 rotated pairs).  Both
    read and write their activations once: algorithmic bytes = 2 x activations +
    weights."""
    rng = np.random.default_rng(0)
    out = {}
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = synth.bf16_from_f32((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    dx, dw, dy = (hip.DeviceArray.from_numpy(x), hip.DeviceArray.from_numpy(w),
                  hip.DeviceArray((T, H), np.float32))
    stream = hip.Stream()
    sec, nsteps = time_steps(lambda i: hip.rms_norm_f32(dx, dw, dy, T, H, 1e-6, stream=stream), steps,
                     warmup, stream)
    algo = 2 * x.nbytes + w.nbytes
    out["rms_norm"] = {"value": round(algo / sec / 1e9, 2), "unit": "GB/s",
                       "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
                       "roofline_frac": round(algo / sec / 1e9 / HBM_PEAK_GBS, 4),
                       "algorithmic_bytes": int(algo),
                       "workload": f"rms_norm_f32: x fp32 [{T},{H}], bf16 weights [{H}]"}
    q = rng.standard_normal((T, heads, D)).astype(np.float32)
    hw = synth.bf16_from_f32((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    dq, dhw, do = (hip.DeviceArray.from_numpy(q), hip.DeviceArray.from_numpy(hw),
                   hip.DeviceArray(q.shape, np.float32))
    sec, nsteps = time_steps(lambda i: hip.head_norm_rope_f32(dq, dhw, do, T, heads, D, D // 2, 10000.0,
                                                      0, heads * D, D, 1e-6, stream=stream),
                     steps, warmup, stream)
    algo = 2 * q.nbytes + hw.nbytes
    out["head_norm_rope"] = {"value": round(algo / sec / 1e9, 2), "unit": "GB/s",
                             "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
                             "roofline_frac": round(algo / sec / 1e9 / HBM_PEAK_GBS, 4),
                             "algorithmic_bytes": int(algo),
                             "workload": f"head_norm_rope_f32: q fp32 [{T},{heads},{D}], "
                                         f"{D // 2} rotated pairs"}
    stream.close()
    for a in (dx, dw, dy, dq, dhw, do):
        a.close()
    return out


def time_dense_mlp_decode(steps, warmup, H=2816, I=2112):
    """The Gemma dense MLP block at batch 1 (fp32 activations, the reference contract):
    gate/up GeGLU GEMV with the RMSNorm fused in -> down GEMV, 2 launches per token,
    weights rotated over enough copies to exceed the MALL.  Algorithmic bytes per token:
    the three NVFP4 matrices plus the activations each kernel reads and writes."""
    h, nw, g, u, d = synth.dense_mlp_case(seed=0, tokens=1, H=H, I=I)
    mats = (g.codes, g.scales, u.codes, u.scales, d.codes, d.scales)
    w_bytes = sum(a.nbytes for a in mats)
    act = (H * 4 + H * 2 + I * 4) + (I * 4 + H * 4)
    algo = w_bytes + act
    copies = max(4, int(np.ceil(2.5 * MALL_BYTES / w_bytes)))
    base = [hip.DeviceArray.from_numpy(a) for a in mats]
    sets = [base]
    for _ in range(copies - 1):
        s = [hip.DeviceArray(a.shape, a.dtype) for a in base]
        for dd, b in zip(s, base):
            dd.copy_from(b)
        sets.append(s)
    dh, dnw = hip.DeviceArray.from_numpy(h), hip.DeviceArray.from_numpy(nw)
    hh, y = hip.DeviceArray((1, I), np.float32), hip.DeviceArray((1, H), np.float32)
    stream = hip.Stream()

    def step(i):
        gc, gs, uc, us, dc, ds = sets[i % copies]
        hip.nvfp4_geglu_rms_norm_f32(dh, dnw, 1e-6, gc, gs, uc, us, hh, 1, I, H, stream=stream)
        hip.nvfp4_matmul_f32(hh, dc, ds, y, 1, H, I, stream=stream)

    sec, nsteps = time_steps(step, steps, warmup, stream)
    stream.close()
    for arrs in sets:
        for a in arrs:
            a.close()
    for a in (dh, dnw, hh, y):
        a.close()
    gbs = algo / sec / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": int(algo),
            "weight_copies_rotated": copies,
            "workload": f"dense MLP decode, batch 1, fp32: RMSNorm [1,{H}] fused into GeGLU "
                        f"NVFP4 [{I}x{H}] x2 -> down NVFP4 [{H}x{I}] (2 launches)"}


def time_router(steps, warmup, E=128, H=2816):
    """Gemma-4 router logits (RMSNorm with router.scale + affine 8-bit projection, fp32)
    at the decode (16 tokens) and prefill (4096 tokens) sizes; FLOPs = 2 T E H."""
    out = {}
    for T, name in ((16, "router_decode"), (4096, "router_prefill")):
        h, rw = synth.router_case(seed=0, tokens=T, E=E, H=H)
        arrs = [hip.DeviceArray.from_numpy(a) for a in (h, rw.norm_w, rw.qw, rw.qs, rw.qb)]
        lg = hip.DeviceArray((T, E), np.float32)
        stream = hip.Stream()
        sec, nsteps = time_steps(lambda i: hip.moe_router_logits_q8(*arrs, lg, T, E, H, 1e-6,
                                                            stream=stream), steps, warmup, stream)
        stream.close()
        for a in arrs + [lg]:
            a.close()
        out[name] = {"value": round(2.0 * T * E * H / sec / 1e12, 3), "unit": "TFLOP/s",
                     "ms_per_step": round(sec * 1e3, 6), "steps": nsteps,
                     "workload": f"router logits: h fp32 [{T},{H}], affine q8 [{E}x{H}] "
                                 f"(group 64), fp32 out [{T},{E}]"}
    return out


def time_slot_streaming(repeats=3):
    """One expert layer file (128 slots at the Gemma-4 stride, 430 MB) streamed into HBM
    with apex_file_to_device (pread into pinned staging, copies overlapped).  The file
    was just written, so it is read from the page cache: this is the host-memory ->
    HBM leg of a load, not the disk."""
    import tempfile
    _, stride, _ = synth.slot_layout(2816, 704)
    size = 128 * stride
    fd, path = tempfile.mkstemp(suffix=".bin")
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(np.random.default_rng(0).integers(0, 256, size, dtype=np.uint8).tobytes())
        dst = hip.DeviceArray((size,), np.uint8)
        times = []
        for _ in range(repeats):
            hip.synchronize()
            t0 = time.perf_counter()
            hip.file_to_device(path, 0, size, dst)
            times.append(time.perf_counter() - t0)
        dst.close()
    finally:
        os.unlink(path)
    sec = float(np.median(times))
    return {"value": round(size / sec / 1e9, 2), "unit": "GB/s", "ms_per_step": round(sec * 1e3, 3),
            "bytes": size, "workload": "expert layer file (128 slots x 3,358,720 B) -> HBM, "
                                       "page-cache source, 8 MiB x 8 pinned staging, 4 reader threads"}


def vendor_bf16_gemm(M, N, K, steps, warmup):
    """Context for the GEMM line: the vendor library's plain bf16 GEMM of the same shape
    (torch -> hipBLASLt, weights already bf16, no FP4 decode).  Not part of the path."""
    try:
        import torch
        if not torch.cuda.is_available():
            return None
        a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        w = torch.randn(N, K, device="cuda", dtype=torch.bfloat16)
        for _ in range(warmup):
            torch.nn.functional.linear(a, w)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            torch.nn.functional.linear(a, w)
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) / 1e3 / steps
        del a, w
        torch.cuda.empty_cache()
        return round(2.0 * M * N * K / sec / 1e12, 2)
    except Exception:  # torch absent or without a GPU: no yardstick
        return None


def calibrate():
    """Known-size kernels for scaling rocprofv3 HBM counters: a 1 GiB streaming read
    and a 256 MiB device-to-device copy."""
    big = hip.DeviceArray((1 << 30,), np.uint8)
    big.fill_bytes(1)
    sink = hip.DeviceArray((hip.read_probe_sink_words(),), np.uint32)
    hip.read_probe(big, sink)
    src = hip.DeviceArray((256 << 20,), np.uint8)
    dst = hip.DeviceArray((256 << 20,), np.uint8)
    src.fill_bytes(2)
    dst.copy_from(src)
    hip.synchronize()
    for a in (big, sink, src, dst):
        a.close()


def load_traffic(kernel: str):
    try:
        return json.loads(TRAFFIC_FILE.read_text()).get(kernel)
    except (OSError, ValueError):
        return None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=4.0,
                    help="seconds of CPU time per baseline configuration (about)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="time only the headline fused-GeGLU workload")
    ap.add_argument("--calibrate", action="store_true",
                    help="run the known-size read and copy kernels first (counter scaling)")
    ap.add_argument("--only", choices=["moe_prefill", "gemm_prefill", "moe_decode", "norms",
                                       "dense_mlp_decode", "router", "slot_streaming",
                                       "dense_prefill"],
                    help="profiling aid: time one secondary workload and print its record only")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: there is no multi-GPU path to time; run with "
              "--gpus 1", file=sys.stderr)
        return 2

    if args.calibrate:
        calibrate()
    if args.only:
        fn = {"moe_prefill": time_moe_prefill, "gemm_prefill": time_gemm_prefill,
              "moe_decode": time_moe_decode, "norms": time_norms,
              "dense_mlp_decode": time_dense_mlp_decode, "router": time_router,
              "slot_streaming": lambda steps, warmup: time_slot_streaming(),
              "dense_prefill": time_dense_prefill}[args.only]
        print(json.dumps({args.only: fn(args.steps, args.warmup)}), flush=True)
        return 0
    r = time_geglu(args.steps, args.warmup)
    gbs = r["algo_bytes"] / r["per_step_s"] / 1e9
    line = {
        "metric": "NVFP4 GEMV weight GB/s (% of HBM peak) + MoE prefill GEMM TFLOP/s (% MFMA)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["per_step_s"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "nvfp4 weights (e2m1 x e4m3), bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded: x ~ N(0,1) bf16, uniform E2M1 codes, E4M3 scales |N(0,1)|*0.05)",
        "config": {
            "workload": "decode fused GeGLU, batch 1: x bf16 [1,5376], gate/up NVFP4 "
                        "[21504x5376], out bf16 [1,21504]",
            "kernel": "apex_nvfp4_geglu_bf16 (nvfp4_gemv_kernel, GeGLU epilogue)",
            "algorithmic_bytes_per_step": r["algo_bytes"],
            "weight_copies_rotated": r["copies"],
            "launch": "back-to-back launches on one stream, HIP events around the timed steps",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic("geglu_decode"),
        },
    }
    # the fastest plain read of the same bytes: how far the kernel is from what any
    # kernel streaming them reaches here
    ceil = time_read_ceiling(r["algo_bytes"], r["copies"], args.steps, args.warmup)
    line["roofline"]["read_ceiling"] = {**ceil, "frac_of_ceiling": round(gbs / ceil["value"], 4)}
    if not args.no_secondary:
        # each record: at least MIN_TIMED_STEPS launches and MIN_TIMED_MS of GPU time
        sec_steps, sec_warm = max(1, args.steps // 100), max(2, args.warmup // 100)
        dec_steps, dec_warm = max(1, args.steps // 10), max(2, args.warmup // 10)
        line["secondary"] = {
            "moe_prefill": time_moe_prefill(sec_steps, sec_warm),
            "gemm_prefill": time_gemm_prefill(sec_steps, sec_warm),
            **time_dense_prefill(sec_steps, sec_warm),
            "moe_decode": time_moe_decode(dec_steps, dec_warm),
        }
        line["secondary"].update(time_norms(dec_steps, dec_warm))
        line["secondary"]["dense_mlp_decode"] = time_dense_mlp_decode(dec_steps, dec_warm)
        line["secondary"].update(time_router(sec_steps, sec_warm))
        line["secondary"]["slot_streaming"] = time_slot_streaming()
    if not args.no_cpu:
        cpu = cpu_baselines(args.cpu_budget)
        # the headline workload's line first, then every configuration's
        line["cpu_baseline"] = {**cpu["geglu_decode"], "configs": cpu}
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
