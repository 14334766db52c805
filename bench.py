#!/usr/bin/env python3
"""Benchmark of the NVFP4 matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--extra]

A step is one launch of the hot-path kernel over one batch of synthetic input with
every operand already resident in HBM.  The headline workload is the decode fused
GeGLU at batch 1: x bf16 [1,5376], gate/up NVFP4 [21504 x 5376], out bf16 [1,21504].
The weights are rotated over several copies (> 256 MB MALL) so every step streams
them from HBM.  Steps are timed with HIP events recorded on the launch stream.

Prints one JSON line: value = algorithmic bytes per step / average step time (GB/s).
The roofline object prices the same kernel against MI355X's 8 TB/s HBM peak; the
cpu_baseline object times the reference's own CPU implementation of the op
(src/tests/cpu_ref.h matvecNvfp4Cpu + geluTanh, compiled from its sources) on a
bounded sample, single-threaded like the reference.
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


def cpu_baseline_geglu(budget_s: float = 10.0, rows=21504, K=5376):
    """The reference's CPU op on the same workload: gate and up matvecNvfp4Cpu
    (fp64 accumulation, single thread) and geluTanh, over a row sample sized to the
    time budget; throughput in the same unit (algorithmic GB/s)."""
    import oracle  # the oracle / reference CPU code is the checker and the baseline only

    x, gate, up, algo_bytes, _ = geglu_workload(rows, K)
    xf = synth.bf16_to_f32(x)
    kind = "reference" if oracle.ref_available() else "port"
    mv = oracle.ref_matvec if kind == "reference" else (lambda c, s, v: oracle.matvec(c, s, v))
    gelu = oracle.ref().ref_gelu_tanh if kind == "reference" else oracle.gelu
    # calibrate on 256 rows, then run a sample sized to the budget
    t = time.perf_counter()
    mv(gate.codes[:256], gate.scales[:256], xf)
    per_row = (time.perf_counter() - t) / 256
    n = int(min(rows, max(256, budget_s / (2 * per_row))))
    t = time.perf_counter()
    g = mv(gate.codes[:n], gate.scales[:n], xf)
    u = mv(up.codes[:n], up.scales[:n], xf)
    h = np.array([gelu(float(a)) for a in g.ravel()], np.float32) * u.ravel()
    dt = time.perf_counter() - t
    bytes_per_row = (algo_bytes - xf.size * 2 - rows * 2) / rows
    sample_bytes = n * bytes_per_row + x.nbytes + n * 2
    return {
        "value": round(sample_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": f"decode GeGLU, gate+up rows 0..{n - 1} of {rows} (K={K}), batch 1, "
                  f"{dt:.1f} s single-threaded, host nproc={os.cpu_count()}",
        "_h": h,
    }


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
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(sharding is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        return 2

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
    if not args.no_cpu:
        cb = cpu_baseline_geglu(args.cpu_budget)
        cb.pop("_h")
        line["cpu_baseline"] = cb
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
