"""Write the golden vectors under tests/golden/ from the reference's own CPU code.

    make -C oracle ref              # builds oracle/_ref/libapexref.so from the reference
    python tests/golden/make_golden.py

The reference's NVFP4 decode and fp64 matvec (src/nvfp4.h:10-43,
src/tests/cpu_ref.h:48-68) are compiled in place from its sources into
oracle/_ref/libapexref.so; this script calls that library on the seeded synthetic
inputs of apex_amd.synth and stores inputs' SHA-256 digests and outputs as small
fixtures.  Only outputs and digests are stored (no reference source text).

Fixtures:
  nvfp4_tables.npz   e2m1[16], e4m3[256] decoded by the reference (fp32)
  gelu.npz           x[513], geluTanh(x) by the reference (fp32)
  matvec_tiny.npz    per case: codes, scales, x (fp32) and the reference's output,
                     for rows 1-64, K 16-256, tokens 1-3, covering all 16 codes
  matvec_2048.npz    the reference's output for the 2048x2048 single GEMV (x = bf16
                     N(0,1), seed 0), 2048 fp32
  rms_norm.npz       per case: x (fp32 [rows, n]), w (bf16 bits [n]), eps and the
                     reference's rmsNormCpu output (src/tests/cpu_ref.h:10-22)
  digests.json       SHA-256 of the synthetic inputs the fixtures were made from
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from apex_amd import synth  # noqa: E402

TINY = [(1, 16, 1), (3, 32, 2), (8, 48, 1), (16, 64, 3), (5, 128, 1), (64, 256, 2),
        (2, 16, 3), (33, 96, 1)]


RMS_CASES = [(1, 16, 1e-6), (3, 100, 1e-5), (2, 2816, 1e-6), (1, 5376, 0.0)]


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tiny_case(i: int, rows: int, K: int, T: int):
    rng = np.random.default_rng(1000 + i)
    w = synth.nvfp4_weights(rng, rows, K)
    x = synth.bf16_to_f32(synth.normal_bf16(rng, (T, K)))
    return w, x


def main() -> None:
    R = oracle.ref()
    e2m1 = np.array([R.ref_e2m1_to_float(c) for c in range(16)], np.float32)
    e4m3 = np.array([R.ref_e4m3_to_float(b) for b in range(256)], np.float32)
    np.savez(HERE / "nvfp4_tables.npz", e2m1=e2m1, e4m3=e4m3)

    gx = np.concatenate([np.linspace(-8, 8, 509, dtype=np.float32),
                         np.array([0.0, -0.0, 1.0, 1e-3], np.float32)])
    gy = np.array([R.ref_gelu_tanh(float(v)) for v in gx], np.float32)
    np.savez(HERE / "gelu.npz", x=gx, y=gy)

    tiny = {}
    digests = {}
    for i, (rows, K, T) in enumerate(TINY):
        w, x = tiny_case(i, rows, K, T)
        y = oracle.ref_matvec(w.codes, w.scales, x)
        tiny[f"c{i}_codes"] = w.codes
        tiny[f"c{i}_scales"] = w.scales
        tiny[f"c{i}_x"] = x
        tiny[f"c{i}_y"] = y
    np.savez(HERE / "matvec_tiny.npz", **tiny)

    x, w = synth.gemv_case(seed=0)
    xf = synth.bf16_to_f32(x)
    y = oracle.ref_matvec(w.codes, w.scales, xf)
    np.savez(HERE / "matvec_2048.npz", y=y)
    digests["gemv_case_seed0"] = sha(w.codes, w.scales, x)

    xg, gate, up = synth.geglu_case(seed=0, rows=64, K=512)
    digests["geglu_case_seed0_64x512"] = sha(xg, gate.codes, gate.scales, up.codes, up.scales)
    a, wg = synth.gemm_case(seed=0, M=16, N=32, K=128)
    digests["gemm_case_seed0_16x32x128"] = sha(wg.codes, wg.scales, a)
    xm, lm, slots = synth.moe_decode_case(seed=0, tokens=2, H=64, I=32, E=4)
    digests["moe_decode_case_seed0_tiny"] = sha(xm, lm, slots.data)
    xp, lp, slotsp = synth.moe_prefill_case(seed=0, tokens=8, H=64, I=32, E=16)
    digests["moe_prefill_case_seed0_tiny"] = sha(xp, lp, slotsp.data)
    norm = {}
    for i, (rows, n, eps) in enumerate(RMS_CASES):
        rng = np.random.default_rng(2000 + i)
        xn = rng.standard_normal((rows, n)).astype(np.float32) * np.float32(1 + i)
        wn = synth.bf16_from_f32((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
        norm[f"c{i}_x"], norm[f"c{i}_w"] = xn, wn
        norm[f"c{i}_eps"] = np.float32(eps)
        norm[f"c{i}_y"] = oracle.ref_rms_norm(xn, wn, eps)
    np.savez(HERE / "rms_norm.npz", **norm)
    (HERE / "digests.json").write_text(json.dumps(digests, indent=1, sort_keys=True) + "\n")
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")), "and digests.json")


if __name__ == "__main__":
    main()
