"""Shared helpers for the parity tests."""
from __future__ import annotations

import numpy as np

from apex_amd import synth

# parity tolerances (rel L2, src/tests/cpu_ref.h:27-46 metric) against the fp64 oracle
TOL_F32 = 1e-3
TOL_BF16 = 1e-2
# the reference's own parity gate for fp32 outputs (src/tests/dense_mlp.cpp:113)
TOL_REF_GATE = 1e-5


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(b))
    den = np.sqrt(np.sum(b * b))
    num = np.sqrt(np.sum((a - b) ** 2))
    return num / den if den > 0 else num


def bf16(a):
    return synth.bf16_to_f32(a)


def all_codes_weights(rows_per_code: int = 1):
    """16 rows (code c in every nibble of row c) x 256 blocks (scale byte b in block b):
    every (E2M1 code, E4M3 scale) pair appears."""
    K = 256 * 16
    rows = 16 * rows_per_code
    codes = np.zeros((rows, K // 8), np.uint32)
    for r in range(rows):
        c = r % 16
        nib = np.uint32(c)
        word = np.uint32(0)
        for i in range(8):
            word |= nib << np.uint32(4 * i)
        codes[r, :] = word
    scales = np.tile(np.arange(256, dtype=np.uint8), (rows, 1))
    return synth.Nvfp4Weights(codes, scales)
