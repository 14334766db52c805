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


def count_outside(got, want, rel: float, abs_frac: float) -> int:
    """Elements of `got` farther from `want` than rel * |want| + abs_frac * rms(want): a
    wrong, missing or misplaced tile, row or column shows up however few elements it
    touches, which a norm over the whole output can hide."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape and np.all(np.isfinite(got))
    rms = np.sqrt(np.mean(want * want))
    return int(np.count_nonzero(np.abs(got - want) > rel * np.abs(want) + abs_frac * rms))


# Per-element bound of a bf16 output: round to nearest even moves a value by at most
# half a bf16 step, 2^-8 of its magnitude, so an output computed in fp32 and rounded once
# lies within 2^-8 |want| of the fp32/fp64 oracle value plus the fp32 accumulation error.
BF16_REL = 2.0 ** -8


def outside_bf16(got, want, abs_frac: float = 1e-5) -> int:
    """count_outside with the bf16 rounding bound: a single zeroed, doubled or misplaced
    output whose magnitude is above abs_frac of the rms is counted.  1e-5 of the rms
    covers the fp32 accumulation of the GEMVs (a few fp32 steps of a dot product) and
    the fp32 cancellation in the oracle's 1 + tanh for strongly negative gates."""
    max_excess(got, want)
    return count_outside(got, want, BF16_REL, abs_frac)


def max_excess(got, want) -> float:
    """Largest |got - want| beyond 2^-8 |want|, in units of rms(want), printed so a run's
    log shows how much of a bound's absolute term was used."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want * want))
    ex = float(np.max(np.abs(got - want) - BF16_REL * np.abs(want)) / rms) if rms > 0 else 0.0
    print(f"max excess over 2^-8|want|: {ex:.3g} of the rms", flush=True)
    return ex


def moe_outside(got, want_r, terms, abs_frac: float = 1e-2) -> int:
    """Elements of a MoE FFN output farther from the composition with bf16-rounded
    intermediates (`want_r`, from moe_ffn_full(..., bf16_intermediates=True,
    with_abs=True)) than one bf16 step of the output and of every term,
    2^-8 (|y| + sum_j |w_j d_j|), plus abs_frac of the output rms.  The abs_frac term
    covers intermediates that round the other way after a different fp32 summation
    order (one bf16 step of an h element moves y by far less than 1e-2 of the rms)."""
    got = np.asarray(got, np.float64)
    want_r = np.asarray(want_r, np.float64)
    assert got.shape == want_r.shape and np.all(np.isfinite(got))
    rms = np.sqrt(np.mean(want_r * want_r))
    slack = np.abs(got - want_r) - (BF16_REL * (np.abs(want_r) + terms) + abs_frac * rms)
    print(f"moe: max excess over one bf16 step of output and terms: {slack.max() / rms + abs_frac:.3g}"
          " of the rms", flush=True)
    return int(np.count_nonzero(slack > 0))


def dequant_f64(codes, scales) -> np.ndarray:
    """The oracle's exact dequantisation (fp32, every value exact), as fp64 for a numpy
    contraction."""
    import oracle
    return oracle.decode(codes, scales).astype(np.float64)


def moe_ffn_full(slots, x, ids, weights, bf16_intermediates: bool = False, with_abs: bool = False):
    """The MoE FFN of every token, grouped by expert: per expert the oracle's exact
    dequantisation of gate, up and down, fp64 numpy products, the oracle's GeGLU on the
    fp32-rounded projections; y[t] = sum_j w[t,j] * down(h[t, expert j]).  The same
    composition as oracle.moe_ffn (pinned against it in the oracle tests), fast enough for
    4096 tokens.  bf16_intermediates: h and each pair's down projection d rounded to
    bf16 (nearest even), as the grouped-GEMM path stores them between its kernels.
    with_abs: also return sum_j |w[t,j] * d[t,j]| per element (the scale of one bf16
    rounding step of the terms)."""
    import oracle
    x = np.asarray(x, np.float64)
    T, k = ids.shape
    y = np.zeros((T, slots.H), np.float64)
    yabs = np.zeros((T, slots.H), np.float64) if with_abs else None
    for e in np.unique(ids):
        t_idx, j_idx = np.nonzero(ids == e)
        g = dequant_f64(slots.piece(e, "gate_w"), slots.piece(e, "gate_s"))
        u = dequant_f64(slots.piece(e, "up_w"), slots.piece(e, "up_s"))
        d = dequant_f64(slots.piece(e, "down_w"), slots.piece(e, "down_s"))
        xe = x[t_idx]
        h = oracle.geglu((xe @ g.T).astype(np.float32), (xe @ u.T).astype(np.float32))
        if bf16_intermediates:
            h = synth.bf16_to_f32(synth.bf16_from_f32(h))
        de = h.astype(np.float64) @ d.T
        if bf16_intermediates:
            de = synth.bf16_to_f32(synth.bf16_from_f32(de.astype(np.float32))).astype(np.float64)
        term = weights[t_idx, j_idx][:, None].astype(np.float64) * de
        y[t_idx] += term
        if with_abs:
            yabs[t_idx] += np.abs(term)
    return (y, yabs) if with_abs else y
