"""The reference-named registry kernel matmul_nvfp4 queued through the Backend exactly
as src/ops.h:34-46 queues it (Dim3{ceil(w_rows / 8), tokens} x 256 threads, fp32 in
and out), at decode and prefill token counts.  A grid that covers every row runs the
same product as apex_nvfp4_matmul_f32 -- an MFMA GEMM from prefill sizes on, seen in
the library's launch counts -- and a grid covering fewer rows writes only those rows,
strided by w_rows (shaders/matmul.metal:14-18).  Tolerance: the reference harness's
gate, rel L2 < 1e-5 (src/tests/dense_mlp.cpp:113)."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import TOL_REF_GATE, rel_l2

pytestmark = pytest.mark.gpu


def queue_matmul(be, x, w, tokens, row_groups):
    """matmulNvfp4 of src/ops.h:34-46 (weights and scales in one buffer, as core.bin
    places them); returns the fp32 output [tokens, w.rows]."""
    cb = w.codes.nbytes
    bx = be.allocate(x.nbytes, "activations")
    bw = be.allocate(cb + w.scales.nbytes, "core_weights")
    by = be.allocate(tokens * w.rows * 4, "activations")
    be.contents(bx, np.float32, x.size)[:] = x.ravel()
    core = be.contents(bw, np.uint8, cb + w.scales.nbytes)
    core[:cb] = w.codes.view(np.uint8).ravel()
    core[cb:] = w.scales.ravel()
    be.run("matmul_nvfp4", [hip.buf(bx), hip.buf(bw), hip.buf(bw, cb), hip.buf(by),
                            hip.u32(w.K), hip.u32(w.rows)], (row_groups, tokens), (256,))
    be.sync()
    y = be.contents(by, np.float32, tokens * w.rows).reshape(tokens, w.rows).copy()
    for b in (bx, bw, by):
        be.release(b)
    return y


@pytest.mark.parametrize("tokens,expect_gemm", [(1, False), (4, False), (128, True), (300, True)])
def test_matmul_nvfp4_reference_launch(tokens, expect_gemm):
    rng = np.random.default_rng(70 + tokens)
    rows, K = 1536, 1024
    w = synth.nvfp4_weights(rng, rows, K)
    x = rng.standard_normal((tokens, K)).astype(np.float32)
    be = hip.Backend(0)
    try:
        before = hip.dense_dispatch_counts()
        y = queue_matmul(be, x, w, tokens, (rows + 7) // 8)
        after = hip.dense_dispatch_counts()
    finally:
        be.close()
    gemms = (after["gemm"] + after["splitk_gemm"]) - (before["gemm"] + before["splitk_gemm"])
    gemvs = after["gemv"] - before["gemv"]
    assert (gemms, gemvs) == ((1, 0) if expect_gemm else (0, 1))
    assert rel_l2(y, oracle.matvec(w.codes, w.scales, x)) < TOL_REF_GATE


def test_matmul_nvfp4_partial_grid_writes_covered_rows_only():
    """A grid of 100 groups of 256 threads covers 800 of 1536 rows: those rows are
    computed (GEMV), the rest of each output row keeps its zero fill."""
    rng = np.random.default_rng(77)
    rows, K, tokens = 1536, 1024, 128
    w = synth.nvfp4_weights(rng, rows, K)
    x = rng.standard_normal((tokens, K)).astype(np.float32)
    be = hip.Backend(0)
    try:
        y = queue_matmul(be, x, w, tokens, 100)
    finally:
        be.close()
    covered = 100 * 256 // 32
    want = oracle.matvec(w.codes[:covered], w.scales[:covered], x)
    assert rel_l2(y[:, :covered], want) < TOL_REF_GATE
    assert not np.any(y[:, covered:])
