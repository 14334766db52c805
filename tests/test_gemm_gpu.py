"""GPU parity of the prefill NVFP4 GEMM (bf16 MFMA on exactly dequantised weights)
against the CPU oracle (fp64 restatement of src/tests/cpu_ref.h matvecNvfp4Cpu)."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import (TOL_BF16, TOL_REF_GATE, bf16, count_outside, dequant_f64, outside_bf16,
                           rel_l2)

pytestmark = pytest.mark.gpu


def dev(a):
    return hip.DeviceArray.from_numpy(a)


def gemm(A, w, tensor_scale=1.0):
    M, K = A.shape
    C = hip.DeviceArray((M, w.rows), np.uint16)
    hip.nvfp4_gemm_bf16(dev(A), dev(w.codes), dev(w.scales), C, M, w.rows, K, tensor_scale)
    hip.synchronize()
    return C.numpy()


@pytest.mark.parametrize("M,N,K", [(256, 448, 512), (300, 512, 256), (37, 224, 64)])
def test_gemm_one_hot_rows_select_weights_exactly(M, N, K):
    """A row m is the one-hot vector e_{p(m)}: C[m, n] = W[n, p(m)] exactly, so the
    output equals the reference dequantisation bit for bit (layout, dequant, tiling)."""
    rng = np.random.default_rng(M + N + K)
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), perm] = 1.0
    got = bf16(gemm(synth.bf16_from_f32(A), w))
    # a sum that starts from +0 turns the -0.0 of code 8 into +0, as the reference's
    # fp64 matvec does (src/tests/cpu_ref.h:57-59): compare with -0 normalised to +0
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got, oracle.matvec(w.codes, w.scales, A))


def test_gemm_one_hot_every_scale_byte():
    """All 256 E4M3 scale bytes -- zero, the subnormals, both signs, 0x7F / 0xFF = +-480 --
    each in 32 blocks, through the MFMA GEMM's exact bf16 dequantisation: one-hot rows pick
    single weights, bit for bit the reference decoder's values (negative scales flip the
    code's sign; +-480 x 6 = +-2880 is exact in bf16)."""
    rng = np.random.default_rng(31)
    N, K, M = 256, 512, 300
    w = synth.nvfp4_weights(rng, N, K)
    w.scales[:] = (np.arange(N * K // 16) * 37 % 256).astype(np.uint8).reshape(N, K // 16)
    perm = rng.integers(0, K, size=M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), perm] = 1.0
    got = bf16(gemm(synth.bf16_from_f32(A), w))
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and a dense product over every byte value against the fp64 contraction
    A2 = synth.normal_bf16(rng, (M, K))
    got2 = bf16(gemm(A2, w))
    want2 = bf16(A2).astype(np.float64) @ dequant_f64(w.codes, w.scales).T
    assert outside_bf16(got2, want2, 2e-3) == 0


@pytest.mark.parametrize("M,N,K", [(64, 224, 704), (300, 448, 2816), (513, 256, 1024),
                                   (130, 1408, 2816)])
def test_gemm_random(M, N, K):
    rng = np.random.default_rng(7 * M + N + K)
    w = synth.nvfp4_weights(rng, N, K)
    A = synth.normal_bf16(rng, (M, K))
    got = bf16(gemm(A, w))
    want = oracle.matvec(w.codes, w.scales, bf16(A))
    assert rel_l2(got, want) < TOL_BF16
    # every element: half a bf16 step plus 2e-3 of the rms (MFMA fp32 accumulation)
    assert outside_bf16(got, want, 2e-3) == 0


def test_gemm_prefill_full_size():
    """Prefill dense GEMM: A [2048,5376] x W [21504x5376], seed 0 (256 x 256 tiles over
    2.625 rounds of the CUs).  Every element against an fp64 contraction of the oracle's
    exact dequantisation: within 2^-8 of its value (bf16 output rounding) plus 2e-3 of the
    output rms (fp32 accumulation); and 48 sampled rows x 1024 sampled columns against the
    oracle's own fp64 matvec."""
    A, w = synth.gemm_case(seed=0)
    M, K = A.shape
    C = bf16(gemm(A, w))
    Af = bf16(A)
    want = Af.astype(np.float64) @ dequant_f64(w.codes, w.scales).T
    assert count_outside(C, want, 2.0 ** -8, 2e-3) == 0
    assert rel_l2(C, want) < TOL_BF16
    rng = np.random.default_rng(1)
    mi = np.sort(rng.choice(M, 48, replace=False))
    ni = np.sort(rng.choice(w.rows, 1024, replace=False))
    assert rel_l2(C[np.ix_(mi, ni)], oracle.matvec_rows(w.codes, w.scales, Af[mi], ni)) < TOL_BF16


def test_geglu_prefill_full_size():
    """Prefill fused GeGLU through the MFMA GEMM: x [2048,5376], gate and up [21504x5376]
    (1344 tiles of 256 tokens x 128 h columns: five whole rounds, the last 1024 h columns
    as narrow tiles).  Every element against gelu_tanh(gate) * up from fp64 contractions
    of the oracle's dequantisation, the oracle's GeGLU."""
    x, g, u = synth.geglu_case(seed=3, tokens=2048)
    xf = bf16(x).astype(np.float64)
    out = hip.DeviceArray((2048, g.rows), np.uint16)
    hip.nvfp4_geglu_bf16(dev(x), dev(g.codes), dev(g.scales), dev(u.codes), dev(u.scales), out, 2048,
                         g.rows, x.shape[1])
    hip.synchronize()
    got = bf16(out.numpy())
    gate = (xf @ dequant_f64(g.codes, g.scales).T).astype(np.float32)
    up = (xf @ dequant_f64(u.codes, u.scales).T).astype(np.float32)
    want = oracle.geglu(gate, up)
    assert count_outside(got, want, 2.0 ** -7, 2e-3) == 0
    assert rel_l2(got, want) < TOL_BF16
    nf, nt, _ = hip.gemm_tail_plan(2048, g.rows, True)
    assert nt == 0 or rel_l2(got[:, nf * 128:], want[:, nf * 128:]) < TOL_BF16


def test_gemm_many_tiles_exact():
    """416 tiles of 256 x 256 (more than one round of the 256 CUs, the second partial),
    K of 7 stages.  One-hot rows make every output a single weight, so a tile computed
    twice, skipped or written to the wrong place shows up exactly.  Random rows then
    check against the oracle on sampled columns, and a repeat launch must be
    bit-identical."""
    rng = np.random.default_rng(12)
    M, N, K = 256, 416 * 256, 448
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), perm] = 1.0
    got = bf16(gemm(synth.bf16_from_f32(A), w))
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    A = synth.normal_bf16(rng, (M, K))
    C = gemm(A, w)
    assert np.array_equal(gemm(A, w), C)
    ni = np.sort(rng.choice(N, 2048, replace=False))
    want = oracle.matvec_rows(w.codes, w.scales, bf16(A), ni)
    assert rel_l2(bf16(C)[:, ni], want) < TOL_BF16


# (M, N, narrow W blocks on 256 CUs): whole 256 x 256 tiles for R rounds, narrow tiles
# (4 waves x 64 rows, nt 32-row W blocks) for the columns past them (N - 65536 columns
# for M = 256); ragged M and N
NARROW_PLAIN = [(256, 70536, 1), (256, 76800, 2), (300, 38440, 2), (520, 25677, 2)]


@pytest.mark.parametrize("M,N,nt", NARROW_PLAIN)
def test_gemm_narrow_tail_tiles_exact(M, N, nt):
    """Columns past the whole tiles' rounds run as narrow tiles (widths 1 and 2, ragged
    M and N): one-hot rows make every output one weight, bit-exact; then random rows
    against the oracle on the narrow columns and a sample of the rest, and the fp32
    matmul (hi + lo split A, 2K columns, fp32 out) the same way."""
    assert hip.gemm_tail_plan(M, N, False, 256)[1] == nt
    assert hip.gemm_tail_plan(M, N, False)[1] > 0  # this device takes narrow tiles too
    rng = np.random.default_rng(N + nt)
    K = 128
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), perm] = 1.0
    got = bf16(gemm(synth.bf16_from_f32(A), w))
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    A = synth.normal_bf16(rng, (M, K))
    C = bf16(gemm(A, w))
    nf = hip.gemm_tail_plan(M, N, False)[0]
    ni = np.concatenate([np.sort(rng.choice(nf * 256, 512, replace=False)), np.arange(nf * 256, N)])
    want = oracle.matvec_rows(w.codes, w.scales, bf16(A), ni)
    assert rel_l2(C[:, ni], want) < TOL_BF16
    if nt == 2 or M != 256:
        X = rng.standard_normal((M, K), dtype=np.float32)
        got = run_matmul_f32(X, w)
        assert rel_l2(got[:, ni], oracle.matvec_rows(w.codes, w.scales, X, ni)) < TOL_REF_GATE


# (M, N, GeGLU): the columns past the whole tiles' rounds run as short tiles (full
# width, 1 to 6 32-row blocks of one tail column each, one per CU of the last round);
# ragged M and N
SHORT = [(2048, 21504, False), (2000, 21404, False), (1300, 30000, False), (30, 102187, False),
         (1024, 21504, True), (1300, 30000, True)]


@pytest.mark.parametrize("M,N,geglu", SHORT)
def test_gemm_short_tail_tiles_exact(M, N, geglu, gemm_threshold):
    """Short tail tiles: plain GEMM with one-hot rows (every output one weight,
    bit-exact), then random rows against the oracle on the tail columns and a sample of
    the rest, bf16 and fp32 (hi + lo split A) out; GeGLU bf16 and fp32 out against the
    oracle's GeGLU on every column."""
    nf, nt, ns = hip.gemm_tail_plan(M, N, geglu, 256)
    tiles_m = (M + 255) // 256
    assert nt == 0 and 0 < ns <= 256 + tiles_m  # the CUs left in the last round
    assert hip.gemm_tail_plan(M, N, geglu)[2] > 0  # this device takes short tiles too
    rng = np.random.default_rng(M + N)
    K = 64 if geglu else 128
    if geglu:
        g, u = synth.nvfp4_weights(rng, N, K), synth.nvfp4_weights(rng, N, K)
        x = synth.normal_bf16(rng, (M, K))
        xf = bf16(x)
        want = oracle.geglu(oracle.matvec(g.codes, g.scales, xf), oracle.matvec(u.codes, u.scales, xf))
        got = run_geglu(x, g, u, False)
        assert count_outside(got, want, 2.0 ** -7, 2e-3) == 0
        assert rel_l2(got, want) < TOL_BF16
        assert rel_l2(run_geglu(xf, g, u, True), want) < TOL_REF_GATE
        return
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), perm] = 1.0
    got = bf16(gemm(synth.bf16_from_f32(A), w))
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    A = synth.normal_bf16(rng, (M, K))
    C = bf16(gemm(A, w))
    ni = np.concatenate([np.sort(rng.choice(nf * 256, 512, replace=False)), np.arange(nf * 256, N)])
    want = oracle.matvec_rows(w.codes, w.scales, bf16(A), ni)
    assert count_outside(C[:, ni], want, 2.0 ** -7, 2e-3) == 0
    X = rng.standard_normal((M, K), dtype=np.float32)
    got = run_matmul_f32(X, w)
    assert rel_l2(got[:, ni], oracle.matvec_rows(w.codes, w.scales, X, ni)) < TOL_REF_GATE


@pytest.mark.parametrize("T,N,nt", [(256, 38400, 2), (300, 20000, 2), (520, 13000, 2)])
def test_geglu_narrow_tail_tiles(T, N, nt, gemm_threshold):
    """GeGLU GEMMs (bf16 and fp32 out) whose last h columns run as narrow tiles of one
    gate and one up block (32 h columns), ragged T and N, against the oracle."""
    assert hip.gemm_tail_plan(T, N, True, 256)[1] == nt
    rng = np.random.default_rng(T + N)
    K = 64
    g, u = synth.nvfp4_weights(rng, N, K), synth.nvfp4_weights(rng, N, K)
    x = synth.normal_bf16(rng, (T, K))
    xf = bf16(x)
    want = oracle.geglu(oracle.matvec(g.codes, g.scales, xf), oracle.matvec(u.codes, u.scales, xf))
    assert rel_l2(run_geglu(x, g, u, False), want) < TOL_BF16
    assert rel_l2(run_geglu(xf, g, u, True, 0.5, 2.0),
                  oracle.geglu(oracle.matvec(g.codes, g.scales, xf, 0.5),
                               oracle.matvec(u.codes, u.scales, xf, 2.0))) < TOL_REF_GATE


def test_gemm_tensor_scale_and_matmul_dispatch(gemm_threshold):
    """apex_nvfp4_matmul_bf16 switches to the GEMM (here from 64 tokens); results agree
    with the GEMM entry point, and a power-of-two tensor scale scales the output
    exactly."""
    hip.set_gemm_min_tokens(64, 0)
    rng = np.random.default_rng(3)
    w = synth.nvfp4_weights(rng, 448, 1024)
    A = synth.normal_bf16(rng, (96, 1024))
    C1 = gemm(A, w, 1.0)
    out = hip.DeviceArray((96, 448), np.uint16)
    hip.nvfp4_matmul_bf16(dev(A), dev(w.codes), dev(w.scales), out, 96, 448, 1024, 1.0)
    hip.synchronize()
    assert np.array_equal(out.numpy(), C1)
    C2 = gemm(A, w, 0.5)
    assert np.array_equal(bf16(C2), bf16(C1) * np.float32(0.5))


# ---- dense matmul / GeGLU through the MFMA GEMM (from 64 tokens), bf16 and fp32 ----


@pytest.fixture
def gemm_threshold():
    """Dense matmul / GeGLU through the GEMM at every token count (the size rule picks
    GEMV or GEMM by grid size); restores the rule afterwards."""
    hip.set_gemm_min_tokens(1, 1)
    yield
    hip.set_gemm_min_tokens(0, 0)


def run_matmul_f32(X, w, ts=1.0):
    T, K = X.shape
    out = hip.DeviceArray((T, w.rows), np.float32)
    hip.nvfp4_matmul_f32(dev(X), dev(w.codes), dev(w.scales), out, T, w.rows, K, ts)
    hip.synchronize()
    return out.numpy()


def run_geglu(x, g, u, f32, gs=1.0, us=1.0, norm=None):
    T, K = x.shape
    out = hip.DeviceArray((T, g.rows), np.float32 if f32 else np.uint16)
    args = (dev(g.codes), dev(g.scales), dev(u.codes), dev(u.scales), out, T, g.rows, K)
    if norm is not None:
        hip.nvfp4_geglu_rms_norm_f32(dev(x), dev(norm[0]), norm[1], *args, gate_scale=gs, up_scale=us)
    elif f32:
        hip.nvfp4_geglu_f32(dev(x), *args, gate_scale=gs, up_scale=us)
    else:
        hip.nvfp4_geglu_bf16(dev(x), *args, gate_scale=gs, up_scale=us)
    hip.synchronize()
    return out.numpy() if f32 else bf16(out.numpy())


@pytest.mark.parametrize("M,N,K", [(300, 448, 512), (64, 100, 320), (129, 37, 64)])
def test_matmul_f32_split_gemm_one_hot_exact(M, N, K, gemm_threshold):
    """fp32 activations through the bf16 hi + lo split GEMM: a one-hot row splits into
    hi = 1, lo = 0, so C[m, n] = W[n, p(m)] exactly (also N not a multiple of 4: one
    fp32 store per element)."""
    rng = np.random.default_rng(M + N)
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    X = np.zeros((M, K), np.float32)
    X[np.arange(M), perm] = 1.0
    got = run_matmul_f32(X, w)
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(300, 448, 1024), (64, 2112, 2816), (100, 36, 128)])
def test_matmul_f32_gemm_matches_oracle_and_gemv(M, N, K, gemm_threshold):
    """The split GEMM meets the reference's fp32 gate (rel L2 < 1e-5) against the fp64
    oracle, and agrees with the fp32 GEMV on the same inputs; a tensor scale of 0.5
    halves the output exactly."""
    rng = np.random.default_rng(3 * M + N)
    w = synth.nvfp4_weights(rng, N, K)
    X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    got = run_matmul_f32(X, w)
    want = oracle.matvec(w.codes, w.scales, X)
    assert rel_l2(got, want) < TOL_REF_GATE
    assert np.array_equal(run_matmul_f32(X, w, 0.5), got * np.float32(0.5))
    hip.set_gemm_min_tokens(0, 1 << 20)   # GEMV for every size
    gemv = run_matmul_f32(X, w)
    assert rel_l2(got, gemv) < TOL_REF_GATE


@pytest.mark.parametrize("T,rows,K", [(300, 448, 1024), (64, 100, 320), (97, 37, 192)])
def test_geglu_gemm_bf16_and_f32(T, rows, K, gemm_threshold):
    """GeGLU GEMM tiles hold 128 gate and 128 up rows of the same outputs: 448 rows end
    in a half-empty tile, 100 and 37 rows need per-element stores.  bf16 against the
    oracle on the bf16 inputs (1e-2), fp32 at the reference gate (1e-5); tensor scales
    apply per matrix."""
    rng = np.random.default_rng(T + rows + K)
    g, u = synth.nvfp4_weights(rng, rows, K), synth.nvfp4_weights(rng, rows, K)
    x = synth.normal_bf16(rng, (T, K))
    xf = bf16(x)
    want = oracle.geglu(oracle.matvec(g.codes, g.scales, xf), oracle.matvec(u.codes, u.scales, xf))
    assert rel_l2(run_geglu(x, g, u, False), want) < TOL_BF16
    assert rel_l2(run_geglu(xf, g, u, True), want) < TOL_REF_GATE
    want_s = oracle.geglu(oracle.matvec(g.codes, g.scales, xf, 0.5),
                          oracle.matvec(u.codes, u.scales, xf, 2.0))
    assert rel_l2(run_geglu(xf, g, u, True, 0.5, 2.0), want_s) < TOL_REF_GATE
    hip.set_gemm_min_tokens(1 << 20, 1 << 20)
    assert rel_l2(run_geglu(xf, g, u, True), want) < TOL_REF_GATE


def test_geglu_rms_norm_gemm_matches_oracle(gemm_threshold):
    """RMSNorm folded into the split pass: 200 tokens of the Gemma dense shape (hidden
    2816, intermediate 2112) against rms_norm + GeGLU in the oracle, and against the
    GEMV form of the same entry point."""
    rng = np.random.default_rng(21)
    T, rows, K, eps = 200, 2112, 2816, 1e-6
    x = (rng.standard_normal((T, K)) * 3).astype(np.float32)
    nw = synth.bf16_from_f32((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    g, u = synth.nvfp4_weights(rng, rows, K), synth.nvfp4_weights(rng, rows, K)
    got = run_geglu(x, g, u, True, norm=(nw, eps))
    xn = oracle.rms_norm(x, nw, eps)
    ids = np.sort(rng.choice(rows, 256, replace=False))
    want = oracle.geglu(oracle.matvec_rows(g.codes, g.scales, xn, ids),
                        oracle.matvec_rows(u.codes, u.scales, xn, ids))
    assert rel_l2(got[:, ids], want) < TOL_REF_GATE
    hip.set_gemm_min_tokens(0, 1 << 20)
    assert rel_l2(run_geglu(x, g, u, True, norm=(nw, eps)), got) < TOL_REF_GATE


@pytest.mark.parametrize("M,N,K", [(200, 301, 2048), (37, 64, 1024)])
def test_split_k_one_hot_exact(M, N, K, gemm_threshold):
    """Grids of few tiles run split-K: each workgroup sums a range of K stages into fp32
    partials and a second pass adds them in split order.  One-hot rows put each output's
    single product in one split (zeros in the others), so the bf16 GEMM and the fp32
    split GEMM (hi / lo halves in separate splits) return W[n, p(m)] exactly; random
    rows match the oracle."""
    rng = np.random.default_rng(M * N)
    w = synth.nvfp4_weights(rng, N, K)
    perm = rng.integers(0, K, size=M)
    X = np.zeros((M, K), np.float32)
    X[np.arange(M), perm] = 1.0
    want = oracle.decode(w.codes, w.scales)[:, perm].T + np.float32(0.0)
    got_b = bf16(gemm(synth.bf16_from_f32(X), w))
    assert np.array_equal(got_b.view(np.uint32), want.view(np.uint32))
    got_f = run_matmul_f32(X, w)
    assert np.array_equal(got_f.view(np.uint32), want.view(np.uint32))
    A = synth.normal_bf16(rng, (M, K))
    assert rel_l2(bf16(gemm(A, w)), oracle.matvec(w.codes, w.scales, bf16(A))) < TOL_BF16
    Xr = rng.standard_normal((M, K)).astype(np.float32)
    assert rel_l2(run_matmul_f32(Xr, w), oracle.matvec(w.codes, w.scales, Xr)) < TOL_REF_GATE


def test_split_pass_long_rows_and_tensor_scales(gemm_threshold):
    """fp32 rows longer than the split pass keeps in registers (K = 8256) take its
    element loop, with and without the RMSNorm folded in; GeGLU tensor scales and the
    matmul tensor scale apply on the split path as on the GEMV."""
    rng = np.random.default_rng(31)
    T, rows, K, eps = 40, 96, 8256, 1e-6
    x = rng.standard_normal((T, K)).astype(np.float32)
    nw = synth.bf16_from_f32((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    g, u = synth.nvfp4_weights(rng, rows, K), synth.nvfp4_weights(rng, rows, K)
    want = oracle.geglu(oracle.matvec(g.codes, g.scales, x, 0.25),
                        oracle.matvec(u.codes, u.scales, x, 4.0))
    assert rel_l2(run_geglu(x, g, u, True, 0.25, 4.0), want) < TOL_REF_GATE
    xn = oracle.rms_norm(x, nw, eps)
    want_n = oracle.geglu(oracle.matvec(g.codes, g.scales, xn), oracle.matvec(u.codes, u.scales, xn))
    assert rel_l2(run_geglu(x, g, u, True, norm=(nw, eps)), want_n) < TOL_REF_GATE
    assert rel_l2(run_matmul_f32(x, g, 2.0), oracle.matvec(g.codes, g.scales, x, 2.0)) < TOL_REF_GATE


def test_gemm_scratch_shared_by_two_streams(gemm_threshold):
    """The fp32 GEMM's split / split-K scratch is one set per device: calls of
    alternating sizes on two streams (the larger ones grow it) are ordered by the
    scratch's event, and every result meets the reference gate."""
    rng = np.random.default_rng(41)
    N, K = 300, 1024
    w = synth.nvfp4_weights(rng, N, K)
    dc, ds = dev(w.codes), dev(w.scales)
    s1, s2 = hip.Stream(), hip.Stream()
    keep = []
    for T, s in [(64, s1), (200, s2), (64, s2), (480, s1), (200, s1), (64, s2)]:
        X = rng.standard_normal((T, K)).astype(np.float32)
        dx, out = dev(X), hip.DeviceArray((T, N), np.float32)
        hip.nvfp4_matmul_f32(dx, dc, ds, out, T, N, K, stream=s)
        keep.append((X, dx, out))
    s1.synchronize()
    s2.synchronize()
    for X, dx, out in keep:
        assert rel_l2(out.numpy(), oracle.matvec(w.codes, w.scales, X)) < TOL_REF_GATE, X.shape
    s1.close()
    s2.close()


@pytest.mark.parametrize("T", [15, 16, 31, 32, 33])
def test_dense_dispatch_boundaries_by_size(T):
    """The default size rule changes path at 16 (GeGLU) and 32 (matmul, grids of few
    tiles) tokens; either side of each boundary meets the same gates: fp32 matmul and
    GeGLU at 1e-5, bf16 at 1e-2."""
    hip.set_gemm_min_tokens(0, 0)
    rng = np.random.default_rng(50 + T)
    N, K = 448, 1024
    g, u = synth.nvfp4_weights(rng, N, K), synth.nvfp4_weights(rng, N, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    assert rel_l2(run_matmul_f32(X, g), oracle.matvec(g.codes, g.scales, X)) < TOL_REF_GATE
    want = oracle.geglu(oracle.matvec(g.codes, g.scales, X), oracle.matvec(u.codes, u.scales, X))
    assert rel_l2(run_geglu(X, g, u, True), want) < TOL_REF_GATE
    xb = synth.bf16_from_f32(X)
    xf = bf16(xb)
    want_b = oracle.geglu(oracle.matvec(g.codes, g.scales, xf), oracle.matvec(u.codes, u.scales, xf))
    assert rel_l2(run_geglu(xb, g, u, False), want_b) < TOL_BF16
    out = hip.DeviceArray((T, N), np.uint16)
    hip.nvfp4_matmul_bf16(dev(xb), dev(g.codes), dev(g.scales), out, T, N, K)
    hip.synchronize()
    assert rel_l2(bf16(out.numpy()), oracle.matvec(g.codes, g.scales, xf)) < TOL_BF16


def test_dense_random_shapes(gemm_threshold):
    """Seeded random shapes through the MFMA GEMM paths (every token count takes the
    GEMM here): bf16 matmul, fp32 matmul (hi + lo split, split-K when the tiles are few)
    and fused GeGLU (bf16 and fp32), M 1..300, N 1..800, K a multiple of 64 up to 2048,
    against the oracle."""
    rng = np.random.default_rng(60)
    for _ in range(8):
        M, N, K = int(rng.integers(1, 301)), int(rng.integers(1, 801)), 64 * int(rng.integers(1, 33))
        print(f"dense GEMM M={M} N={N} K={K}", flush=True)
        w = synth.nvfp4_weights(rng, N, K)
        A = synth.normal_bf16(rng, (M, K))
        want = oracle.matvec(w.codes, w.scales, bf16(A))
        got = bf16(gemm(A, w))
        assert rel_l2(got, want) < TOL_BF16, (M, N, K)
        assert outside_bf16(got, want, 2e-3) == 0, (M, N, K)
        X = rng.standard_normal((M, K), dtype=np.float32)
        assert rel_l2(run_matmul_f32(X, w), oracle.matvec(w.codes, w.scales, X)) < TOL_REF_GATE, (M, N, K)
        u = synth.nvfp4_weights(rng, N, K)
        gx = oracle.geglu(oracle.matvec(w.codes, w.scales, bf16(A)), oracle.matvec(u.codes, u.scales, bf16(A)))
        got = run_geglu(A, w, u, False)
        assert rel_l2(got, gx) < TOL_BF16, (M, N, K)
        assert count_outside(got, gx, 2.0 ** -7, 2e-3) == 0, (M, N, K)
        gx = oracle.geglu(oracle.matvec(w.codes, w.scales, X), oracle.matvec(u.codes, u.scales, X))
        assert rel_l2(run_geglu(X, w, u, True), gx) < TOL_REF_GATE, (M, N, K)
