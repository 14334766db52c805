"""GPU parity of the prefill NVFP4 GEMM (bf16 MFMA on exactly dequantised weights)
against the CPU oracle (fp64 restatement of src/tests/cpu_ref.h matvecNvfp4Cpu)."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import TOL_BF16, bf16, rel_l2

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


@pytest.mark.parametrize("M,N,K", [(64, 224, 704), (300, 448, 2816), (513, 256, 1024),
                                   (130, 1408, 2816)])
def test_gemm_random(M, N, K):
    rng = np.random.default_rng(7 * M + N + K)
    w = synth.nvfp4_weights(rng, N, K)
    A = synth.normal_bf16(rng, (M, K))
    got = bf16(gemm(A, w))
    want = oracle.matvec(w.codes, w.scales, bf16(A))
    assert rel_l2(got, want) < TOL_BF16


def test_gemm_prefill_full_size_sampled():
    """Prefill dense GEMM: A [2048,5376] x W [21504x5376], seed 0.  The oracle checks
    48 sampled rows of A against 1024 sampled weight rows; every row of the output is
    checked against its own fp32 sum-of-row invariant."""
    A, w = synth.gemm_case(seed=0)
    M, K = A.shape
    C = bf16(gemm(A, w))
    rng = np.random.default_rng(1)
    mi = np.sort(rng.choice(M, 48, replace=False))
    ni = np.sort(rng.choice(w.rows, 1024, replace=False))
    want = oracle.matvec_rows(w.codes, w.scales, bf16(A[mi]), ni)
    assert rel_l2(C[np.ix_(mi, ni)], want) < TOL_BF16
    # all rows/cols at once: C . 1 = A . (W^T 1); W^T 1 is the column sum of the
    # dequantised weights, exact in fp64
    wsum = np.zeros(K, np.float64)
    for r0 in range(0, w.rows, 2048):
        wsum += synth.Nvfp4Weights(w.codes[r0:r0 + 2048], w.scales[r0:r0 + 2048]).dequant().sum(0, dtype=np.float64)
    lhs = C.astype(np.float64).sum(1)
    rhs = bf16(A).astype(np.float64) @ wsum
    # each output carries its bf16 rounding (~2^-9 / sqrt(3) relative, random sign), so
    # the row sums agree to ~1e-3; a wrong index or dropped term would be O(1)
    assert rel_l2(lhs, rhs) < TOL_BF16


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


def test_gemm_tensor_scale_and_matmul_dispatch():
    """apex_nvfp4_matmul_bf16 switches to the GEMM from 64 tokens; results agree with
    the GEMM entry point, and a power-of-two tensor scale scales the output exactly."""
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
