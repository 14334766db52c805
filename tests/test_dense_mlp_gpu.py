"""The Gemma dense MLP block end to end at its real shape (hidden 2816, intermediate
2112), as the reference's test-mlp harness runs it (src/tests/dense_mlp.cpp:79-101):
RMSNorm (pre_feedforward_layernorm) -> gate / up NVFP4 GEMVs -> GeGLU -> down GEMV,
against the oracle composition rmsNormCpu + denseMlpCpu (dense_mlp.cpp:148-182).  K =
2112 makes the scale rows 132 bytes long, so they are only 4-byte aligned.  Gate: the
reference's rel L2 < 1e-5 for the fp32 contract; 1e-2 for bf16 activations."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import TOL_BF16, TOL_REF_GATE, bf16, rel_l2

pytestmark = pytest.mark.gpu

H, I, EPS = 2816, 2112, 1e-6


def dev(a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def want(case):
    h, nw, g, u, d = case
    x = oracle.rms_norm(h, nw, EPS)
    return oracle.dense_mlp((g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales), x)


@pytest.mark.parametrize("T", [1, 5, 64])
def test_dense_mlp_fp32_reference_composition(T):
    """rmsNorm, then matmulNvfp4 x2, geglu_f32, matmulNvfp4 (4 launches, src/ops.h:57-69)."""
    case = synth.dense_mlp_case(seed=T, tokens=T)
    h, nw, g, u, d = case
    print(f"dense mlp fp32 T={T}", flush=True)
    dh, dnw, xn = dev(h), dev(nw), hip.DeviceArray((T, H), np.float32)
    gate, up, y = (hip.DeviceArray((T, I), np.float32), hip.DeviceArray((T, I), np.float32),
                   hip.DeviceArray((T, H), np.float32))
    hip.rms_norm_f32(dh, dnw, xn, T, H, EPS)
    hip.nvfp4_matmul_f32(xn, dev(g.codes), dev(g.scales), gate, T, I, H)
    hip.nvfp4_matmul_f32(xn, dev(u.codes), dev(u.scales), up, T, I, H)
    hip.geglu_f32(gate, up, gate, T * I)
    hip.nvfp4_matmul_f32(gate, dev(d.codes), dev(d.scales), y, T, H, I)
    hip.synchronize()
    assert rel_l2(y.numpy(), want(case)) < TOL_REF_GATE


@pytest.mark.parametrize("T", [1, 5])
def test_dense_mlp_fp32_fused(T):
    """rmsNorm, fused gate/up GeGLU GEMV, down GEMV (3 launches)."""
    case = synth.dense_mlp_case(seed=100 + T, tokens=T)
    h, nw, g, u, d = case
    xn, hh, y = (hip.DeviceArray((T, H), np.float32), hip.DeviceArray((T, I), np.float32),
                 hip.DeviceArray((T, H), np.float32))
    hip.rms_norm_f32(dev(h), dev(nw), xn, T, H, EPS)
    hip.nvfp4_geglu_f32(xn, dev(g.codes), dev(g.scales), dev(u.codes), dev(u.scales), hh, T, I, H)
    hip.nvfp4_matmul_f32(hh, dev(d.codes), dev(d.scales), y, T, H, I)
    hip.synchronize()
    assert rel_l2(y.numpy(), want(case)) < TOL_REF_GATE


@pytest.mark.parametrize("T", [1, 5])
def test_dense_mlp_fp32_norm_fused(T):
    """RMSNorm fused into the gate/up GeGLU GEMV, down GEMV (2 launches): the same
    reference gate; 5 tokens run as blocks of 2, 2 and 1."""
    case = synth.dense_mlp_case(seed=300 + T, tokens=T)
    h, nw, g, u, d = case
    hh, y = hip.DeviceArray((T, I), np.float32), hip.DeviceArray((T, H), np.float32)
    hip.nvfp4_geglu_rms_norm_f32(dev(h), dev(nw), EPS, dev(g.codes), dev(g.scales), dev(u.codes),
                                 dev(u.scales), hh, T, I, H)
    hip.nvfp4_matmul_f32(hh, dev(d.codes), dev(d.scales), y, T, H, I)
    hip.synchronize()
    assert rel_l2(y.numpy(), want(case)) < TOL_REF_GATE


def test_geglu_norm_fused_matches_separate_norm_and_rejects_bad_layouts():
    """Odd sizes (K = 320: the last chunk plane of x partly padding, 37 rows) against
    the separate rms_norm_f32 + geglu_nvfp4_f32 launches, and the fused form's layout
    requirements (fp32 x, K % 32 == 0) turned into errors, not a wrong result."""
    rng = np.random.default_rng(7)
    T, rows, K = 3, 37, 320
    h = rng.standard_normal((T, K)).astype(np.float32) * 3
    nw = synth.bf16_from_f32(rng.standard_normal(K).astype(np.float32))
    g, u = synth.nvfp4_weights(rng, rows, K), synth.nvfp4_weights(rng, rows, K)
    xn, sep, fused = (hip.DeviceArray((T, K), np.float32), hip.DeviceArray((T, rows), np.float32),
                      hip.DeviceArray((T, rows), np.float32))
    hip.rms_norm_f32(dev(h), dev(nw), xn, T, K, EPS)
    hip.nvfp4_geglu_f32(xn, dev(g.codes), dev(g.scales), dev(u.codes), dev(u.scales), sep, T, rows, K)
    hip.nvfp4_geglu_rms_norm_f32(dev(h), dev(nw), EPS, dev(g.codes), dev(g.scales), dev(u.codes),
                                 dev(u.scales), fused, T, rows, K)
    hip.synchronize()
    assert rel_l2(fused.numpy(), sep.numpy()) < 1e-6
    xg = oracle.rms_norm(h, nw, EPS)
    ref = oracle.geglu(oracle.matvec(g.codes, g.scales, xg), oracle.matvec(u.codes, u.scales, xg))
    assert rel_l2(fused.numpy(), ref) < TOL_REF_GATE
    g16 = synth.nvfp4_weights(rng, rows, 16 * 3)   # K = 48: not a multiple of 32
    with pytest.raises(hip.ApexHipError):
        hip.nvfp4_geglu_rms_norm_f32(dev(h[:, :48]), dev(nw[:48]), EPS, dev(g16.codes),
                                     dev(g16.scales), dev(g16.codes), dev(g16.scales), fused,
                                     T, rows, 48)


@pytest.mark.parametrize("T", [1, 96])
def test_dense_mlp_bf16(T):
    """bf16 activations after the norm: fused GeGLU and down projection (96 tokens: the
    GeGLU as an MFMA GEMM, the down projection's 11 tiles still a GEMV); the oracle runs
    the same composition on the bf16-rounded normed input."""
    case = synth.dense_mlp_case(seed=200 + T, tokens=T)
    h, nw, g, u, d = case
    x = oracle.rms_norm(h, nw, EPS)
    xb = synth.bf16_from_f32(x)
    ref = oracle.dense_mlp((g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales), bf16(xb))
    hh, y = hip.DeviceArray((T, I), np.uint16), hip.DeviceArray((T, H), np.uint16)
    hip.nvfp4_geglu_bf16(dev(xb), dev(g.codes), dev(g.scales), dev(u.codes), dev(u.scales), hh,
                         T, I, H)
    hip.nvfp4_matmul_bf16(hh, dev(d.codes), dev(d.scales), y, T, H, I)
    hip.synchronize()
    assert rel_l2(bf16(y.numpy()), ref) < TOL_BF16
