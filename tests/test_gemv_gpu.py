"""GPU parity of the decode-regime kernels (GEMV, fused GeGLU, dequant) against the
CPU oracle, through the C ABI.  Oracle = fp64 restatement of src/tests/cpu_ref.h."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import (TOL_BF16, TOL_REF_GATE, all_codes_weights, bf16, count_outside,
                           outside_bf16, rel_l2)

pytestmark = pytest.mark.gpu


def dev(a):
    return hip.DeviceArray.from_numpy(a)


def run_matmul(x, w, bf16_io, tensor_scale=1.0):
    T, K = x.shape
    out = hip.DeviceArray((T, w.rows), np.uint16 if bf16_io else np.float32)
    f = hip.nvfp4_matmul_bf16 if bf16_io else hip.nvfp4_matmul_f32
    f(dev(x), dev(w.codes), dev(w.scales), out, T, w.rows, K, tensor_scale)
    hip.synchronize()
    return out.numpy()


def test_dequant_bit_exact_every_code_and_scale():
    """src/nvfp4.h:27-43 on the device: all 16 x 256 (code, scale) pairs, bit for bit,
    including code 8 -> -0.0 and scales 0x7F/0xFF -> +-480."""
    w = all_codes_weights()
    want = oracle.decode(w.codes, w.scales)
    out = hip.DeviceArray((w.rows, w.K), np.float32)
    hip.nvfp4_dequant(dev(w.codes), dev(w.scales), out, w.rows, w.K)
    got = out.numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    outb = hip.DeviceArray((w.rows, w.K), np.uint16)
    hip.nvfp4_dequant(dev(w.codes), dev(w.scales), outb, w.rows, w.K)
    # every e2m1 x e4m3 product has <= 6 significant bits: bf16 holds it exactly
    assert np.array_equal(bf16(outb.numpy()).view(np.uint32), want.view(np.uint32))


def test_dequant_random_matches_reference_decoder():
    _, w = synth.gemv_case(seed=3, rows=64, K=2048)
    out = hip.DeviceArray((w.rows, w.K), np.float32)
    hip.nvfp4_dequant(dev(w.codes), dev(w.scales), out, w.rows, w.K)
    assert np.array_equal(out.numpy().view(np.uint32), oracle.decode(w.codes, w.scales).view(np.uint32))


def test_gemv_2048_f32_contract():
    """Single NVFP4 GEMV 2048x2048 (the reference op), fp32 in/out, seed 0."""
    x, w = synth.gemv_case(seed=0)
    xf = bf16(x)
    got = run_matmul(xf, w, bf16_io=False)
    want = oracle.matvec(w.codes, w.scales, xf)
    assert rel_l2(got, want) < TOL_REF_GATE


def test_gemv_2048_bf16():
    """Same case with bf16 activations and bf16 output (the configured dtype)."""
    x, w = synth.gemv_case(seed=0)
    got = bf16(run_matmul(x, w, bf16_io=True))
    want = oracle.matvec(w.codes, w.scales, bf16(x))
    assert rel_l2(got, want) < TOL_BF16
    # every element within half a bf16 step of the oracle's value (plus 1e-4 of the
    # rms for the fp32 accumulation): one wrong or misplaced output fails this
    assert outside_bf16(got, want) == 0


@pytest.mark.parametrize("rows,K,T", [
    (1, 16, 1), (3, 48, 2), (7, 32, 1), (64, 704, 3), (37, 2112, 5), (300, 2816, 1),
    (128, 5376, 2), (16, 8192, 4), (9, 8208, 2), (33, 1024, 16), (200, 256, 9),
])
def test_gemv_shapes_f32(rows, K, T):
    rng = np.random.default_rng(rows * 1000 + K + T)
    w = synth.nvfp4_weights(rng, rows, K)
    x = rng.standard_normal((T, K), dtype=np.float32)
    got = run_matmul(x, w, bf16_io=False)
    want = oracle.matvec(w.codes, w.scales, x)
    assert rel_l2(got, want) < TOL_REF_GATE


@pytest.mark.parametrize("rows,K,T", [(5, 16, 1), (64, 704, 1), (300, 2816, 3), (96, 5376, 1),
                                      (17, 8192, 2), (40, 4112, 1)])
def test_gemv_shapes_bf16(rows, K, T):
    rng = np.random.default_rng(rows + 7 * K + T)
    w = synth.nvfp4_weights(rng, rows, K)
    x = synth.normal_bf16(rng, (T, K))
    got = bf16(run_matmul(x, w, bf16_io=True))
    want = oracle.matvec(w.codes, w.scales, bf16(x))
    assert rel_l2(got, want) < TOL_BF16
    assert outside_bf16(got, want) == 0


def test_tensor_scale_is_linear():
    """The per-tensor FP32 scale multiplies the output (power of two: exactly)."""
    x, w = synth.gemv_case(seed=1, rows=256, K=2048)
    xf = bf16(x)
    a = run_matmul(xf, w, bf16_io=False, tensor_scale=1.0)
    b = run_matmul(xf, w, bf16_io=False, tensor_scale=0.25)
    assert np.array_equal(b, a * np.float32(0.25))
    c = run_matmul(xf, w, bf16_io=False, tensor_scale=0.3)
    assert rel_l2(c, oracle.matvec(w.codes, w.scales, xf, tensor_scale=0.3)) < TOL_REF_GATE


def run_geglu(x, gate, up, bf16_io):
    T, K = x.shape
    out = hip.DeviceArray((T, gate.rows), np.uint16 if bf16_io else np.float32)
    f = hip.nvfp4_geglu_bf16 if bf16_io else hip.nvfp4_geglu_f32
    f(dev(x), dev(gate.codes), dev(gate.scales), dev(up.codes), dev(up.scales), out, T,
      gate.rows, K)
    hip.synchronize()
    return out.numpy()


def geglu_oracle(x_f32, gate, up):
    g = oracle.matvec(gate.codes, gate.scales, x_f32)
    u = oracle.matvec(up.codes, up.scales, x_f32)
    return oracle.geglu(g, u)


@pytest.mark.parametrize("rows,K,T", [(8, 32, 1), (704, 2816, 1), (333, 2112, 2), (64, 5376, 4)])
def test_fused_geglu_small(rows, K, T):
    rng = np.random.default_rng(rows + K + T)
    x = synth.normal_bf16(rng, (T, K))
    gate = synth.nvfp4_weights(rng, rows, K)
    up = synth.nvfp4_weights(rng, rows, K)
    want = geglu_oracle(bf16(x), gate, up)
    got = bf16(run_geglu(x, gate, up, True))
    assert rel_l2(got, want) < TOL_BF16
    assert outside_bf16(got, want) == 0
    got = run_geglu(bf16(x), gate, up, False)
    assert rel_l2(got, want) < TOL_REF_GATE
    assert count_outside(got, want, 1e-5, 1e-4) == 0


def test_fused_geglu_decode_full_size():
    """Decode fused GeGLU at batch 1: x [1,5376], gate/up [21504 x 5376], seed 0, bf16 in
    and out.  Besides the rel L2 gate, every one of the 21,504 outputs lies within half a
    bf16 step of the oracle's value (plus 1e-4 of the rms): a single zeroed, swapped or
    misplaced output fails (the checker itself is tested on the CPU,
    test_oracle.py::test_elementwise_checker_catches_one_wrong_output)."""
    x, gate, up = synth.geglu_case(seed=0)
    got = bf16(run_geglu(x, gate, up, True))
    want = geglu_oracle(bf16(x), gate, up)
    assert rel_l2(got, want) < TOL_BF16
    assert outside_bf16(got, want) == 0


def test_fused_geglu_decode_full_size_f32():
    """The same workload through the reference's fp32 contract (apex_nvfp4_geglu_f32: fp32
    x in, fp32 out), at the reference harness's gate (src/tests/dense_mlp.cpp:113), and
    every element within 1e-5 of its value plus 1e-4 of the rms."""
    x, gate, up = synth.geglu_case(seed=0)
    xf = bf16(x)
    got = run_geglu(xf, gate, up, False)
    want = geglu_oracle(xf, gate, up)
    assert rel_l2(got, want) < TOL_REF_GATE
    assert count_outside(got, want, 1e-5, 1e-4) == 0


def test_standalone_geglu_f32_in_place():
    rng = np.random.default_rng(5)
    g = rng.standard_normal(10001, dtype=np.float32) * 3
    u = rng.standard_normal(10001, dtype=np.float32)
    dg, du = dev(g), dev(u)
    hip.geglu_f32(dg, du, dg, g.size)  # in place, as src/ops.h:67 does
    hip.synchronize()
    assert rel_l2(dg.numpy(), oracle.geglu(g, u)) < 1e-6


@pytest.mark.parametrize("bf16_io", [False, True])
def test_gemv_every_scale_code(bf16_io):
    """Every row holds every E4M3 scale code, including 0x7F/0xFF (+-480 in the
    reference, NaN in the hardware fp8 conversion): the kernel's exact fallback must
    reproduce the reference decode."""
    w = all_codes_weights(rows_per_code=2)
    rng = np.random.default_rng(11)
    x = synth.normal_bf16(rng, (1, w.K))
    got = run_matmul(x if bf16_io else bf16(x), w, bf16_io=bf16_io)
    got = bf16(got) if bf16_io else got
    want = oracle.matvec(w.codes, w.scales, bf16(x))
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) < (TOL_BF16 if bf16_io else TOL_REF_GATE)


def test_gemv_some_rows_with_480_scales():
    """Random weights where a few rows carry 0x7F / 0xFF scales among ordinary ones."""
    rng = np.random.default_rng(12)
    w = synth.nvfp4_weights(rng, 300, 5376)
    for r, col, code in [(3, 0, 0x7F), (77, 335, 0xFF), (150, 100, 0x7F), (299, 7, 0xFF)]:
        w.scales[r, col] = code
    x = synth.normal_bf16(rng, (1, w.K))
    want = oracle.matvec(w.codes, w.scales, bf16(x))
    got = run_matmul(bf16(x), w, bf16_io=False)
    assert rel_l2(got, want) < TOL_REF_GATE
    gotb = bf16(run_matmul(x, w, bf16_io=True))
    assert rel_l2(gotb, want) < TOL_BF16
    for r in (3, 77, 150, 299):
        assert abs(gotb[0, r] - want[0, r]) <= 1e-2 * abs(want[0, r]) + 1e-3


def test_fused_geglu_every_scale_code():
    gate = all_codes_weights()
    up = synth.Nvfp4Weights(gate.codes[::-1].copy(), gate.scales[:, ::-1].copy())
    rng = np.random.default_rng(13)
    x = synth.normal_bf16(rng, (1, gate.K)) * 0 + synth.bf16_from_f32(
        rng.standard_normal((1, gate.K), dtype=np.float32) * 0.01)
    want = geglu_oracle(bf16(x), gate, up)
    got = run_geglu(bf16(x), gate, up, False)
    assert rel_l2(got, want) < TOL_REF_GATE


def test_gemv_embedding_rows():
    """The largest GEMV a matmulNvfp4 caller has: the embedding table used as a linear
    layer, 262,144 rows x K 2816 (embed_tokens.weight [262144, 352] u32 in the model
    listing), batch 1, fp32 and bf16 activations; the oracle checks 2048 sampled rows."""
    rng = np.random.default_rng(31)
    rows, K = 262144, 2816
    w = synth.nvfp4_weights(rng, rows, K)
    sample = np.sort(rng.choice(rows, 2048, replace=False))
    for bf16_io in (False, True):
        x = synth.normal_bf16(rng, (1, K)) if bf16_io else rng.standard_normal((1, K), dtype=np.float32)
        got = run_matmul(x, w, bf16_io)
        got = bf16(got) if bf16_io else got
        want = oracle.matvec(w.codes[sample], w.scales[sample], bf16(x) if bf16_io else x)
        assert rel_l2(got[:, sample], want) < (TOL_BF16 if bf16_io else TOL_REF_GATE), bf16_io


def test_zero_tokens_write_nothing():
    """tokens = 0 is a valid call: the matmul (fp32 and bf16 activations), the fused GeGLU
    and the MoE FFN return success and leave their outputs as they were."""
    rng = np.random.default_rng(32)
    rows, K = 64, 256
    w = synth.nvfp4_weights(rng, rows, K)
    dw = (dev(w.codes), dev(w.scales))
    for f, xt, ot in [(hip.nvfp4_matmul_f32, np.float32, np.float32),
                      (hip.nvfp4_matmul_bf16, np.uint16, np.uint16)]:
        out = hip.DeviceArray((1, rows), ot)
        out.fill_bytes(0x5A)
        f(dev(np.zeros((1, K), xt)), *dw, out, 0, rows, K)
        hip.synchronize()
        assert np.all(out.numpy().view(np.uint8) == 0x5A)
    out = hip.DeviceArray((1, rows), np.uint16)
    out.fill_bytes(0x5A)
    hip.nvfp4_geglu_bf16(dev(np.zeros((1, K), np.uint16)), *dw, *dw, out, 0, rows, K)
    hip.synchronize()
    assert np.all(out.numpy().view(np.uint8) == 0x5A)
    E, H, I = 8, 256, 128
    slots = synth.expert_slots(rng, E, H, I)
    ds = dev(slots.data)
    y = hip.DeviceArray((1, H), np.uint16)
    y.fill_bytes(0x5A)
    ws = hip.DeviceArray((hip.moe_workspace_bytes(1, E, 2, H, I),), np.uint8)
    hip.moe_ffn_bf16(dev(np.zeros((1, H), np.uint16)), dev(np.zeros((1, E), np.uint16)),
                     hip.moe_slots(ds, slots.stride, slots.offsets), y, 0, E, 2, H, I, ws)
    hip.synchronize()
    assert np.all(y.numpy().view(np.uint8) == 0x5A)
