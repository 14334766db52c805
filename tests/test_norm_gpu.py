"""GPU parity of rms_norm_f32 and head_norm_rope_f32 against the CPU oracle, through
the C ABI and through the Backend registry with the reference's launch shapes
(src/ops.h:18-26, 71-118).  Tolerance: the reference's own test-norm gate, rel L2
< 1e-5 (src/tests/test_norm.cpp:89-91)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import TOL_REF_GATE, rel_l2

pytestmark = pytest.mark.gpu


def dev(a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


class Offset:
    """A device address `nbytes` past the start of a DeviceArray (misaligned rows)."""

    def __init__(self, arr, nbytes):
        self.arr = arr
        self.ptr = arr.ptr + nbytes


def weights(rng, n):
    return synth.bf16_from_f32((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))


@pytest.mark.parametrize("rows,n", [(1, 2816), (7, 2816), (64, 5376), (3, 2112), (5, 1000),
                                    (2, 4096), (1, 16), (1, 3)])
def test_rms_norm_matches_oracle(rows, n):
    rng = np.random.default_rng(rows * 7919 + n)
    x = rng.standard_normal((rows, n)).astype(np.float32) * 3
    w = weights(rng, n)
    eps = 1e-6
    y = hip.DeviceArray((rows, n), np.float32)
    print(f"rms_norm rows={rows} n={n}", flush=True)
    hip.rms_norm_f32(dev(x), dev(w), y, rows, n, eps)
    hip.synchronize()
    want = oracle.rms_norm(x, w, eps)
    assert rel_l2(y.numpy(), want) < TOL_REF_GATE
    assert np.max(np.abs(y.numpy() - want)) < 1e-5 * np.max(np.abs(want)) + 1e-6


def test_rms_norm_in_place_and_misaligned():
    rng = np.random.default_rng(11)
    rows, n = 4, 2816
    x = rng.standard_normal((rows, n)).astype(np.float32)
    w = weights(rng, n + 1)
    want = oracle.rms_norm(x, w[1:], 1e-5)
    # in place, aligned
    d = dev(x)
    hip.rms_norm_f32(d, dev(w[1:].copy()), d, rows, n, 1e-5)
    hip.synchronize()
    assert rel_l2(d.numpy(), want) < TOL_REF_GATE
    # rows and weights at 4- and 2-byte offsets (the element-wise path)
    xb = np.concatenate([np.zeros(1, np.float32), x.ravel()])
    dx, dw = dev(xb), dev(w)
    y = hip.DeviceArray((rows * n + 1,), np.float32)
    hip.rms_norm_f32(Offset(dx, 4), Offset(dw, 2), Offset(y, 4), rows, n, 1e-5)
    hip.synchronize()
    assert rel_l2(y.numpy()[1:].reshape(rows, n), want) < TOL_REF_GATE


CASES = [
    # tokens, heads, head_dim, rope_pairs, base, abs_pos, has_weight
    (1, 8, 256, 128, 10000.0, 0, True),
    (3, 16, 256, 128, 10000.0, 5, True),
    (2, 8, 512, 64, 1000000.0, 17, True),
    (4, 4, 256, 0, 10000.0, 9, True),
    (2, 8, 256, 128, 10000.0, 30, False),
    (5, 2, 128, 32, 10000.0, 3, True),
    (1, 1, 2, 1, 10000.0, 2, True),
]


@pytest.mark.parametrize("T,Hh,D,pairs,base,pos,has_w", CASES)
def test_head_norm_rope_matches_oracle(T, Hh, D, pairs, base, pos, has_w):
    rng = np.random.default_rng(T * 1000 + Hh * 10 + D)
    x = rng.standard_normal((T, Hh, D)).astype(np.float32)
    w = weights(rng, D)
    eps = 1e-6
    y = hip.DeviceArray((T * Hh * D,), np.float32)
    print(f"head_norm_rope T={T} heads={Hh} D={D} pairs={pairs} pos={pos}", flush=True)
    hip.head_norm_rope_f32(dev(x), dev(w) if has_w else None, y, T, Hh, D, pairs, base, pos,
                           Hh * D, D, eps, has_weights=has_w)
    hip.synchronize()
    want = oracle.head_norm_rope(x, w, pairs, base, pos, eps, has_weight=has_w)
    assert rel_l2(y.numpy(), want) < TOL_REF_GATE


def test_head_norm_rope_strided_output_leaves_gaps_alone():
    """Heads written into a wider [T, 2 * heads * D] buffer (q/k/v packing): the gaps
    keep their contents."""
    rng = np.random.default_rng(21)
    T, Hh, D = 3, 4, 256
    x = rng.standard_normal((T, Hh, D)).astype(np.float32)
    w = weights(rng, D)
    ts, hs = 2 * Hh * D, D
    n = T * ts
    y = dev(np.full(n, 7.0, np.float32))
    hip.head_norm_rope_f32(dev(x), dev(w), y, T, Hh, D, 128, 10000.0, 4, ts, hs, 1e-6)
    hip.synchronize()
    want = oracle.head_norm_rope(x, w, 128, 10000.0, 4, 1e-6, out_token_stride=ts,
                                 out_head_stride=hs, out_size=n)
    got = y.numpy()
    mask = np.zeros(n, bool)
    for t in range(T):
        mask[t * ts: t * ts + Hh * D] = True
    assert rel_l2(got[mask], want[mask]) < TOL_REF_GATE
    assert np.all(got[~mask] == 7.0)


def test_head_norm_rope_far_positions_rotate_without_scaling():
    """At large positions the fp32 angle (abs_pos + t) * f rounds differently on the
    device and the host, so compare what the position cannot change: every pair keeps
    the norm of the un-rotated (rope_pairs = 0) output, and the un-rotated pairs match
    the oracle."""
    rng = np.random.default_rng(31)
    T, Hh, D, pairs = 2, 8, 256, 64
    x = rng.standard_normal((T, Hh, D)).astype(np.float32)
    w = weights(rng, D)
    y = hip.DeviceArray((T, Hh, D), np.float32)
    hip.head_norm_rope_f32(dev(x), dev(w), y, T, Hh, D, pairs, 10000.0, 100000, Hh * D, D, 1e-6)
    hip.synchronize()
    got = y.numpy().astype(np.float64)
    n = oracle.head_norm_rope(x, w, 0, 10000.0, 0, 1e-6).reshape(T, Hh, D).astype(np.float64)
    half = D // 2
    gn = np.hypot(got[..., :half], got[..., half:])
    nn = np.hypot(n[..., :half], n[..., half:])
    assert np.allclose(gn, nn, rtol=1e-5, atol=1e-6)
    assert np.allclose(got[..., pairs:half], n[..., pairs:half], rtol=1e-5, atol=1e-6)


def test_reference_launches_through_the_backend():
    """rmsNorm / headNormRope exactly as src/ops.h queues them: Dim3{rows} and
    Dim3{tokens, heads} with 256 threads, weights at an offset in a shared buffer."""
    rng = np.random.default_rng(41)
    be = hip.Backend(0)
    try:
        rows, n, eps = 6, 2816, 1e-6
        x = rng.standard_normal((rows, n)).astype(np.float32)
        w = weights(rng, n)
        core = np.zeros(4096 + n * 2, np.uint8)
        core[4096:] = w.view(np.uint8)
        bx, bc = be.allocate(x.nbytes, "activations"), be.allocate(core.nbytes, "core_weights")
        by = be.allocate(x.nbytes, "activations")
        be.contents(bx, np.float32, x.size)[:] = x.ravel()
        be.contents(bc, np.uint8, core.size)[:] = core
        be.run("rms_norm_f32", [hip.buf(bx), hip.buf(bc, 4096), hip.buf(by), hip.u32(n),
                                hip.f32(eps)], (rows,), (256,))
        be.sync()
        got = be.contents(by, np.float32, x.size).reshape(rows, n)
        assert rel_l2(got, oracle.rms_norm(x, w, eps)) < TOL_REF_GATE

        T, Hh, D = 3, 8, 256
        q = rng.standard_normal((T, Hh, D)).astype(np.float32)
        hw = weights(rng, D)
        bq, bw = be.allocate(q.nbytes, "activations"), be.allocate(hw.nbytes, "core_weights")
        bo = be.allocate(q.nbytes, "activations")
        be.contents(bq, np.float32, q.size)[:] = q.ravel()
        be.contents(bw, np.uint16, hw.size)[:] = hw
        be.run("head_norm_rope_f32",
               [hip.buf(bq), hip.buf(bw), hip.buf(bo), hip.u32(Hh), hip.u32(D), hip.u32(1),
                hip.u32(128), hip.f32(10000.0), hip.u32(11), hip.u32(Hh * D), hip.u32(D),
                hip.f32(eps)], (T, Hh), (256,))
        be.sync()
        got = be.contents(bo, np.float32, q.size)
        assert rel_l2(got, oracle.head_norm_rope(q, hw, 128, 10000.0, 11, eps)) < TOL_REF_GATE
        for b in (bx, bc, by, bq, bw, bo):
            be.release(b)
    finally:
        be.close()
