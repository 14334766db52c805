"""GPU parity of the Gemma-4 router front-end (docs/B6_3_attention.md:721-725): router
logits (RMSNorm with router.scale, affine 8-bit projection), routing from fp32 logits
with the per-expert scale, and the MoE FFN routed from them, against the CPU oracle.
Parity vs mlx-lm's router numerics is unpinned (not importable); the oracle's own
definition is pinned by tests/test_oracle.py."""
import numpy as np
import pytest

import oracle
from apex_amd import hip, synth
from tests.helpers import TOL_BF16, bf16, rel_l2

pytestmark = pytest.mark.gpu

EPS = 1e-6


def dev(a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def router_logits(h, rw):
    T, H = h.shape
    E = rw.qw.shape[0]
    out = hip.DeviceArray((T, E), np.float32)
    hip.moe_router_logits_q8(dev(h), dev(rw.norm_w), dev(rw.qw), dev(rw.qs), dev(rw.qb), out, T,
                             E, H, EPS)
    hip.synchronize()
    return out.numpy()


def test_router_small_shape_then_larger_shape():
    """Each router kernel first runs a small shape, then a larger one with more dynamic
    LDS: the LDS limit is raised once, to the kernel's largest possible size, so the
    second call must launch.  Placed first in the file so these are the process's first
    router launches.  VALU form (more than 256 tokens: 8-token tiles): 257 tokens at
    H 64, E 8, then 300 at H 2816, E 64.  Fused MFMA form (from 512 tokens): 512 tokens
    at H 1024, E 8, then 8192 at H 2816, E 128, checked on a 64-token sample."""
    rng = np.random.default_rng(21)
    for T, E, H, sample in [(257, 8, 64, None), (300, 64, 2816, None),
                            (512, 8, 1024, None), (8192, 128, 2816, 64)]:
        h, rw = synth.router_case(seed=T + E, tokens=T, E=E, H=H)
        print(f"router logits T={T} E={E} H={H}", flush=True)
        got = router_logits(h, rw)
        rows = np.arange(T) if sample is None else np.sort(rng.choice(T, sample, replace=False))
        want = oracle.moe_router_logits(h[rows], rw.norm_w, rw.qw, rw.qs, rw.qb, EPS)
        assert rel_l2(got[rows], want) < 1e-5, (T, E, H)


@pytest.mark.parametrize("T,E,H", [(1, 128, 2816), (16, 128, 2816), (300, 128, 2816),
                                   (33, 64, 256), (9, 200, 4096), (257, 8, 64),
                                   (600, 128, 2816), (515, 200, 1024), (512, 8, 4096),
                                   (520, 128, 2880), (530, 16, 320), (512, 256, 192),
                                   (513, 129, 64)])
def test_router_logits_match_oracle(T, E, H):
    """From 512 tokens the fused MFMA form runs (the scaled rows split into bf16 hi + lo
    on the fly, codes exact in bf16, the RMSNorm factor applied to the finished sums;
    experts in blocks of 128, so E 200 takes two), below the VALU kernels.  Its K
    chunks are 256 columns: H 2880, 320, 192 and 64 end on a partial chunk of 1, 1, 3
    and 1 groups; E 129 and 256 fill one expert block with one or all rows."""
    h, rw = synth.router_case(seed=T + E, tokens=T, E=E, H=H)
    print(f"router logits T={T} E={E} H={H}", flush=True)
    got = router_logits(h, rw)
    want = oracle.moe_router_logits(h, rw.norm_w, rw.qw, rw.qs, rw.qb, EPS)
    assert rel_l2(got, want) < 1e-5
    assert np.max(np.abs(got - want)) < 1e-4 * np.max(np.abs(want))


def oracle_route(logits, pes, k):
    ids, w = oracle.moe_route(logits, k)
    return ids, w * bf16(pes)[ids]


def separated(logits, k, gap=1e-3):
    """Tokens whose k-th and (k+1)-th largest logits differ by more than `gap` (the
    routing of the others may legitimately flip under fp32 rounding)."""
    s = -np.sort(-logits, axis=1)
    return (s[:, k - 1] - s[:, k]) > gap


def test_route_f32_with_per_expert_scale():
    h, rw = synth.router_case(seed=11, tokens=64, E=128, H=2816)
    lg = oracle.moe_router_logits(h, rw.norm_w, rw.qw, rw.qs, rw.qb, EPS)
    T, E, k = 64, 128, 8
    ids, w = hip.DeviceArray((T, k), np.int32), hip.DeviceArray((T, k), np.float32)
    hip.moe_route_f32(dev(lg), dev(rw.pes), ids, w, T, E, k)
    hip.synchronize()
    want_ids, want_w = oracle_route(lg, rw.pes, k)
    assert np.array_equal(ids.numpy(), want_ids)
    np.testing.assert_allclose(w.numpy(), want_w, rtol=3e-6, atol=1e-7)
    # without a scale: plain softmax weights summing to 1
    hip.moe_route_f32(dev(lg), None, ids, w, T, E, k)
    hip.synchronize()
    np.testing.assert_allclose(w.numpy().sum(axis=1), 1.0, rtol=1e-5)
    # -0 and +0 tie (lower id first), as equal values do
    z = np.full((1, E), -1.0, np.float32)
    z[0, 9], z[0, 4] = 0.0, -0.0
    ids1, w1 = hip.DeviceArray((1, 2), np.int32), hip.DeviceArray((1, 2), np.float32)
    hip.moe_route_f32(dev(z), None, ids1, w1, 1, E, 2)
    hip.synchronize()
    assert ids1.numpy().tolist() == [[4, 9]]


@pytest.mark.parametrize("T,path", [(16, 0), (16, 2), (300, 0)])
def test_moe_block_from_the_hidden_state(T, path):
    """router logits -> MoE FFN routed from them (fp32 logits, per-expert scale), hidden
    2816, intermediate 704, 128 experts, top-8, against the oracle composition
    (router logits, top-k softmax times the scale, per-pair dense FFN, slot-order sum)."""
    E, H, I, k = 128, 2816, 704, 8
    h, rw = synth.router_case(seed=20 + T, tokens=T, E=E, H=H)
    rng = np.random.default_rng(30 + T)
    x = synth.normal_bf16(rng, (T, H))
    slots = synth.expert_slots(rng, E, H, I)
    hip.set_moe_path(path)
    try:
        dl = hip.DeviceArray((T, E), np.float32)
        hip.moe_router_logits_q8(dev(h), dev(rw.norm_w), dev(rw.qw), dev(rw.qs), dev(rw.qb), dl, T,
                                 E, H, EPS)
        base = dev(slots.data)
        y = hip.DeviceArray((T, H), np.uint16)
        ws = hip.DeviceArray((hip.moe_workspace_bytes(T, E, k, H, I),), np.uint8)
        hip.moe_ffn_f32logits_bf16(dev(x), dl, dev(rw.pes), hip.moe_slots(base, slots.stride,
                                                                         slots.offsets), y, T, E,
                                   k, H, I, ws)
        hip.synchronize()
        got = bf16(y.numpy())
    finally:
        hip.set_moe_path(0)
    lg = dl.numpy()
    rows = np.nonzero(separated(lg, k))[0]
    if T > 48:
        rows = np.random.default_rng(7).choice(rows, 48, replace=False)
        rows.sort()
    assert len(rows) > 0
    ids, w = oracle_route(lg[rows], rw.pes, k)
    want = oracle.moe_ffn(slots, bf16(x)[rows], ids, w)
    assert rel_l2(got[rows], want) < TOL_BF16
    assert np.all(np.isfinite(got))
