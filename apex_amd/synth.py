"""Seeded synthetic inputs for the NVFP4 matmul path (numpy only).

Weights use the reference's NVFP4 layout (src/ops.h:9-16, src/nvfp4.h:27-43):
codes are uint32 [rows, K/8] with element 8w+i in nibble i (LSB first) of word w,
scales are uint8 [rows, K/16] FP8 E4M3 codes.  Distributions:

* activations and router logits: N(0,1) rounded to bf16 (round-to-nearest-even);
* codes: every nibble uniform over the 16 E2M1 codes (uniform random bytes);
* scales: |N(0,1)| * 0.05 rounded to E4M3 (round-to-nearest-even, saturating);
* per-tensor FP32 scale: 1.0.

Draw order inside every builder is fixed (documented per function), so a seed pins
the bytes.  tests/test_synth.py pins the generator with SHA-256 digests.
"""
from __future__ import annotations

import dataclasses

import numpy as np

E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)

# Byte offsets of the six pieces of one expert slot, in the order tools/repack.py:182-189
# fixes (gate W, gate S, up W, up S, down W, down S), and the 16 KiB-aligned stride.
PIECES = ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")
SLOT_ALIGN = 16384


def bf16_from_f32(a) -> np.ndarray:
    """Round float32 to bf16 bits (uint16), nearest-even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_from_f32(v) -> np.ndarray:
    """Round float32 to FP8 E4M3 codes, nearest-even, saturating at +-448."""
    v = np.asarray(v, dtype=np.float32).astype(np.float64)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.abs(v)
    out = np.zeros(a.shape, dtype=np.uint8)
    sub = a < 2.0 ** -6
    out[sub] = np.rint(a[sub] * 512.0).astype(np.uint8)  # 8 lands exactly on code 0x08
    nrm = ~sub
    an = np.minimum(a[nrm], 464.0)
    frac, ex = np.frexp(an)  # an = frac * 2^ex, frac in [0.5, 1)
    ex = ex - 1
    mant = np.rint((2.0 * frac - 1.0) * 8.0)
    carry = mant == 8.0
    mant[carry] = 0.0
    ex[carry] += 1
    code = ((ex + 7) << 3).astype(np.int64) | mant.astype(np.int64)
    code[(an >= 464.0) | (code > 0x7E)] = 0x7E
    out[nrm] = code.astype(np.uint8)
    return out | sign


def e4m3_to_f32(b) -> np.ndarray:
    """Decode E4M3 codes like src/nvfp4.h:17-25 (0x7F/0xFF -> +-480, no NaN)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    e = (b >> 3) & 0xF
    m = (b & 7).astype(np.float64)
    v = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    return np.where(b & 0x80, -v, v).astype(np.float32)


def normal_bf16(rng: np.random.Generator, shape) -> np.ndarray:
    return bf16_from_f32(rng.standard_normal(shape, dtype=np.float32))


@dataclasses.dataclass
class Nvfp4Weights:
    codes: np.ndarray   # uint32 [rows, K/8]
    scales: np.ndarray  # uint8  [rows, K/16]
    tensor_scale: float = 1.0

    @property
    def rows(self) -> int:
        return self.codes.shape[0]

    @property
    def K(self) -> int:
        return self.codes.shape[1] * 8

    def dequant(self) -> np.ndarray:
        """fp32 [rows, K] = e2m1 * e4m3 * tensor_scale (exact for a power-of-two scale)."""
        c = self.codes.view(np.uint8)
        lo = (c & 0xF).astype(np.int64)
        hi = (c >> 4).astype(np.int64)
        nib = np.stack([lo, hi], axis=-1).reshape(self.rows, self.K)
        w = E2M1_VALUES[nib] * np.repeat(e4m3_to_f32(self.scales), 16, axis=1)
        return (w * np.float32(self.tensor_scale)).astype(np.float32)


def nvfp4_weights(rng: np.random.Generator, rows: int, K: int) -> Nvfp4Weights:
    """Draw order: code bytes (rows*K/2 uniform uint8), then rows*K/16 normals for scales."""
    if K % 16:
        raise ValueError("K must be a multiple of 16")
    codes = rng.integers(0, 256, size=rows * K // 2, dtype=np.uint8)
    codes = codes.view(np.uint32).reshape(rows, K // 8)
    scales = e4m3_from_f32(np.abs(rng.standard_normal(rows * K // 16, dtype=np.float32)) * 0.05)
    return Nvfp4Weights(codes, scales.reshape(rows, K // 16))


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------

def gemv_case(seed: int = 0, tokens: int = 1, rows: int = 2048, K: int = 2048):
    """Single NVFP4 GEMV (2048x2048 at batch 1 by default).  Draws: W, then x [T,K]."""
    rng = np.random.default_rng(seed)
    w = nvfp4_weights(rng, rows, K)
    x = normal_bf16(rng, (tokens, K))
    return x, w


def dense_mlp_case(seed: int = 0, tokens: int = 1, H: int = 2816, I: int = 2112):
    """Gemma dense MLP block (tools/out.txt:121-186 shapes): residual input h fp32 [T,H]
    ~N(0,1), pre-FFN RMSNorm weights bf16 [H] ~1+0.1N(0,1), gate/up NVFP4 [I,H], down
    NVFP4 [H,I].  Draws: h, norm weights, gate, up, down."""
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((tokens, H), dtype=np.float32)
    norm_w = bf16_from_f32((1.0 + 0.1 * rng.standard_normal(H, dtype=np.float32)).astype(np.float32))
    gate = nvfp4_weights(rng, I, H)
    up = nvfp4_weights(rng, I, H)
    down = nvfp4_weights(rng, H, I)
    return h, norm_w, gate, up, down


@dataclasses.dataclass
class RouterWeights:
    """Gemma-4 router tensors (tools/out.txt:247-290): router.scale bf16 [H],
    router.proj affine 8-bit (weight u32 [E, H/4], scales and biases bf16 [E, H/64])
    and router.per_expert_scale bf16 [E]."""
    norm_w: np.ndarray
    qw: np.ndarray
    qs: np.ndarray
    qb: np.ndarray
    pes: np.ndarray

    def dequant(self) -> np.ndarray:
        """fp64 [E, H]: scale * q + bias per 64-element group."""
        q = self.qw.view(np.uint8).astype(np.float64)
        E, H = q.shape
        s = np.repeat(bf16_to_f32(self.qs).astype(np.float64), 64, axis=1)
        b = np.repeat(bf16_to_f32(self.qb).astype(np.float64), 64, axis=1)
        return s * q + b


def router_weights(rng: np.random.Generator, E: int = 128, H: int = 2816) -> RouterWeights:
    """Draw order: norm weights ~1+0.1N, codes (uniform bytes), group scales
    |N|*0.004+0.001, group biases -127.5*scale+0.01N (centred groups), per-expert
    scales ~1+0.1N."""
    norm_w = bf16_from_f32((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    q = rng.integers(0, 256, size=(E, H), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((E, H // 64))) * 0.004 + 0.001).astype(np.float32)
    qs = bf16_from_f32(sc)
    bi = (-127.5 * bf16_to_f32(qs) + 0.01 * rng.standard_normal((E, H // 64))).astype(np.float32)
    qb = bf16_from_f32(bi)
    pes = bf16_from_f32((1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32))
    return RouterWeights(norm_w, q.view(np.uint32).reshape(E, H // 4), qs, qb, pes)


def router_case(seed: int = 0, tokens: int = 16, E: int = 128, H: int = 2816):
    """Router front-end input: raw hidden h fp32 [T, H] ~ N(0,1), then the router weights."""
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((tokens, H), dtype=np.float32)
    return h, router_weights(rng, E, H)


def geglu_case(seed: int = 0, tokens: int = 1, rows: int = 21504, K: int = 5376):
    """Decode fused GeGLU.  Draws: x [T,K], gate W, up W."""
    rng = np.random.default_rng(seed)
    x = normal_bf16(rng, (tokens, K))
    gate = nvfp4_weights(rng, rows, K)
    up = nvfp4_weights(rng, rows, K)
    return x, gate, up


def gemm_case(seed: int = 0, M: int = 2048, N: int = 21504, K: int = 5376):
    """Prefill dense GEMM A[M,K] x W[N,K]^T.  Draws: W, then A."""
    rng = np.random.default_rng(seed)
    w = nvfp4_weights(rng, N, K)
    a = normal_bf16(rng, (M, K))
    return a, w


@dataclasses.dataclass
class ExpertSlots:
    """128 experts in the fixed-stride slot format of tools/repack.py:180-257."""
    data: np.ndarray            # uint8 [E * stride]
    stride: int
    offsets: dict               # piece name -> byte offset inside a slot
    E: int
    H: int
    I: int

    def piece(self, e: int, name: str) -> np.ndarray:
        I, H = self.I, self.H
        base = e * self.stride + self.offsets[name]
        shapes = {"gate_w": (I, H // 8, np.uint32), "gate_s": (I, H // 16, np.uint8),
                  "up_w": (I, H // 8, np.uint32), "up_s": (I, H // 16, np.uint8),
                  "down_w": (H, I // 8, np.uint32), "down_s": (H, I // 16, np.uint8)}
        r, c, dt = shapes[name]
        n = r * c * np.dtype(dt).itemsize
        return self.data[base:base + n].view(dt).reshape(r, c)


def slot_layout(H: int, I: int):
    sizes = {"gate_w": I * H // 2, "gate_s": I * H // 16, "up_w": I * H // 2,
             "up_s": I * H // 16, "down_w": H * I // 2, "down_s": H * I // 16}
    offsets, off = {}, 0
    for name in PIECES:
        offsets[name] = off
        off += sizes[name]
    stride = (off + SLOT_ALIGN - 1) // SLOT_ALIGN * SLOT_ALIGN
    return offsets, stride, off


def expert_slots(rng: np.random.Generator, E: int, H: int, I: int) -> ExpertSlots:
    """Draws per expert e = 0..E-1: gate W, up W, down W (each codes then scales)."""
    offsets, stride, _ = slot_layout(H, I)
    data = np.zeros(E * stride, dtype=np.uint8)
    for e in range(E):
        base = e * stride
        for proj, (rows, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            w = nvfp4_weights(rng, rows, K)
            cw = w.codes.view(np.uint8).reshape(-1)
            cs = w.scales.reshape(-1)
            o = base + offsets[proj + "_w"]
            data[o:o + cw.size] = cw
            o = base + offsets[proj + "_s"]
            data[o:o + cs.size] = cs
    return ExpertSlots(data, stride, offsets, E, H, I)


def moe_decode_case(seed: int = 0, tokens: int = 16, H: int = 2816, I: int = 704, E: int = 128):
    """MoE decode.  Draws: x [T,H], logits [T,E] (both N(0,1) bf16), then expert slots."""
    rng = np.random.default_rng(seed)
    x = normal_bf16(rng, (tokens, H))
    logits = normal_bf16(rng, (tokens, E))
    slots = expert_slots(rng, E, H, I)
    return x, logits, slots


def zipf_logits(rng: np.random.Generator, tokens: int, E: int, s: float = 1.1,
                n_empty: int = 8) -> np.ndarray:
    """Skewed router logits: popularity p_e ~ rank_e^-s over a seeded permutation of
    experts, the n_empty lowest-ranked experts get p = 0 (logit -inf, never routed);
    logits[t,e] = bf16(log p_e + Gumbel(t,e)).  Draws: permutation, then T*E Gumbels."""
    rank = rng.permutation(E) + 1
    p = rank.astype(np.float64) ** -s
    p[rank > E - n_empty] = 0.0
    p /= p.sum()
    with np.errstate(divide="ignore"):
        logp = np.log(p)
    g = rng.gumbel(size=(tokens, E))
    return bf16_from_f32((logp[None, :] + g).astype(np.float32))


def moe_prefill_case(seed: int = 0, tokens: int = 4096, H: int = 2816, I: int = 704,
                     E: int = 128):
    """MoE prefill with Zipf(1.1) routing.  Draws: x [T,H], skewed logits, expert slots."""
    rng = np.random.default_rng(seed)
    x = normal_bf16(rng, (tokens, H))
    logits = zipf_logits(rng, tokens, E)
    slots = expert_slots(rng, E, H, I)
    return x, logits, slots


# ---- packed model directories (tools/repack.py:180-257 format) ---------------------

PIECE_NAMES = {"gate_w": "gate_proj.weight", "gate_s": "gate_proj.scales",
               "up_w": "up_proj.weight", "up_s": "up_proj.scales",
               "down_w": "down_proj.weight", "down_s": "down_proj.scales"}


def write_packed_model(out_dir, seed: int = 0, layers: int = 2, E: int = 128, H: int = 2816,
                       I: int = 704):
    """A synthetic packed model directory in the repack format: layer_NN.bin (E expert
    slots at a fixed page-aligned stride, the six pieces in the fixed order),
    core.bin (per layer: pre_feedforward_layernorm_2.weight and the router tensors,
    page-aligned) and manifest.json.  Returns (manifest dict, per-layer ExpertSlots,
    per-layer RouterWeights)."""
    import hashlib
    import json
    from pathlib import Path

    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    rng = np.random.default_rng(seed)
    page = SLOT_ALIGN
    tensors, core = [], bytearray()

    def add_core(name, dtype, shape, arr):
        off = (len(core) + page - 1) // page * page
        core.extend(b"\0" * (off - len(core)))
        data = np.ascontiguousarray(arr).tobytes()
        core.extend(data)
        tensors.append({"name": name, "dtype": dtype, "shape": list(shape), "offset": off,
                        "nbytes": len(data), "sha256": hashlib.sha256(data).hexdigest()})

    layer_entries, all_slots, all_routers = [], [], []
    for layer in range(layers):
        slots = expert_slots(rng, E, H, I)
        rw = router_weights(rng, E, H)
        norm2 = bf16_from_f32((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        p = f"layers.{layer}."
        add_core(p + "pre_feedforward_layernorm_2.weight", "BF16", [H], norm2)
        add_core(p + "router.scale", "BF16", [H], rw.norm_w)
        add_core(p + "router.proj.weight", "U32", [E, H // 4], rw.qw)
        add_core(p + "router.proj.scales", "BF16", [E, H // 64], rw.qs)
        add_core(p + "router.proj.biases", "BF16", [E, H // 64], rw.qb)
        add_core(p + "router.per_expert_scale", "BF16", [E], rw.pes)
        name = f"layer_{layer:02d}.bin"
        (out / name).write_bytes(slots.data.tobytes())
        shapes = {"gate_w": ("U32", [I, H // 8]), "gate_s": ("U8", [I, H // 16]),
                  "up_w": ("U32", [I, H // 8]), "up_s": ("U8", [I, H // 16]),
                  "down_w": ("U32", [H, I // 8]), "down_s": ("U8", [H, I // 16])}
        used = sum(int(np.prod(shapes[k][1])) * (4 if shapes[k][0] == "U32" else 1) for k in PIECES)
        layer_entries.append({
            "layer": layer, "file": name, "size": E * slots.stride, "num_experts": E,
            "stride": slots.stride,
            "pieces": [{"name": PIECE_NAMES[k], "dtype": shapes[k][0], "shape": shapes[k][1],
                        "offset": slots.offsets[k],
                        "nbytes": int(np.prod(shapes[k][1])) * (4 if shapes[k][0] == "U32" else 1)}
                       for k in PIECES],
            "expert_sha256": [hashlib.sha256(slots.data[e * slots.stride:e * slots.stride + used]
                                             .tobytes()).hexdigest() for e in range(E)],
        })
        all_slots.append(slots)
        all_routers.append(rw)
    core.extend(b"\0" * ((len(core) + page - 1) // page * page - len(core)))
    (out / "core.bin").write_bytes(bytes(core))
    manifest = {
        "version": 1, "alignment": page,
        "text_config": {
            "hidden_size": H, "intermediate_size": 2112, "moe_intermediate_size": I,
            "num_attention_heads": 16, "num_key_value_heads": 8, "head_dim": 256,
            "num_hidden_layers": layers, "num_experts": E, "top_k_experts": 8,
            "vocab_size": 262144, "sliding_window": 1024, "rms_norm_eps": 1e-6,
            "final_logit_softcapping": 30.0,
            "layer_types": ["sliding_attention"] * layers,
            "global_head_dim": 512, "num_global_key_value_heads": 2, "attention_k_eq_v": True,
            "rope_parameters": {"sliding_attention": {"rope_theta": 10000.0},
                                "full_attention": {"rope_theta": 1000000.0,
                                                   "partial_rotary_factor": 0.25}},
        },
        "quantization": {"group_size": 64, "bits": 8, "mode": "affine"},
        "core": {"file": "core.bin", "tensors": tensors, "size": len(core)},
        "layers": layer_entries,
    }
    (out / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    return manifest, all_slots, all_routers
