"""Python access to the CPU oracle (liboracle.so) and, where it was built, to the
reference's own CPU code (oracle/_ref/libapexref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product path (apex_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libapexref.so"

_P = C.c_void_p
_SZ = C.c_size_t
_F = C.c_float


class ExpertLayout(C.Structure):
    _fields_ = [("slot_stride", _SZ), ("gate_w", _SZ), ("gate_s", _SZ), ("up_w", _SZ),
                ("up_s", _SZ), ("down_w", _SZ), ("down_s", _SZ)]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        L.orc_e2m1_to_float.restype = _F
        L.orc_e2m1_to_float.argtypes = [C.c_uint32]
        L.orc_e4m3_to_float.restype = _F
        L.orc_e4m3_to_float.argtypes = [C.c_uint8]
        L.orc_decode_row.argtypes = [_P, _P, _P, _SZ]
        L.orc_matvec_nvfp4.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ, _F]
        L.orc_matvec_nvfp4_rows.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _P, _SZ, _F]
        L.orc_gelu_tanh.restype = _F
        L.orc_gelu_tanh.argtypes = [_F]
        L.orc_geglu.argtypes = [_P, _P, _P, _SZ]
        L.orc_dense_mlp.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ]
        L.orc_diff.argtypes = [_P, _P, _SZ, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.orc_moe_route.argtypes = [_P, _SZ, _SZ, _SZ, _P, _P]
        L.orc_moe_ffn.argtypes = [_P, C.POINTER(ExpertLayout), _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ]
        L.orc_e4m3_from_float.restype = C.c_uint8
        L.orc_e4m3_from_float.argtypes = [_F]
        L.orc_bf16_to_float.restype = _F
        L.orc_bf16_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_bf16.restype = C.c_uint16
        L.orc_float_to_bf16.argtypes = [_F]
        L.orc_rms_norm.argtypes = [_P, _P, _P, _SZ, _SZ, _F]
        L.orc_moe_router_logits_q8.argtypes = [_P, _P, _F, _P, _P, _P, _SZ, _SZ, _SZ, _P]
        L.orc_head_norm_rope.argtypes = [_P, _P, C.c_int, _P, _SZ, _SZ, _SZ, _SZ, _F, C.c_uint32,
                                         _SZ, _SZ, _F]
        _lib = L
    return _lib


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data


def e2m1(code: int) -> float:
    return lib().orc_e2m1_to_float(code)


def e4m3(byte: int) -> float:
    return lib().orc_e4m3_to_float(byte)


def decode(codes, scales) -> np.ndarray:
    """Dequantise every row: fp32 [rows, K]."""
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint8)
    rows, K = codes.shape[0], codes.shape[1] * 8
    out = np.empty((rows, K), np.float32)
    for r in range(rows):
        lib().orc_decode_row(pc + r * K // 2, ps + r * K // 16, out[r].ctypes.data, K)
    return out


def matvec(codes, scales, x, tensor_scale: float = 1.0) -> np.ndarray:
    """fp32 [T, rows] = W x (fp64 accumulation), x fp32 [T, K]."""
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    rows, K = codes.shape[0], codes.shape[1] * 8
    T = x.shape[0]
    assert x.shape[1] == K
    out = np.empty((T, rows), np.float32)
    lib().orc_matvec_nvfp4(pc, ps, px, out.ctypes.data, T, rows, K, tensor_scale)
    return out


def matvec_rows(codes, scales, x, row_ids, tensor_scale: float = 1.0) -> np.ndarray:
    """fp32 [T, len(row_ids)]: the matvec restricted to the listed rows."""
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    ids, pi = _c(row_ids, np.int64)
    K = codes.shape[1] * 8
    T = x.shape[0]
    out = np.empty((T, ids.size), np.float32)
    lib().orc_matvec_nvfp4_rows(pc, ps, px, out.ctypes.data, T, K, pi, ids.size, tensor_scale)
    return out


def gelu(g: float) -> float:
    return lib().orc_gelu_tanh(g)


def geglu(gate, up) -> np.ndarray:
    gate, pg = _c(gate, np.float32)
    up, pu = _c(up, np.float32)
    out = np.empty_like(gate)
    lib().orc_geglu(pg, pu, out.ctypes.data, gate.size)
    return out


def dense_mlp(gate, up, down, x) -> np.ndarray:
    """gate/up/down: (codes, scales) pairs; x fp32 [T, H] -> fp32 [T, H]."""
    gc, pgc = _c(gate[0], np.uint32)
    gs, pgs = _c(gate[1], np.uint8)
    uc, puc = _c(up[0], np.uint32)
    us, pus = _c(up[1], np.uint8)
    dc, pdc = _c(down[0], np.uint32)
    ds, pds = _c(down[1], np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    I, H = gc.shape[0], gc.shape[1] * 8
    out = np.empty((x.shape[0], H), np.float32)
    lib().orc_dense_mlp(pgc, pgs, puc, pus, pdc, pds, px, out.ctypes.data, x.shape[0], H, I)
    return out


def diff(a, b):
    """(max_abs, rel_l2) as src/tests/cpu_ref.h:27-46."""
    a, pa = _c(np.ravel(a), np.float32)
    b, pb = _c(np.ravel(b), np.float32)
    assert a.size == b.size
    mx, rel = C.c_double(), C.c_double()
    lib().orc_diff(pa, pb, a.size, C.byref(mx), C.byref(rel))
    return mx.value, rel.value


def moe_route(logits, k: int):
    """Top-k (ties to the lower id) + softmax over the k: ids int32 [T,k], w fp32 [T,k]."""
    logits, pl = _c(np.atleast_2d(logits), np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib().orc_moe_route(pl, T, E, k, ids.ctypes.data, w.ctypes.data)
    return ids, w


def moe_ffn(slots, x, ids, weights) -> np.ndarray:
    """slots: apex_amd.synth.ExpertSlots; x fp32 [T,H]; ids/weights [T,k] -> fp32 [T,H]."""
    data, pd = _c(slots.data, np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    ids, pi = _c(ids, np.int32)
    w, pw = _c(weights, np.float32)
    o = slots.offsets
    lay = ExpertLayout(slots.stride, o["gate_w"], o["gate_s"], o["up_w"], o["up_s"],
                       o["down_w"], o["down_s"])
    T, k = ids.shape
    y = np.empty((T, slots.H), np.float32)
    lib().orc_moe_ffn(pd, C.byref(lay), px, pi, pw, y.ctypes.data, T, k, slots.H, slots.I)
    return y


def e4m3_from_float(v: float) -> int:
    return lib().orc_e4m3_from_float(v)


def bf16_to_float(b: int) -> float:
    return lib().orc_bf16_to_float(b)


def float_to_bf16(f: float) -> int:
    return lib().orc_float_to_bf16(f)


def rms_norm(x, w_bf16, eps: float) -> np.ndarray:
    """RMSNorm of every row of x [rows, n] fp32 with bf16 weights [n]."""
    x, px = _c(np.atleast_2d(x), np.float32)
    w, pw = _c(w_bf16, np.uint16)
    y = np.empty_like(x)
    lib().orc_rms_norm(px, pw, y.ctypes.data, x.shape[0], x.shape[1], eps)
    return y


def moe_router_logits(h, norm_w, qw, qs, qb, eps: float) -> np.ndarray:
    """Router logits fp32 [T, E] (orc_moe_router_logits_q8)."""
    h, ph = _c(np.atleast_2d(h), np.float32)
    nw, pnw = _c(norm_w, np.uint16)
    qw, pqw = _c(qw, np.uint32)
    qs, pqs = _c(qs, np.uint16)
    qb, pqb = _c(qb, np.uint16)
    T, H = h.shape
    E = qw.shape[0]
    out = np.empty((T, E), np.float32)
    lib().orc_moe_router_logits_q8(ph, pnw, eps, pqw, pqs, pqb, T, E, H, out.ctypes.data)
    return out


def head_norm_rope(x, w_bf16, rope_pairs: int, rope_base: float, abs_pos: int, eps: float,
                   has_weight: bool = True, out_token_stride=None, out_head_stride=None,
                   out_size=None) -> np.ndarray:
    """x [tokens, heads, head_dim] fp32 -> flat fp32 output laid out by the strides
    (default: dense [tokens, heads, head_dim])."""
    x, px = _c(x, np.float32)
    T, Hh, D = x.shape
    ots = Hh * D if out_token_stride is None else out_token_stride
    ohs = D if out_head_stride is None else out_head_stride
    n = out_size if out_size is not None else (T - 1) * ots + (Hh - 1) * ohs + D
    y = np.zeros(n, np.float32)
    w, pw = _c(w_bf16 if w_bf16 is not None else np.zeros(D, np.uint16), np.uint16)
    lib().orc_head_norm_rope(px, pw, 1 if has_weight else 0, y.ctypes.data, T, Hh, D, rope_pairs,
                             rope_base, abs_pos, ots, ohs, eps)
    return y


# ---- the reference's own CPU code, compiled from its sources (where available) ----

def ref_available() -> bool:
    return REF_PATH.exists()


def ref():
    """ctypes handle on oracle/_ref/libapexref.so (built from src/nvfp4.h, src/tests/cpu_ref.h)."""
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise ImportError(f"{REF_PATH} missing (reference not mounted when built)")
        R = C.CDLL(str(REF_PATH))
        R.ref_e2m1_to_float.restype = _F
        R.ref_e2m1_to_float.argtypes = [C.c_uint32]
        R.ref_e4m3_to_float.restype = _F
        R.ref_e4m3_to_float.argtypes = [C.c_uint8]
        R.ref_decode_row.argtypes = [_P, _P, _P, _SZ]
        R.ref_matvec_nvfp4.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ]
        R.ref_gelu_tanh.restype = _F
        R.ref_gelu_tanh.argtypes = [_F]
        R.ref_diff.argtypes = [_P, _P, _SZ, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        R.ref_rms_norm.argtypes = [_P, _P, _P, _SZ, _F]
        R.ref_geglu.argtypes = [_P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ]
        R.ref_moe_ffn.argtypes = [_P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _SZ, _SZ,
                                  _SZ, _SZ, _SZ]
        _ref = R
    return _ref


def ref_matvec(codes, scales, x) -> np.ndarray:
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    rows, K = codes.shape[0], codes.shape[1] * 8
    out = np.empty((x.shape[0], rows), np.float32)
    ref().ref_matvec_nvfp4(pc, ps, px, out.ctypes.data, x.shape[0], rows, K)
    return out


def ref_decode(codes, scales) -> np.ndarray:
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint8)
    rows, K = codes.shape[0], codes.shape[1] * 8
    out = np.empty((rows, K), np.float32)
    for r in range(rows):
        ref().ref_decode_row(pc + r * K // 2, ps + r * K // 16, out[r].ctypes.data, K)
    return out


def ref_rms_norm(x, w_bf16, eps: float) -> np.ndarray:
    """The reference's rmsNormCpu (src/tests/cpu_ref.h:10-22), row by row."""
    x, px = _c(np.atleast_2d(x), np.float32)
    w, pw = _c(w_bf16, np.uint16)
    y = np.empty_like(x)
    n = x.shape[1]
    for r in range(x.shape[0]):
        ref().ref_rms_norm(px + r * n * 4, pw, y[r].ctypes.data, n, eps)
    return y


def ref_geglu(gate, up, x) -> np.ndarray:
    """gelu_tanh(Wg x) * (Wu x) with the reference's matvecNvfp4Cpu and geluTanh;
    gate/up are (codes, scales) pairs, x fp32 [T, K] -> fp32 [T, rows]."""
    gc, pgc = _c(gate[0], np.uint32)
    gs, pgs = _c(gate[1], np.uint8)
    uc, puc = _c(up[0], np.uint32)
    us, pus = _c(up[1], np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    rows, K = gc.shape[0], gc.shape[1] * 8
    out = np.empty((x.shape[0], rows), np.float32)
    ref().ref_geglu(pgc, pgs, puc, pus, px, out.ctypes.data, x.shape[0], rows, K)
    return out


def ref_moe_ffn(slots, x, ids, weights, experts: int) -> np.ndarray:
    """The MoE expert FFN with the reference's CPU functions (tokens grouped per expert);
    slots: apex_amd.synth.ExpertSlots, x fp32 [T, H], ids / weights [T, k] -> fp32 [T, H]."""
    data, pd = _c(slots.data, np.uint8)
    x, px = _c(np.atleast_2d(x), np.float32)
    ids, pi = _c(ids, np.int32)
    w, pw = _c(weights, np.float32)
    o = slots.offsets
    T, k = ids.shape
    y = np.empty((T, slots.H), np.float32)
    ref().ref_moe_ffn(pd, slots.stride, o["gate_w"], o["gate_s"], o["up_w"], o["up_s"],
                      o["down_w"], o["down_s"], px, pi, pw, y.ctypes.data, T, k, experts,
                      slots.H, slots.I)
    return y
