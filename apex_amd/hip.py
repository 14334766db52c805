"""ctypes binding of the C ABI in include/apex_hip.h (libapex_hip.so).

Python is test and benchmark plumbing here; the product is the HIP library and the
C++ host layer.  Nothing in this module computes on the CPU: every op is a call into
the HIP library, and importing an op without the built library raises.

Two ways in, mirroring the C ABI:
  * Backend / Buffer: the reference's Backend interface (src/backend/backend.h:39-63)
    -- allocate, wrap_no_copy, contents, release, run(kernel, args, grid, block), sync.
  * DeviceArray + the functions at the bottom: direct entry points on device memory.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libapex_hip.so"

_lib = None


class ApexHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"apex_hip error {code}: {msg}")
        self.code = code


class Arg(C.Structure):
    _fields_ = [("buffer", C.c_void_p), ("offset", C.c_size_t), ("bytes", C.c_void_p),
                ("size", C.c_size_t)]


class Dim3(C.Structure):
    _fields_ = [("x", C.c_uint32), ("y", C.c_uint32), ("z", C.c_uint32)]


def dim3(x, y=1, z=1) -> Dim3:
    return Dim3(x, y, z)


_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float
_SZ = C.c_size_t
_I = C.c_int

_PROTOS = {
    "apex_hip_last_error": (C.c_char_p, []),
    "apex_hip_abi_version": (_I, []),
    "apex_hip_backend_create": (_I, [_I, C.POINTER(_P)]),
    "apex_hip_backend_destroy": (None, [_P]),
    "apex_hip_device_name": (_I, [_P, C.c_char_p, _SZ]),
    "apex_hip_wrap_no_copy": (_I, [_P, _P, _SZ, C.POINTER(_P)]),
    "apex_hip_allocate": (_I, [_P, _SZ, C.c_char_p, C.POINTER(_P)]),
    "apex_hip_contents": (_I, [_P, _P, C.POINTER(_P)]),
    "apex_hip_release": (_I, [_P, _P]),
    "apex_hip_run": (_I, [_P, C.c_char_p, C.POINTER(Arg), _SZ, Dim3, Dim3]),
    "apex_hip_sync": (_I, [_P]),
    "apex_hip_buffer_device_ptr": (_I, [_P, C.POINTER(_P)]),
    "apex_hip_buffer_length": (_SZ, [_P]),
    "apex_hip_backend_stream": (_P, [_P]),
    "apex_hip_kernel_count": (_I, []),
    "apex_hip_kernel_name": (C.c_char_p, [_I]),
    "apex_hip_kernel_signature": (C.c_char_p, [C.c_char_p]),
    "apex_hip_validate_run": (_I, [C.c_char_p, C.POINTER(Arg), _SZ, Dim3, Dim3]),
    "apex_nvfp4_matmul_f32": (_I, [_P, _P, _P, _F, _P, _U32, _U32, _U32, _P]),
    "apex_nvfp4_matmul_bf16": (_I, [_P, _P, _P, _F, _P, _U32, _U32, _U32, _P]),
    "apex_nvfp4_gemm_bf16": (_I, [_P, _P, _P, _F, _P, _U32, _U32, _U32, _P]),
    "apex_nvfp4_geglu_f32": (_I, [_P, _P, _P, _F, _P, _P, _F, _P, _U32, _U32, _U32, _P]),
    "apex_nvfp4_geglu_bf16": (_I, [_P, _P, _P, _F, _P, _P, _F, _P, _U32, _U32, _U32, _P]),
    "apex_nvfp4_geglu_rms_norm_f32": (_I, [_P, _P, _F, _P, _P, _F, _P, _P, _F, _P, _U32, _U32,
                                           _U32, _P]),
    "apex_geglu_f32": (_I, [_P, _P, _P, _U32, _P]),
    "apex_nvfp4_dequant_f32": (_I, [_P, _P, _F, _P, _U32, _U32, _P]),
    "apex_nvfp4_dequant_bf16": (_I, [_P, _P, _F, _P, _U32, _U32, _P]),
    "apex_hip_device_count": (_I, [C.POINTER(_I)]),
    "apex_hip_set_device": (_I, [_I]),
    "apex_hip_malloc": (_I, [_SZ, C.POINTER(_P)]),
    "apex_hip_free": (_I, [_P]),
    "apex_hip_memcpy_h2d": (_I, [_P, _P, _SZ]),
    "apex_hip_memcpy_d2h": (_I, [_P, _P, _SZ]),
    "apex_hip_memcpy_d2d": (_I, [_P, _P, _SZ]),
    "apex_hip_memset": (_I, [_P, _I, _SZ]),
    "apex_hip_mem_info": (_I, [_P, _P]),
    "apex_hip_device_synchronize": (_I, []),
    "apex_hip_stream_create": (_I, [C.POINTER(_P)]),
    "apex_hip_stream_destroy": (_I, [_P]),
    "apex_hip_stream_synchronize": (_I, [_P]),
    "apex_hip_event_create": (_I, [C.POINTER(_P)]),
    "apex_hip_event_destroy": (_I, [_P]),
    "apex_hip_event_record": (_I, [_P, _P]),
    "apex_hip_event_synchronize": (_I, [_P]),
    "apex_hip_event_elapsed_ms": (_I, [_P, _P, C.POINTER(_F)]),
    "apex_hip_read_probe": (_I, [_P, _SZ, _P, _P]),
    "apex_hip_read_probe_sink_words": (_I, []),
    "apex_hip_set_gemv_waves_per_cu": (_I, [_I]),
    "apex_hip_set_gemm_min_tokens": (_I, [_U32, _U32]),
    "apex_hip_dense_dispatch_counts": (_I, [_P]),
    "apex_hip_gemm_tail_plan": (_I, [_U32, _U32, _I, _U32, _P]),
    "apex_moe_route_bf16": (_I, [_P, _U32, _U32, _U32, _P, _P, _P]),
    "apex_moe_workspace_bytes": (_SZ, [_U32, _U32, _U32, _U32, _U32]),
    "apex_moe_workspace_plan_offset": (_SZ, [_U32, _U32, _U32, _U32, _U32]),
    "apex_moe_ffn_bf16": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _SZ, _P]),
    "apex_hip_set_moe_path": (_I, [_I]),
    "apex_moe_ffn_bf16_noalloc": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P]),
    "apex_rms_norm_f32": (_I, [_P, _P, _P, _U32, _U32, _F, _P]),
    "apex_file_to_device": (_I, [C.c_char_p, _U64, _U64, _P, _U64, _U32, _P]),
    "apex_experts_to_device": (_I, [C.c_char_p, _U64, _U64, _P, _U32, _P, _U64, _U64, _U32, _P]),
    "apex_hip_load_file": (_I, [_P, _P, _U64, C.c_char_p, _U64, _U64]),
    "apex_moe_router_logits_q8": (_I, [_P, _P, _F, _P, _P, _P, _U32, _U32, _U32, _P, _P]),
    "apex_moe_route_f32": (_I, [_P, _P, _U32, _U32, _U32, _P, _P, _P]),
    "apex_moe_ffn_f32logits_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P,
                                         _SZ, _P]),
    "apex_head_norm_rope_f32": (_I, [_P, _P, _I, _P, _U32, _U32, _U32, _U32, _F, _U32, _U32, _U32,
                                     _F, _P]),
}


def lib():
    """Load libapex_hip.so (raises if it has not been built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: run `python -m apex_amd.build` first")
        L = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in _PROTOS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_PROTOS)


def check(rc: int) -> None:
    if rc != 0:
        raise ApexHipError(rc, lib().apex_hip_last_error().decode())


def device_count() -> int:
    n = C.c_int(0)
    check(lib().apex_hip_device_count(C.byref(n)))
    return n.value


def set_device(device: int) -> None:
    check(lib().apex_hip_set_device(device))


# ---------------------------------------------------------------------------------
# Device memory and timing plumbing
# ---------------------------------------------------------------------------------

class DeviceArray:
    """A device allocation with a numpy dtype/shape, freed on close() or GC."""

    def __init__(self, shape, dtype):
        self.shape = tuple(np.atleast_1d(np.asarray(shape, dtype=np.int64)).tolist())
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().apex_hip_malloc(self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(lib().apex_hip_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().apex_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def copy_from(self, other: "DeviceArray") -> None:
        assert other.nbytes == self.nbytes
        check(lib().apex_hip_memcpy_d2d(self.ptr, other.ptr, self.nbytes))

    def fill_bytes(self, value: int) -> None:
        check(lib().apex_hip_memset(self.ptr, value, self.nbytes))

    def close(self) -> None:
        if getattr(self, "ptr", 0):
            lib().apex_hip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = C.c_void_p()
        check(lib().apex_hip_stream_create(C.byref(p)))
        self.handle = p.value

    def synchronize(self):
        check(lib().apex_hip_stream_synchronize(self.handle))

    def close(self):
        if self.handle:
            lib().apex_hip_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(lib().apex_hip_event_create(C.byref(p)))
        self.handle = p.value

    def record(self, stream=None):
        check(lib().apex_hip_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self):
        check(lib().apex_hip_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().apex_hip_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def close(self):
        if self.handle:
            lib().apex_hip_event_destroy(self.handle)
            self.handle = None


def mem_info() -> tuple:
    """(free, total) bytes of the current device."""
    free, total = C.c_size_t(0), C.c_size_t(0)
    check(lib().apex_hip_mem_info(C.byref(free), C.byref(total)))
    return free.value, total.value


def synchronize():
    check(lib().apex_hip_device_synchronize())


def _s(stream):
    return stream.handle if stream is not None else None


# ---------------------------------------------------------------------------------
# Direct entry points (device pointers)
# ---------------------------------------------------------------------------------

def nvfp4_matmul_f32(x, codes, scales, out, tokens, rows, K, tensor_scale=1.0, stream=None):
    check(lib().apex_nvfp4_matmul_f32(x.ptr, codes.ptr, scales.ptr, tensor_scale, out.ptr,
                                      tokens, rows, K, _s(stream)))


def nvfp4_matmul_bf16(x, codes, scales, out, tokens, rows, K, tensor_scale=1.0, stream=None):
    check(lib().apex_nvfp4_matmul_bf16(x.ptr, codes.ptr, scales.ptr, tensor_scale, out.ptr,
                                       tokens, rows, K, _s(stream)))


def nvfp4_gemm_bf16(A, codes, scales, C, M, N, K, tensor_scale=1.0, stream=None):
    check(lib().apex_nvfp4_gemm_bf16(A.ptr, codes.ptr, scales.ptr, tensor_scale, C.ptr, M, N, K,
                                     _s(stream)))


def nvfp4_geglu_f32(x, gc, gs, uc, us, out, tokens, rows, K, gate_scale=1.0, up_scale=1.0,
                    stream=None):
    check(lib().apex_nvfp4_geglu_f32(x.ptr, gc.ptr, gs.ptr, gate_scale, uc.ptr, us.ptr, up_scale,
                                     out.ptr, tokens, rows, K, _s(stream)))


def nvfp4_geglu_rms_norm_f32(x, norm_w, eps, gc, gs, uc, us, out, tokens, rows, K,
                             gate_scale=1.0, up_scale=1.0, stream=None):
    """rms_norm_f32 of each x row (bf16 weights norm_w [K]) fused into the fp32 GeGLU GEMV."""
    check(lib().apex_nvfp4_geglu_rms_norm_f32(x.ptr, norm_w.ptr, eps, gc.ptr, gs.ptr, gate_scale,
                                              uc.ptr, us.ptr, up_scale, out.ptr, tokens, rows, K,
                                              _s(stream)))


def nvfp4_geglu_bf16(x, gc, gs, uc, us, out, tokens, rows, K, gate_scale=1.0, up_scale=1.0,
                     stream=None):
    check(lib().apex_nvfp4_geglu_bf16(x.ptr, gc.ptr, gs.ptr, gate_scale, uc.ptr, us.ptr, up_scale,
                                      out.ptr, tokens, rows, K, _s(stream)))


def geglu_f32(gate, up, out, count, stream=None):
    check(lib().apex_geglu_f32(gate.ptr, up.ptr, out.ptr, count, _s(stream)))


def nvfp4_dequant(codes, scales, out, rows, K, tensor_scale=1.0, stream=None):
    f = lib().apex_nvfp4_dequant_bf16 if out.dtype == np.uint16 else lib().apex_nvfp4_dequant_f32
    check(f(codes.ptr, scales.ptr, tensor_scale, out.ptr, rows, K, _s(stream)))


def rms_norm_f32(x, w, y, rows, hidden_dim, eps, stream=None):
    check(lib().apex_rms_norm_f32(x.ptr, w.ptr, y.ptr, rows, hidden_dim, eps, _s(stream)))


def head_norm_rope_f32(x, w, y, tokens, heads, head_dim, rope_pairs, rope_base, abs_pos,
                       out_token_stride, out_head_stride, eps, has_weights=True, stream=None):
    check(lib().apex_head_norm_rope_f32(x.ptr, w.ptr if w is not None else None,
                                        1 if has_weights else 0, y.ptr, tokens, heads, head_dim,
                                        rope_pairs, rope_base, abs_pos, out_token_stride,
                                        out_head_stride, eps, _s(stream)))


def file_to_device(path, file_offset, nbytes, dst, dst_offset=0, chunk_bytes=0, n_buffers=0,
                   stream=None):
    check(lib().apex_file_to_device(str(path).encode(), file_offset, nbytes, dst.ptr + dst_offset,
                                    chunk_bytes, n_buffers, _s(stream)))


def experts_to_device(path, stride, slot_bytes, experts, dst, dst_stride, chunk_bytes=0,
                      n_buffers=0, stream=None):
    ids = np.ascontiguousarray(experts, np.int32)
    check(lib().apex_experts_to_device(str(path).encode(), stride, slot_bytes, ids.ctypes.data,
                                       len(ids), dst.ptr, dst_stride, chunk_bytes, n_buffers,
                                       _s(stream)))


def read_probe(buf, sink, stream=None) -> None:
    check(lib().apex_hip_read_probe(buf.ptr, buf.nbytes, sink.ptr, _s(stream)))


def read_probe_sink_words() -> int:
    return lib().apex_hip_read_probe_sink_words()


def set_gemv_waves_per_cu(waves: int) -> None:
    check(lib().apex_hip_set_gemv_waves_per_cu(waves))


def set_gemm_min_tokens(bf16_tokens: int = 0, f32_tokens: int = 0) -> None:
    """Tokens from which the dense matmul / GeGLU run as MFMA GEMMs (0: by size)."""
    check(lib().apex_hip_set_gemm_min_tokens(bf16_tokens, f32_tokens))


def dense_dispatch_counts() -> dict:
    """Dense-product launches of this process so far, by form."""
    c = (C.c_uint64 * 4)()
    check(lib().apex_hip_dense_dispatch_counts(C.cast(c, C.c_void_p)))
    return {"gemv": c[0], "gemm": c[1], "splitk_gemm": c[2], "f32_split": c[3]}


def gemm_tail_plan(m: int, n: int, geglu: bool = False, ncu: int = 0) -> tuple:
    """(whole n-tiles, narrow-tile W blocks, short tiles) of the MFMA GEMM's cover of an
    m x n output on ncu CUs (0: the current device's); narrow and short 0: whole tiles
    only."""
    out = (C.c_uint32 * 3)()
    check(lib().apex_hip_gemm_tail_plan(m, n, int(geglu), ncu, C.cast(out, C.c_void_p)))
    return out[0], out[1], out[2]


# ---- MoE expert FFN --------------------------------------------------------------

class MoeSlots(C.Structure):
    """apex_moe_slots: expert e's pieces at base + e * stride + offset."""
    _fields_ = [("base", C.c_void_p), ("stride", C.c_uint64), ("gate_w", C.c_uint64),
                ("gate_s", C.c_uint64), ("up_w", C.c_uint64), ("up_s", C.c_uint64),
                ("down_w", C.c_uint64), ("down_s", C.c_uint64)]


def moe_slots(base: DeviceArray, stride: int, offsets: dict) -> MoeSlots:
    o = offsets
    return MoeSlots(base.ptr, stride, o["gate_w"], o["gate_s"], o["up_w"], o["up_s"],
                    o["down_w"], o["down_s"])


def moe_route_bf16(logits, ids, weights, tokens, experts, top_k, stream=None):
    check(lib().apex_moe_route_bf16(logits.ptr, tokens, experts, top_k, ids.ptr, weights.ptr,
                                    _s(stream)))


def moe_router_logits_q8(h, norm_w, proj_w, proj_s, proj_b, logits, tokens, experts, hidden,
                         eps=1e-6, stream=None):
    check(lib().apex_moe_router_logits_q8(h.ptr, norm_w.ptr, eps, proj_w.ptr, proj_s.ptr,
                                          proj_b.ptr, tokens, experts, hidden, logits.ptr,
                                          _s(stream)))


def moe_route_f32(logits, per_expert_scale, ids, weights, tokens, experts, top_k, stream=None):
    check(lib().apex_moe_route_f32(logits.ptr, per_expert_scale.ptr if per_expert_scale is not None
                                   else None, tokens, experts, top_k, ids.ptr, weights.ptr,
                                   _s(stream)))


def moe_ffn_f32logits_bf16(x, logits, per_expert_scale, slots: "MoeSlots", y, tokens, experts,
                           top_k, hidden, inter, workspace, stream=None):
    check(lib().apex_moe_ffn_f32logits_bf16(
        x.ptr, logits.ptr, per_expert_scale.ptr if per_expert_scale is not None else None,
        C.byref(slots), y.ptr, tokens, experts, top_k, hidden, inter, workspace.ptr,
        workspace.nbytes, _s(stream)))


def moe_workspace_bytes(tokens, experts, top_k, hidden, inter) -> int:
    return lib().apex_moe_workspace_bytes(tokens, experts, top_k, hidden, inter)


def moe_workspace_plan(workspace, tokens, experts, top_k, hidden, inter) -> dict:
    """The grouping plan apex_moe_ffn_bf16 left in `workspace` (apex_moe_workspace_plan_offset):
    counts, offsets, active experts and both pair <-> position maps, as numpy arrays."""
    off = lib().apex_moe_workspace_plan_offset(tokens, experts, top_k, hidden, inter)
    E, P = experts, tokens * top_k
    words = workspace.numpy()[off:off + 4 * (16 + 3 * E + 1 + 2 * P)].view(np.int32)
    hdr, rest = words[:16], words[16:]
    cnt, rest = rest[:E], rest[E:]
    offs, rest = rest[:E + 1], rest[E + 1:]
    act, rest = rest[:E], rest[E:]
    return {"active": int(hdr[0]), "cnt": cnt.copy(), "off": offs.copy(), "act": act[:hdr[0]].copy(),
            "pos_of_pair": rest[:P].copy(), "pair_of_pos": rest[P:2 * P].copy()}


def moe_ffn_bf16(x, logits, slots: MoeSlots, y, tokens, experts, top_k, hidden, inter, workspace,
                 stream=None):
    check(lib().apex_moe_ffn_bf16(x.ptr, logits.ptr, C.byref(slots), y.ptr, tokens, experts,
                                  top_k, hidden, inter, workspace.ptr, workspace.nbytes,
                                  _s(stream)))


def moe_ffn_bf16_noalloc(x, logits, slots: MoeSlots, y, tokens, experts, top_k, hidden, inter,
                         stream=None):
    """apex_moe_ffn_bf16's decode path on the library's fixed workspace (no allocation)."""
    check(lib().apex_moe_ffn_bf16_noalloc(x.ptr, logits.ptr, C.byref(slots), y.ptr, tokens, experts,
                                          top_k, hidden, inter, _s(stream)))


def set_moe_path(path: int) -> None:
    """0 by size (default), 1 grouped GEMV, 2 grouped GEMM."""
    check(lib().apex_hip_set_moe_path(path))


def moe_forward(x, logits, slots, top_k=8):
    """Host convenience: numpy bf16 x [T,H], logits [T,E], apex_amd.synth.ExpertSlots ->
    numpy bf16 y [T,H], computed by apex_moe_ffn_bf16 on the current device."""
    T, H = x.shape
    E = logits.shape[1]
    dx, dl = DeviceArray.from_numpy(x), DeviceArray.from_numpy(logits)
    ds = DeviceArray.from_numpy(slots.data)
    y = DeviceArray((T, H), np.uint16)
    ws = DeviceArray((moe_workspace_bytes(T, E, top_k, H, slots.I),), np.uint8)
    moe_ffn_bf16(dx, dl, moe_slots(ds, slots.stride, slots.offsets), y, T, E, top_k, H, slots.I, ws)
    synchronize()
    return y.numpy()


# ---------------------------------------------------------------------------------
# Backend interface (src/backend/backend.h:39-63)
# ---------------------------------------------------------------------------------

class Buffer:
    def __init__(self, backend: "Backend", handle: int, nbytes: int):
        self.backend = backend
        self.handle = handle
        self.nbytes = nbytes

    @property
    def device_ptr(self) -> int:
        p = C.c_void_p()
        check(lib().apex_hip_buffer_device_ptr(self.handle, C.byref(p)))
        return p.value or 0


def buf(b: Buffer, offset: int = 0):
    """Arg::buf (backend.h:21-23)."""
    return ("buf", b, offset)


def u32(v: int):
    """Arg::val with a uint32_t (backend.h:24-27)."""
    return ("val", C.c_uint32(v))


def f32(v: float):
    """Arg::val with a float."""
    return ("val", C.c_float(v))


def make_args(args):
    arr = (Arg * max(1, len(args)))()
    keep = []
    for i, a in enumerate(args):
        if a[0] == "buf":
            arr[i] = Arg(a[1].handle if a[1] is not None else None, a[2], None, 0)
        else:
            v = a[1]
            keep.append(v)
            arr[i] = Arg(None, 0, C.cast(C.pointer(v), C.c_void_p), C.sizeof(v))
    return arr, keep


class Backend:
    """Python mirror of apex::HipBackend, for tests written like the reference's."""

    def __init__(self, device: int = 0):
        p = C.c_void_p()
        check(lib().apex_hip_backend_create(device, C.byref(p)))
        self.handle = p.value
        self._wrapped = {}

    def device_name(self) -> str:
        b = C.create_string_buffer(256)
        check(lib().apex_hip_device_name(self.handle, b, 256))
        return b.value.decode()

    def allocate(self, nbytes: int, category: str = "scratch") -> Buffer:
        p = C.c_void_p()
        check(lib().apex_hip_allocate(self.handle, nbytes, category.encode(), C.byref(p)))
        return Buffer(self, p.value, nbytes)

    def wrap_no_copy(self, host: np.ndarray) -> Buffer:
        p = C.c_void_p()
        check(lib().apex_hip_wrap_no_copy(self.handle, host.ctypes.data, host.nbytes, C.byref(p)))
        b = Buffer(self, p.value, host.nbytes)
        self._wrapped[p.value] = host  # keep the host bytes alive
        return b

    def contents(self, b: Buffer, dtype=np.uint8, count=None) -> np.ndarray:
        p = C.c_void_p()
        check(lib().apex_hip_contents(self.handle, b.handle, C.byref(p)))
        dt = np.dtype(dtype)
        n = b.nbytes // dt.itemsize if count is None else count
        if n == 0:
            return np.empty(0, dt)
        raw = (C.c_char * (n * dt.itemsize)).from_address(p.value)
        return np.frombuffer(raw, dtype=dt, count=n)

    def load_file(self, b: Buffer, offset: int, path, file_offset: int, nbytes: int) -> None:
        check(lib().apex_hip_load_file(self.handle, b.handle, offset, str(path).encode(),
                                       file_offset, nbytes))

    def release(self, b: Buffer) -> None:
        check(lib().apex_hip_release(self.handle, b.handle))
        self._wrapped.pop(b.handle, None)
        b.handle = None

    def run(self, kernel: str, args, threadgroups, threads_per_group) -> None:
        arr, keep = make_args(args)
        check(lib().apex_hip_run(self.handle, kernel.encode(), arr, len(args),
                                 dim3(*threadgroups), dim3(*threads_per_group)))

    def sync(self) -> None:
        check(lib().apex_hip_sync(self.handle))

    @property
    def stream_handle(self):
        return lib().apex_hip_backend_stream(self.handle)

    def close(self) -> None:
        if self.handle:
            lib().apex_hip_backend_destroy(self.handle)
            self.handle = None


def validate_run(kernel: str, args, threadgroups=(1,), threads_per_group=(256,)) -> None:
    arr, keep = make_args(args)
    check(lib().apex_hip_validate_run(kernel.encode(), arr, len(args), dim3(*threadgroups),
                                      dim3(*threads_per_group)))


def kernel_names():
    L = lib()
    return [L.apex_hip_kernel_name(i).decode() for i in range(L.apex_hip_kernel_count())]


def kernel_signature(name: str):
    s = lib().apex_hip_kernel_signature(name.encode())
    return s.decode() if s else None
