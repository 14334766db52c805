"""CPU checks of the C ABI: the library loads, exports every symbol include/apex_hip.h
declares, and its kernel registry rejects malformed runs (src/backend/metal_backend.cpp
error behaviour) before anything touches a GPU."""
import ctypes as C
import re
from pathlib import Path

import pytest

from apex_amd import hip

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "apex_hip.h"

E_OK, E_INVALID, E_UNKNOWN_KERNEL, E_ARGS = 0, 1, 2, 3
E_THREADGROUP = 7


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(apex_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def header_constant(name):
    m = re.search(rf"(?:#define\s+{name}\s+|\b{name}\s*=\s*)(-?\d+)", HEADER.read_text())
    return int(m.group(1))


def test_library_exports_every_declared_function():
    lib = C.CDLL(str(hip.LIB_PATH))
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a prototype for each of them
    assert sorted(hip.exported_symbols()) == names


def test_error_codes_match_header():
    assert header_constant("APEX_HIP_OK") == E_OK
    assert header_constant("APEX_HIP_E_INVALID") == E_INVALID
    assert header_constant("APEX_HIP_E_UNKNOWN_KERNEL") == E_UNKNOWN_KERNEL
    assert header_constant("APEX_HIP_E_ARGS") == E_ARGS
    assert header_constant("APEX_HIP_E_THREADGROUP") == E_THREADGROUP


def test_abi_version():
    assert hip.lib().apex_hip_abi_version() == header_constant("APEX_HIP_ABI_VERSION")


EXPECTED = {
    "matmul_nvfp4": "BBBBUU",
    "geglu_f32": "BBBU",
    "matmul_nvfp4_bf16": "BBBBUUUF",
    "geglu_nvfp4_f32": "BBBBBBUUUFF",
    "geglu_nvfp4_bf16": "BBBBBBUUUFF",
    "geglu_nvfp4_rms_norm_f32": "BBBBBBBUUUFFF",
    "gemm_nvfp4_bf16": "BBBBUUUF",
    "dequant_nvfp4_f32": "BBBUUF",
    "dequant_nvfp4_bf16": "BBBUUF",
    "rms_norm_f32": "BBBUF",
    "head_norm_rope_f32": "BBBUUUUFUUUF",
    "moe_router_logits_q8_f32": "BBBBBBUUUF",
    "moe_route_f32": "BBBBUUUU",
    "moe_ffn_f32logits_nvfp4_bf16": "BBBBBBUUUUUUUUUUUUU",
}


def test_registry_names_and_signatures():
    names = hip.kernel_names()
    for k, sig in EXPECTED.items():
        assert k in names
        assert hip.kernel_signature(k) == sig
    assert hip.kernel_signature("no_such_kernel") is None
    # every registered name is documented in the header
    text = HEADER.read_text()
    for k in names:
        assert f"`{k}`" in text or f" {k} " in text or f"{k}:" in text or k in text


class FakeArray:
    """A non-null device address for host-side validation paths that fail first."""
    ptr = 0x1000


class FakeBuffer:
    """validate_run never dereferences a buffer handle: any non-null value works."""
    handle = 0x1000


def buf(off=0):
    return ("buf", FakeBuffer(), off)


def u32(v):
    return ("val", C.c_uint32(v))


def f32(v):
    return ("val", C.c_float(v))


def matmul_args():
    return [buf(), buf(), buf(), buf(), u32(2048), u32(2048)]


def rc_of(fn):
    try:
        fn()
        return E_OK
    except hip.ApexHipError as e:
        return e.code


def test_validate_accepts_the_reference_launch():
    # src/ops.h:36-45: grid {ceil(rows/8), tokens}, 256 threads
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args(), (256, 1), (256,))) == 0
    assert rc_of(lambda: hip.validate_run("geglu_f32", [buf(), buf(), buf(), u32(10)],
                                          (1,), (256,))) == 0


def test_validate_unknown_kernel():
    rc = rc_of(lambda: hip.validate_run("attention_f32", matmul_args()))
    assert rc == E_UNKNOWN_KERNEL
    assert "attention_f32" in hip.lib().apex_hip_last_error().decode()


def test_validate_accepts_the_reference_norm_launches():
    # src/ops.h:18-26: Dim3{rows}, 256 threads; src/ops.h:88-118: Dim3{tokens, heads}
    assert rc_of(lambda: hip.validate_run("rms_norm_f32", [buf(), buf(), buf(), u32(2816),
                                                           f32(1e-6)], (4,), (256,))) == 0
    args = [buf(), buf(), buf(), u32(8), u32(256), u32(1), u32(128), f32(1e4), u32(0),
            u32(2048), u32(256), f32(1e-6)]
    assert rc_of(lambda: hip.validate_run("head_norm_rope_f32", args, (3, 8), (256,))) == 0


def test_head_norm_rope_shape_errors_are_host_checks():
    """Invalid head shapes are rejected before any device work (no GPU needed)."""
    fake = FakeArray()
    for head_dim, pairs in ((255, 0), (1024, 0), (256, 129)):
        rc = rc_of(lambda: hip.head_norm_rope_f32(fake, fake, fake, 1, 1, head_dim, pairs, 1e4,
                                                  0, head_dim, head_dim, 1e-6))
        assert rc == E_INVALID, (head_dim, pairs)


def test_validate_wrong_arg_count():
    rc = rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args()[:5]))
    assert rc == E_ARGS
    assert "expected 6" in hip.lib().apex_hip_last_error().decode()


def test_validate_wrong_arg_kind():
    a = matmul_args()
    a[1] = u32(3)  # a value where a buffer belongs
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", a)) == E_ARGS
    a = matmul_args()
    a[4] = buf()  # a buffer where a value belongs
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", a)) == E_ARGS
    a = matmul_args()
    a[5] = ("val", C.c_uint64(3))  # an 8-byte value
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", a)) == E_ARGS
    a = matmul_args()
    a[0] = ("buf", None, 0)  # a null buffer
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", a)) == E_ARGS


def test_validate_threadgroup_limits():
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args(), (1,), (2048,))) == \
        E_THREADGROUP
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args(), (1,), (32, 32, 2))) == \
        E_THREADGROUP
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args(), (0,), (256,))) == \
        E_INVALID
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4", matmul_args(), (1,), (32, 32))) == 0


def test_validate_bf16_signature():
    a = [buf(), buf(), buf(), buf(), u32(1), u32(64), u32(64), f32(1.0)]
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4_bf16", a)) == 0
    a[7] = u32(1)  # U and F are both 4-byte values: the kind check is on size only
    assert rc_of(lambda: hip.validate_run("matmul_nvfp4_bf16", a)) == 0


def test_null_out_pointers_are_rejected():
    L = hip.lib()
    assert L.apex_hip_backend_create(0, None) != 0
    assert L.apex_hip_device_count(None) != 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """The product path has no fallback: without the built library every op raises."""
    monkeypatch.setattr(hip, "LIB_PATH", tmp_path / "libapex_hip.so")
    monkeypatch.setattr(hip, "_lib", None)
    with pytest.raises(ImportError):
        hip.lib()


def test_gemm_tail_plan_covers_and_fits():
    """The MFMA GEMM's cover of C on 256 CUs (host logic, no device): whole tiles for the
    first nf n-tiles; past them either narrow tiles of nt (1 or 2; GeGLU 2) 32-row W
    blocks or ns short tiles (full width, at most 6 32-row blocks of one tail column).
    Whenever narrow tiles are used they cover every column, fit in the CUs left by the
    whole tiles' rounds plus one, and no narrower width would fit; short tiles only when
    no narrow width fits, one per CU left, none empty.  The benchmark's GeGLU shape takes
    2-block narrow tiles, its plain shape short tiles."""
    ncu = 256
    assert hip.gemm_tail_plan(2048, 21504, False, ncu) == (64, 0, 256)
    assert hip.gemm_tail_plan(2048, 21504, True, ncu) == (160, 2, 0)
    assert hip.gemm_tail_plan(256, 76800, False, ncu) == (256, 2, 0)
    assert hip.gemm_tail_plan(2048, 16384, False, ncu) == (64, 0, 0)  # exactly 2 rounds
    assert hip.gemm_tail_plan(256, 256 * 200, False, ncu) == (200, 0, 0)  # one round
    assert hip.gemm_tail_plan(30, 102187, False, ncu) == (256, 0, 144)  # one block per tail column
    rng = __import__("numpy").random.default_rng(5)
    used = short = 0
    for _ in range(400):
        M, N = int(rng.integers(1, 5000)), int(rng.integers(1, 200000))
        for geglu in (False, True):
            tn = 128 if geglu else 256
            tm, tiles_n = -(-M // 256), -(-N // tn)
            nf, nt, ns = hip.gemm_tail_plan(M, N, geglu, ncu)
            if nt == 0 and ns == 0:
                assert nf == tiles_n
                continue
            assert nt == 0 or ns == 0
            R = tm * tiles_n // ncu
            slots = (R + 1) * ncu - tm * nf
            assert 0 < nf < tiles_n and tm * nf <= R * ncu
            if ns:
                short += 1
                C, B = -(-(N - nf * tn) // tn), -(-M // 32)
                assert C <= ns <= min(slots, C * B)
                assert -(-B // (ns // C)) <= 6
                continue
            used += 1
            assert nt == 2 if geglu else 1 <= nt <= 2
            tc = (16 if geglu else 32) * nt
            assert tm * -(-(N - nf * tn) // tc) <= slots
            if nt > (2 if geglu else 1):
                tc1 = (16 if geglu else 32) * (nt - (2 if geglu else 1))
                assert tm * -(-(N - nf * tn) // tc1) > slots
    assert used > 20 and short > 20
    with pytest.raises(hip.ApexHipError):
        hip.gemm_tail_plan(0, 5, False, ncu)
