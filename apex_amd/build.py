"""Build the gfx950 HIP library, the C++ host layer and the CPU oracle, in tree.

    python -m apex_amd.build            # full rebuild (what __graft_entry__.build() runs)
    python -m apex_amd.build --changed  # rebuild only units whose sources changed

Outputs (git-ignored, shipped with the tree):
    apex_amd/lib/libapex_hip.so    HIP kernels + the C ABI of include/apex_hip.h
    apex_amd/lib/libapex_host.so   C++ apex::HipBackend over that C ABI
    tests/host/test_host           C++ checks of the host layer (test infrastructure)
    oracle/liboracle.so            CPU oracle (test infrastructure)
    oracle/_ref/libapexref.so      reference CPU code, only where the reference is mounted
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "apex_amd"
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"
ORACLE = ROOT / "oracle"
REFERENCE = Path("/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-fp32 VALU forms are disabled for all device code (see DESIGN: hardware notes).
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++20", "-fPIC", "-Wall",
             "-Wno-unused-function", "-Wno-unused-variable",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", str(INCLUDE), "-I", str(CSRC)]
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-I", str(INCLUDE), "-I", str(HOST)]

HIP_UNITS = ["hip_impl.cpp", "gemv.hip", "gemv_f32.hip", "gemv_bf16_plain.hip", "moe.hip",
             "gemv_bf16_geglu.hip", "gemm.hip", "norm.hip", "file_io.cpp"]
HOST_UNITS = ["hip_backend.cpp"]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _deps(src: Path):
    return [src] + sorted(CSRC.glob("*.h")) + [INCLUDE / "apex_hip.h"]


def _stale(obj: Path, src: Path) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in _deps(src))


def _compile_hip(unit: str, changed_only: bool) -> Path:
    src = CSRC / unit
    obj = OBJ / (unit.rsplit(".", 1)[0] + ".o")
    if changed_only and not _stale(obj, src):
        return obj
    lang = ["-x", "hip"] if unit.endswith(".cpp") else []
    _run([HIPCC] + HIP_FLAGS + lang + ["-c", str(src), "-o", str(obj)])
    return obj


def build_hip(changed_only: bool = False, jobs: int | None = None) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(HIP_UNITS), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda u: _compile_hip(u, changed_only), HIP_UNITS))
    out = LIB / "libapex_hip.so"
    tmp = LIB / "libapex_hip.so.tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", str(tmp)] +
         [str(o) for o in objs])
    os.replace(tmp, out)
    return out


def build_host() -> None:
    """C++ host layer: apex::HipBackend (links only the C ABI)."""
    LIB.mkdir(parents=True, exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    _run([cxx] + CXX_FLAGS + ["-shared", "-o", str(LIB / "libapex_host.so")] +
         [str(HOST / u) for u in HOST_UNITS] + ["-L", str(LIB), "-lapex_hip",
                                                "-Wl,-rpath,$ORIGIN"])


def build_host_tests() -> None:
    """tests/host/test_host: the C++ checks of the host layer (links the oracle)."""
    src = ROOT / "tests" / "host" / "test_host.cpp"
    if not src.exists():
        return
    cxx = os.environ.get("CXX", "g++")
    _run([cxx] + CXX_FLAGS + ["-I", str(ORACLE), "-o", str(src.with_suffix("")), str(src),
                              "-L", str(LIB), "-lapex_host", "-lapex_hip", "-L", str(ORACLE),
                              "-loracle", f"-Wl,-rpath,{LIB}:{ORACLE}",
                              "-Wl,-rpath,$ORIGIN/../../apex_amd/lib:$ORIGIN/../../oracle"])


def build_oracle() -> None:
    """CPU oracle, and the reference's own CPU code when the reference is mounted."""
    _run(["make", "-s", "-C", str(ORACLE), "liboracle.so"])
    if (REFERENCE / "src" / "nvfp4.h").exists():
        _run(["make", "-s", "-C", str(ORACLE), "ref", f"REFERENCE={REFERENCE}"])


def build(changed_only: bool = False) -> None:
    if not changed_only:
        shutil.rmtree(OBJ, ignore_errors=True)
        for p in (ORACLE / "liboracle.so",):
            if p.exists():
                p.unlink()
    build_oracle()
    build_hip(changed_only)
    build_host()
    build_host_tests()


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv[1:])
    print("built", LIB / "libapex_hip.so")
