"""The C++ host layer (apex::HipBackend, ops.h) through its own C++ checks
(tests/host/test_host.cpp), reference-harness style: contents() / run / sync and rel L2
against the oracle."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "host" / "test_host"


def binary():
    if not BIN.exists():
        from apex_amd import build
        build.build_host()
        build.build_host_tests()
    return str(BIN)


def run(*args, timeout=300):
    r = subprocess.run([binary(), *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=timeout)
    print(r.stdout)
    return r


@pytest.fixture(scope="module")
def packed_dir(tmp_path_factory):
    """A small packed model directory in the repack format (2 layers, 16 experts)."""
    from apex_amd import synth
    d = tmp_path_factory.mktemp("packed")
    synth.write_packed_model(d, seed=4, layers=2, E=16, H=512, I=256)
    return str(d)


def test_host_layer_without_device(packed_dir):
    """On a machine without a GPU the backend constructor throws std::runtime_error;
    the manifest reader (ModelInfo::load) needs no device."""
    import torch  # noqa: F401  (only to mirror the environment; the check is C++)
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = run("--no-gpu", "--packed", packed_dir)
    assert r.returncode == 0, r.stdout
    assert "PASS HipBackend without a device throws" in r.stdout
    assert "PASS Profile: calls, total, shortest and longest per phase" in r.stdout
    for name in ("config and quantization", "expert slot pieces", "layer files", "core tensors",
                 "unknown tensor throws"):
        assert f"PASS manifest: {name}" in r.stdout


@pytest.mark.gpu
def test_host_layer_on_gpu(packed_dir):
    r = run("--packed", packed_dir)
    assert r.returncode == 0, r.stdout
    assert "FAIL" not in r.stdout
    for name in ("denseMlp fp32 (4 launches) vs oracle", "denseMlpFused fp32 (2 launches) vs oracle",
                 "denseMlp fp32 at 128 tokens vs oracle", "denseMlp fp32 at 512 tokens vs oracle",
                 "denseMlp at 128 tokens: matmul_nvfp4 ran 3 MFMA GEMMs",
                 "denseMlp at 512 tokens: matmul_nvfp4 ran 3 MFMA GEMMs",
                 "denseMlpFused at 512 tokens: 2 MFMA GEMMs",
                 "matmulNvfp4Bf16 T=96", "moeFfn vs oracle", "rmsNorm vs oracle",
                 "headNormRope vs oracle", "unknown kernel throws", "manifest: layer files",
                 "packed router logits vs oracle", "packed MoE block vs oracle",
                 "Backend::sync timed under gpu_sync"):
        assert f"PASS {name}" in r.stdout
