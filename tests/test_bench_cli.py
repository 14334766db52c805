"""bench.py's command-line contract on the CPU: it measures one GPU and refuses a
multi-GPU request (flag or torchrun world size) with a message and exit status 2,
before touching any device."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "4"})])
def test_bench_refuses_more_than_one_gpu(args, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py")] + args, cwd=ROOT,
                       env={**os.environ, **env}, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""
