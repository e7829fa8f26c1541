"""bench.py's contract on a machine without a GPU: it measures one GPU's
share only, so a request for several GPUs (the flag, or a launcher's
WORLD_SIZE) ends with a message and a non-zero status before any device
work."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], cwd=ROOT, capture_output=True, text=True,
                       timeout=120, env={**os.environ, **env})
    assert r.returncode == 2, r.stderr
    assert "single MI355X" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout == ""   # no JSON line
