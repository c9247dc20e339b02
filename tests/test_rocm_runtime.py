"""Hot-path parity on the ROCm HIP runtime alone (the one a host without
torch, like molten's Rust host, binds): tests/rocm_runtime_worker.py runs
full-size configurations 1, 2, 3 and 5 in a child process in which torch
cannot be imported, against the oracle."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu


def test_hot_path_on_rocm_runtime(dev):
    worker = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rocm_runtime_worker.py")
    r = subprocess.run([sys.executable, worker], capture_output=True, text=True, timeout=110)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("OK")]
    assert [ln.split()[1] for ln in lines] == ["config1", "config2", "config5_b1", "config5_b8", "config3",
                                               "runtime"], r.stdout
    assert "torch" not in lines[-1], lines[-1]
