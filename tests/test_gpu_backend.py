"""eps::HipCacheBackend (the C++ drop-in for the reference's CudaCacheBackend)
against the oracle: runs tests/cpp/hip_backend_test on the GPU.

The program re-expresses the reference's tests/cuda_tests.cpp scenarios and
compares gathers, assembled features and optimizer states bit for bit."""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "cpp" / "_build" / "hip_backend_test"

pytestmark = pytest.mark.gpu


def test_hip_backend_matches_oracle(torch_gpu):
    assert PROGRAM.exists(), "build the test program with __graft_entry__.build()"
    print(f"case: {PROGRAM.name}", flush=True)
    done = subprocess.run([str(PROGRAM)], capture_output=True, text=True, timeout=300)
    print(done.stdout, done.stderr)
    assert done.returncode == 0, done.stderr
    assert done.stdout.startswith("PASS")
