"""eps::HipCacheBackend (the C++ drop-in for the reference's CudaCacheBackend)
on the GPU, through three test programs under tests/cpp:

* hip_backend_test re-expresses the reference's tests/cuda_tests.cpp scenarios
  and compares gathers, assembled features and optimizer states with the
  oracle bit for bit;
* hip_stress is the reference's concurrent checked-read stress
  (tests/cuda_stress.cpp:35-105: 8 caller threads x 64 batches x 4,096 keys
  against one backend, closed-form weights, statistics unchanged) plus the
  128-job queue rule;
* hip_consumer_test is the reference's device-output hand-off
  (tests/worker_agent_cuda.cu:50-81): a model on a non-blocking stream of its
  own, the outstanding-output budget, results outliving the backend."""
import json
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
BUILD = ROOT / "tests" / "cpp" / "_build"
PROGRAM = BUILD / "hip_backend_test"

pytestmark = pytest.mark.gpu


def test_hip_backend_matches_oracle(torch_gpu):
    assert PROGRAM.exists(), "build the test program with __graft_entry__.build()"
    print(f"case: {PROGRAM.name}", flush=True)
    done = subprocess.run([str(PROGRAM)], capture_output=True, text=True, timeout=300)
    print(done.stdout, done.stderr)
    assert done.returncode == 0, done.stderr
    assert done.stdout.startswith("PASS")


def run(name, *args, timeout=300):
    program = BUILD / name
    assert program.exists(), "build the test programs with __graft_entry__.build()"
    print(f"case: {name} {' '.join(args)}", flush=True)
    done = subprocess.run([str(program), *args], capture_output=True, text=True, timeout=timeout)
    print(done.stdout, done.stderr)
    assert done.returncode == 0, done.stderr
    return done.stdout


def test_checked_read_stress(torch_gpu):
    """8 threads x 64 batches x 4,096 keys on 262,144 rows of dimension 128:
    every pooled value equals the sequential fp32 sum of the closed-form
    weights (error 0), the device statistics are unchanged, and a burst behind
    a long gather is refused with capacity_exceeded once 128 calls wait."""
    out = run("hip_stress", "262144", "128", "8", "64", timeout=240)
    line = json.loads(out.strip().splitlines()[-1])
    assert line["maximum_absolute_error"] == 0
    assert line["checked_batches"] == 512 and line["key_occurrences"] == 512 * 4096
    assert line["queue_refused"] > 0 and line["queue_served"] >= 128


def test_consumer_stream_and_output_budget(torch_gpu):
    out = run("hip_consumer_test", timeout=120)
    assert out.startswith("PASS")
