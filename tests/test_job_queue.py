"""The backend's operation queue on the host (no GPU): runs
tests/cpp/job_queue_test.  One thread runs the operations in submission order;
at most 128 wait in a HipCacheBackend (the reference's executor depth,
src/cuda/cache_backend.cu:222) and a call beyond the depth resolves at once to
capacity_exceeded without running; job errors map to the reference's codes;
closing runs what is queued and refuses the rest."""
import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "cpp" / "_build" / "job_queue_test"


def test_job_queue_contract():
    subprocess.run(["make", "-s", "-C", str(PROGRAM.parents[1]), "_build/job_queue_test"], check=True)
    done = subprocess.run([str(PROGRAM)], capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert done.stdout.startswith("job_queue_test: ok")
