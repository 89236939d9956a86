"""The update's decision functions on the host (no GPU).

Runs tests/cpp/guard_test: the overflow guard's gradient bound and per-table
check (csrc/guard.hpp, the functions the update kernels evaluate) are sound
against fp32 sums and fp32 Adam steps of random states inside the bounds, each
bound decides on a case built for it, and the range checks of sorted keys and
reference words reject every out-of-range field at its boundary."""
import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "cpp" / "_build" / "guard_test"


def test_guard_functions():
    subprocess.run(["make", "-s", "-C", str(PROGRAM.parents[1]), "_build/guard_test"], check=True)
    done = subprocess.run([str(PROGRAM)], capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert done.stdout.startswith("guard_test: ok")
