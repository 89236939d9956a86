"""The backend's snapshot encoder (host code, no GPU) against the oracle.

Runs tests/cpp/snapshot_format_test: the field encoder and publication that
HipCacheBackend::WriteSnapshot uses write two stores' content (bounded and
unbounded tables, first-touch and imported rows, an advanced optimizer clock),
and the oracle's restatement of src/store/snapshot.cpp:159-194 must write the
same bytes; existing files are never replaced and no staging file is left."""
import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "cpp" / "_build" / "snapshot_format_test"


def test_snapshot_encoder_matches_oracle_writer():
    if not PROGRAM.exists():
        subprocess.run(["make", "-s", "-C", str(PROGRAM.parents[1]), "_build/snapshot_format_test"],
                       check=True)
    done = subprocess.run([str(PROGRAM)], capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert done.stdout.startswith("PASS")
