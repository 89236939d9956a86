"""Pins the oracle's snapshot format (src/store/snapshot.cpp) on the CPU.

* tests/golden/snapshot-v1-unbounded.bin is the reference's own compatibility
  fixture (tests/fixtures/snapshot-v1-unbounded.bin, described in
  tests/fixtures/README.md there): format 1, run "legacy-unbounded", one table
  of one row, FNV-1a checksum 0x0f7d76d9f8d09430.  The oracle reader must
  decode exactly that content and checksum.
* Format 2 files written by the reference's own WriteSnapshot (oracle/_ref)
  must read back to the reference's row state and be rewritten byte for byte
  by the oracle writer.
* Corrupt, truncated and extended files are rejected (the reference's
  CorruptSnapshotIsRejected, tests/core_tests.cpp:131-140).
"""
import pathlib
import struct

import numpy as np
import pytest

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "snapshot-v1-unbounded.bin"
F32 = np.float32


def test_fixture_v1_decodes_to_its_documented_content():
    r = oracle.snapshot_read(GOLDEN)
    assert (r["run"], r["shard"], r["shard_count"], r["epoch"], r["version"]) == \
        ("legacy-unbounded", 0, 1, 1, 1)
    assert r["checksum"] == 0x0F7D76D9F8D09430
    (t,) = r["tables"]
    d = t.defn
    assert (d.id, d.dim, d.shard_count, d.bounded, d.init_seed) == (1, 2, 1, 0, 42)
    assert [F32(x) for x in (d.learning_rate, d.beta1, d.beta2, d.epsilon, d.initial_beta1_power,
                             d.initial_beta2_power, d.init_min, d.init_max)] == \
        [F32(0.1), F32(0.9), F32(0.999), F32(1e-8), F32(0.9), F32(0.999), F32(0.25), F32(0.25)]
    assert t.powers() == (F32(0.9), F32(0.999), 0)
    assert list(t.keys()) == [1]
    w, m, v, updates = t.read(1)
    assert w.tolist() == [0.25, 0.25] and not m.any() and not v.any() and updates == 0


def test_fixture_checksum_is_fnv1a_of_the_payload():
    data = GOLDEN.read_bytes()
    stored = struct.unpack("<Q", data[-8:])[0]
    assert oracle.fnv1a(data[:-8]) == stored == 0x0F7D76D9F8D09430
    # FNV-1a of the empty string is its offset basis; one byte is one round.
    assert oracle.fnv1a(b"") == oracle.FNV_OFFSET
    assert oracle.fnv1a(b"a") == ((oracle.FNV_OFFSET ^ 0x61) * 1099511628211) % (1 << 64)


def test_format2_round_trip_keeps_every_byte(tmp_path):
    a = oracle.Store(oracle.table_def(id=3, dim=4, bounds=(-0.5, 0.5), init_min=-0.1, init_max=0.1, seed=9))
    b = oracle.Store(oracle.table_def(id=1, dim=2, init_min=-1, init_max=1, seed=5))
    for key in (7, 3, 11):
        a.ensure(key)
    b.import_row(5, [1.5, -2.0], [0.25, 0.0], [0.5, 1e-30], updates=9)
    first = tmp_path / "one.bin"
    oracle.snapshot_write(first, "run-a", 0, 1, 1, [a, b])
    r = oracle.snapshot_read(first)
    assert r["version"] == 2 and [t.defn.id for t in r["tables"]] == [3, 1]
    assert list(r["tables"][0].keys()) == [7, 3, 11]
    second = tmp_path / "two.bin"
    oracle.snapshot_write(second, r["run"], r["shard"], r["shard_count"], r["epoch"], r["tables"])
    assert first.read_bytes() == second.read_bytes()


def test_reader_rejects_damaged_files(tmp_path):
    good = GOLDEN.read_bytes()
    cases = {
        "flip": good[:-9] + bytes([good[-9] ^ 1]) + good[-8:],   # tests/core_tests.cpp:136
        "truncated": good[:-3],
        "trailing": good + b"\0",
        "magic": b"\0" + good[1:],
    }
    for name, data in cases.items():
        path = tmp_path / name
        path.write_bytes(data)
        with pytest.raises(ValueError):
            oracle.snapshot_read(path)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
def test_oracle_matches_reference_write_snapshot(tmp_path):
    rng = np.random.default_rng(5)
    defs = [oracle.table_def(id=1, dim=2, lr=0.1, init_min=-1, init_max=1, seed=42),
            oracle.table_def(id=4, dim=8, lr=0.01, init_min=-0.05, init_max=0.05, seed=7,
                             bounds=(-0.04, 0.045)),
            oracle.table_def(id=9, dim=5, lr=1e-3, init_min=-0.05, init_max=0.05, seed=3001)]
    ref = oracle.RefShard(defs)
    for d in defs:
        for key in rng.permutation(40)[:17]:
            w = rng.normal(0, 0.02, d.dim)
            ref.import_row(d.id, int(key) * 3 + 1, w, rng.normal(0, 1e-3, d.dim),
                           rng.random(d.dim) * 1e-4, updates=int(rng.integers(0, 50)))
    # Advance each table's optimizer clock and touch new rows (first-touch order).
    from test_oracle_vs_reference import random_feature
    for step in range(3):
        feats = [random_feature(rng, [oracle.SUM, oracle.MEAN, oracle.SEQUENCE][i], 9, 5, 60, i)
                 for i in range(3)]
        grads = []
        for d, f in zip(defs, feats):
            ref.prepare(d.id, f)
            grads.append(rng.normal(0, 0.1, (f.rows, d.dim)).astype(F32))
        assert ref.push(grads) == 0
    path = tmp_path / "snap" / "shard-0.bin"
    ref.write_snapshot(path, "run-ref")
    r = oracle.snapshot_read(path)
    assert (r["run"], r["shard"], r["shard_count"], r["epoch"], r["version"]) == ("run-ref", 0, 1, 1, 2)
    assert sorted(t.defn.id for t in r["tables"]) == [1, 4, 9]
    for t in r["tables"]:
        assert t.powers() == ref.powers(t.defn.id)
        assert t.powers()[2] == 3
        for key in t.keys():
            got, want = t.read(int(key)), ref.read(t.defn.id, int(key))
            assert all(np.array_equal(x, y) for x, y in zip(got[:3], want[:3])) and got[3] == want[3]
    again = tmp_path / "again.bin"
    oracle.snapshot_write(again, r["run"], r["shard"], r["shard_count"], r["epoch"], r["tables"])
    assert again.read_bytes() == path.read_bytes()
