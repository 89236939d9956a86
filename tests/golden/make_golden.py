#!/usr/bin/env python3
"""Writes the golden vectors of tests/golden/ from the reference's own sources.

Runs only where oracle/_ref/libeps_ref.so was compiled from the reference
checkout (oracle/Makefile `ref`).  The fixtures are data: seeded inputs and the
outputs the compiled reference produced for them.

  shard_trajectory.npz  3 tables (dims 8 bounded, 32, 64), 5 steps of 6 features
                        (sum / mean / sequence, empty bags, padded lengths):
                        per feature the pooled partial sums (PrepareFeature),
                        unique keys in first-occurrence order and the occurrence
                        map; per table the ReduceGradients rows and values and,
                        after each push, the beta powers; after steps 1 and 4 every
                        touched row's w, m, v and update counter.
  host_backend.npz      HostCacheBackend: load, 4 ApplyHost steps with clipping,
                        read-back state.
  compact.npz           BuildCompactGradients + ExpandCompactGradients of one push.
"""
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle  # noqa: E402

TABLES = [dict(id=3, dim=8, lr=0.01, init_min=-0.05, init_max=0.05, seed=7, bounds=(-0.04, 0.045)),
          dict(id=5, dim=32, lr=1e-3, init_min=-0.05, init_max=0.05, seed=3001),
          dict(id=9, dim=64, lr=1e-3, init_min=-0.05, init_max=0.05, seed=42)]
SPACE = [64, 256, 512]
STEPS, FEATURES, BAGS, MAX_LEN = 5, 6, 16, 8
STATE_STEPS = (1, 4)  # steps after which every touched row is recorded


class Feature:
    def __init__(self, feature, pooling, keys, offsets, lengths):
        self.feature, self.pooling = feature, pooling
        self.keys, self.offsets, self.valid_lengths = keys, offsets, lengths
        self.weights = None

    @property
    def rows(self):
        return len(self.keys) if self.pooling == oracle.SEQUENCE else len(self.valid_lengths)


def shard_trajectory(out):
    rng = np.random.default_rng(20261201)
    defs = [oracle.table_def(**t) for t in TABLES]
    ref = oracle.RefShard(defs)
    out["table_ids"] = np.array([t["id"] for t in TABLES], np.uint32)
    out["table_dims"] = np.array([t["dim"] for t in TABLES], np.uint32)
    out["table_space"] = np.array(SPACE, np.uint64)
    # lr, init_min, init_max, bounded, weight_min, weight_max, seed (as float64)
    out["table_params"] = np.array([[t["lr"], t["init_min"], t["init_max"], "bounds" in t,
                                     t.get("bounds", (0, 0))[0], t.get("bounds", (0, 0))[1], t["seed"]]
                                    for t in TABLES], np.float64)
    out["steps"] = np.array([STEPS, FEATURES], np.uint32)
    for s in range(STEPS):
        feats, grads, tab = [], [], []
        for f in range(FEATURES):
            t = (s + f) % len(TABLES)
            pooling = [oracle.SUM, oracle.MEAN, oracle.SEQUENCE][f % 3]
            lengths = rng.integers(0, MAX_LEN + 1, BAGS)
            offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
            keys = (rng.zipf(1.2, int(offsets[-1])) % SPACE[t]).astype(np.uint64)
            valid = (lengths + (rng.random(BAGS) < 0.25) * rng.integers(1, 3, BAGS)).astype(np.uint64)
            feat = Feature(f, pooling, keys, offsets, valid)
            rows = feat.rows
            grad = rng.normal(0, 0.5 if s % 2 else 0.05, (rows, TABLES[t]["dim"])).astype(np.float32)
            unique, occ, contribution = ref.prepare(TABLES[t]["id"], feat)
            p = f"s{s}_f{f}_"
            out[p + "table"] = np.array([t], np.uint32)
            out[p + "pooling"] = np.array([pooling], np.uint32)
            out[p + "keys"], out[p + "offsets"], out[p + "valid_lengths"] = keys, offsets, valid
            out[p + "gradient"] = grad
            out[p + "unique"], out[p + "occurrence_to_unique"] = unique, occ
            out[p + "pooled"] = contribution
            feats.append(feat)
            grads.append(grad)
            tab.append(t)
        for t, spec in enumerate(TABLES):
            keys, values = ref.reduce(spec["id"], grads)
            out[f"s{s}_t{t}_reduce_keys"], out[f"s{s}_t{t}_reduce_values"] = keys, values
        assert ref.push(grads) == 0, ref.error()
        for t, spec in enumerate(TABLES):
            b1, b2, seq = ref.powers(spec["id"])
            out[f"s{s}_t{t}_powers"] = np.array([b1, b2], np.float32)
            out[f"s{s}_t{t}_sequence"] = np.array([seq], np.uint64)
            if s not in STATE_STEPS:
                continue
            touched = np.unique(np.concatenate([feats[i].keys for i in range(FEATURES) if tab[i] == t]
                                               or [np.zeros(0, np.uint64)]))
            state = np.zeros((len(touched), 3 * spec["dim"]), np.float32)
            updates = np.zeros(len(touched), np.uint64)
            for i, k in enumerate(touched):
                w, m, v, u = ref.read(spec["id"], int(k))
                state[i] = np.concatenate([w, m, v])
                updates[i] = u
            out[f"s{s}_t{t}_touched"], out[f"s{s}_t{t}_state"] = touched, state
            out[f"s{s}_t{t}_updates"] = updates


def host_backend(out):
    dim, keys = 16, np.array([11, 4, 29], np.uint64)
    d = oracle.table_def(id=2, dim=dim, lr=0.05, init_min=-0.1, init_max=0.1, seed=5,
                         bounds=(-0.03, 0.03))
    backend = oracle.RefHostBackend()
    backend.define(d)
    rng = np.random.default_rng(77)
    packed = rng.normal(0, 0.02, (len(keys), 3 * dim)).astype(np.float32)
    packed[:, 2 * dim:] = np.abs(packed[:, 2 * dim:])
    slots = backend.load(2, dim, keys, packed, np.array([5, 0, 2], np.uint64))
    out["keys"], out["initial"], out["initial_updates"] = keys, packed, np.array([5, 0, 2], np.uint64)
    b1, b2 = np.float32(0.9), np.float32(0.999)
    for s in range(4):
        g = rng.normal(0, 1.0, (len(keys), dim)).astype(np.float32)
        assert backend.apply(2, 0.05, b1, b2, keys, g, dim) == 0, backend.error()
        out[f"step{s}_gradient"] = g
        out[f"step{s}_powers"] = np.array([b1, b2], np.float32)
        b1, b2 = np.float32(b1 * np.float32(0.9)), np.float32(b2 * np.float32(0.999))
    final, updates = backend.read(2, dim, keys, slots)
    out["final"], out["final_updates"] = final, updates


def compact(out):
    rng = np.random.default_rng(31)
    spec = dict(id=6, dim=16, lr=0.01, init_min=-0.05, init_max=0.05, seed=11)
    ref = oracle.RefShard([oracle.table_def(**spec)])
    grads = []
    for f, pooling in enumerate([oracle.MEAN, oracle.SUM, oracle.SEQUENCE]):
        lengths = rng.integers(0, 6, 12)
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
        keys = (rng.zipf(1.4, int(offsets[-1])) % 20).astype(np.uint64)
        feat = Feature(f, pooling, keys, offsets, (lengths + 1).astype(np.uint64))
        ref.prepare(6, feat)
        g = rng.normal(0, 0.1, (feat.rows, 16)).astype(np.float32)
        grads.append(g)
        out[f"f{f}_pooling"], out[f"f{f}_keys"] = np.array([pooling], np.uint32), keys
        out[f"f{f}_offsets"], out[f"f{f}_valid_lengths"] = offsets, feat.valid_lengths
        out[f"f{f}_gradient"] = g
    row_keys, values = ref.reduce(6, grads)
    sv, off, src, sc = ref.build_compact(6, grads, row_keys)
    out["row_keys"], out["reduce_values"] = row_keys, values
    out["source_values"], out["row_offsets"], out["source_rows"], out["scales"] = sv, off, src, sc
    out["expanded"] = oracle.ref_expand_compact(6, row_keys, 16, sv, off, src, sc)


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libeps_ref.so is not built (oracle/Makefile ref)")
    for name, fn in (("shard_trajectory", shard_trajectory), ("host_backend", host_backend),
                     ("compact", compact)):
        out = {}
        fn(out)
        np.savez_compressed(HERE / f"{name}.npz", **out)
        print(f"{name}.npz: {len(out)} arrays")


if __name__ == "__main__":
    main()
