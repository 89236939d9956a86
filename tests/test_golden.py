"""The oracle reproduces the golden vectors that the reference's own sources
wrote (tests/golden/make_golden.py, run against oracle/_ref), bit for bit.

This pins the oracle wherever the reference checkout is absent; the GPU path is
checked against the same vectors in tests/test_gpu_golden.py."""
import pathlib

import numpy as np

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz")  # data only: no pickles


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


class Feature:
    def __init__(self, g, s, f):
        p = f"s{s}_f{f}_"
        self.table = int(g[p + "table"][0])
        self.feature, self.pooling = f, int(g[p + "pooling"][0])
        self.keys, self.offsets = g[p + "keys"], g[p + "offsets"]
        self.valid_lengths, self.gradient = g[p + "valid_lengths"], g[p + "gradient"]
        self.weights = None

    @property
    def rows(self):
        return len(self.keys) if self.pooling == oracle.SEQUENCE else len(self.valid_lengths)


def table_defs(g):
    defs = []
    for tid, dim, (lr, lo, hi, bounded, wmin, wmax, seed) in zip(g["table_ids"], g["table_dims"],
                                                                  g["table_params"]):
        defs.append(oracle.table_def(id=int(tid), dim=int(dim), lr=float(lr), init_min=float(lo),
                                     init_max=float(hi), seed=int(seed),
                                     bounds=(float(wmin), float(wmax)) if bounded else None))
    return defs


def test_shard_trajectory():
    g = load("shard_trajectory")
    steps, features = (int(x) for x in g["steps"])
    stores = [oracle.Store(d) for d in table_defs(g)]
    for s in range(steps):
        feats = [Feature(g, s, f) for f in range(features)]
        for f in feats:
            unique, occ, pooled = stores[f.table].prepare(f)
            p = f"s{s}_f{f.feature}_"
            assert same(unique, g[p + "unique"]), f"step {s} feature {f.feature}: unique rows"
            assert same(occ, g[p + "occurrence_to_unique"]), f"step {s} feature {f.feature}: occurrence map"
            assert same(pooled, g[p + "pooled"]), f"step {s} feature {f.feature}: pooled sums"
        for t, store in enumerate(stores):
            mine = [f for f in feats if f.table == t]
            keys, values = store.reduce_gradients(mine, [f.gradient for f in mine])
            assert same(keys, g[f"s{s}_t{t}_reduce_keys"]), f"step {s} table {t}: reduced rows"
            assert same(values, g[f"s{s}_t{t}_reduce_values"]), f"step {s} table {t}: reduced values"
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
        for t, store in enumerate(stores):
            b1, b2, seq = store.powers()
            assert same(np.array([b1, b2], np.float32), g[f"s{s}_t{t}_powers"])
            assert seq == int(g[f"s{s}_t{t}_sequence"][0])
            if f"s{s}_t{t}_touched" in g:
                state, updates = store.read_many(g[f"s{s}_t{t}_touched"])
                assert same(state.reshape(len(updates), -1), g[f"s{s}_t{t}_state"]), f"step {s} table {t}"
                assert same(updates, g[f"s{s}_t{t}_updates"])


def test_host_backend_apply_steps():
    g = load("host_backend")
    dim = g["initial"].shape[1] // 3
    w, m, v = (g["initial"][:, i * dim:(i + 1) * dim] for i in range(3))
    step = 0
    while f"step{step}_gradient" in g:
        b1p, b2p = g[f"step{step}_powers"]
        rc, w, m, v = oracle.adam_rows_ctx(w, m, v, g[f"step{step}_gradient"], 0.9, 0.999, 1e-8, 0.05,
                                           b1p, b2p, (-0.03, 0.03))
        assert rc == 0
        step += 1
    assert same(np.concatenate([w, m, v], 1), g["final"])
    assert same(g["final_updates"], g["initial_updates"] + step)


def test_compact_build_and_expand():
    g = load("compact")
    store = oracle.Store(oracle.table_def(id=6, dim=16, lr=0.01, init_min=-0.05, init_max=0.05, seed=11))
    feats, grads = [], []
    for f in range(3):
        feat = type("F", (), {})()
        feat.pooling, feat.feature = int(g[f"f{f}_pooling"][0]), f
        feat.keys, feat.offsets = g[f"f{f}_keys"], g[f"f{f}_offsets"]
        feat.valid_lengths, feat.weights = g[f"f{f}_valid_lengths"], None
        store.prepare(feat)
        feats.append(feat)
        grads.append(g[f"f{f}_gradient"])
    keys, values = store.reduce_gradients(feats, grads)
    assert same(keys, g["row_keys"]) and same(values, g["reduce_values"])
    sv, off, src, sc = oracle.build_compact(feats, grads, 16, keys)
    assert same(sv, g["source_values"]) and same(off, g["row_offsets"])
    assert same(src, g["source_rows"]) and same(sc, g["scales"])
    assert same(oracle.expand_compact(keys, 16, sv, off, src, sc), g["expanded"])
    assert same(g["expanded"], g["reduce_values"]), "CSR expansion must equal ReduceGradients"
