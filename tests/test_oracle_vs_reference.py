"""Pins the oracle against the reference's own CPU sources (oracle/_ref).

oracle/_ref/libeps_ref.so is compiled from the reference checkout by
oracle/Makefile (`make ref`); where it is absent these tests skip and the
committed golden fixtures (tests/test_golden.py) carry the same pin.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")

F32 = np.float32


class Feat:
    def __init__(self, pooling, keys, offsets, lengths, feature=0):
        self.pooling, self.feature = pooling, feature
        self.keys = np.asarray(keys, np.uint64)
        self.offsets = np.asarray(offsets, np.uint64)
        self.valid_lengths = np.asarray(lengths, np.uint64)
        self.weights = None

    @property
    def rows(self):
        return len(self.keys) if self.pooling == oracle.SEQUENCE else len(self.valid_lengths)


def random_feature(rng, pooling, bags, max_len, key_space, feature, shard=0, shards=1):
    lengths = rng.integers(0, max_len + 1, bags)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
    keys = (rng.zipf(1.3, int(offsets[-1])) % key_space).astype(np.uint64)
    keys = keys * np.uint64(shards) + np.uint64(shard)
    valid = lengths + (rng.random(bags) < 0.25) * rng.integers(0, 3, bags)  # padded originals
    return Feat(pooling, keys, offsets, valid, feature)


DEFS = [dict(id=1, dim=2, lr=0.1, init_min=-1, init_max=1, seed=42),
        dict(id=4, dim=8, lr=0.01, init_min=-0.05, init_max=0.05, seed=7, bounds=(-0.04, 0.045)),
        dict(id=9, dim=64, lr=1e-3, init_min=-0.05, init_max=0.05, seed=3001)]


@pytest.mark.parametrize("shard,shards", [(0, 1), (1, 3)])
def test_shard_steps_bit_exact(shard, shards):
    rng = np.random.default_rng(11 + shard)
    defs = [oracle.table_def(shard=shard, shard_count=shards, **d) for d in DEFS]
    ref = oracle.RefShard(defs, shard, shards)
    ours = [oracle.Store(d) for d in defs]
    table_ids = [d.id for d in defs]
    for step in range(6):
        feats, fstore = [], []
        for fi in range(5):
            t = int(rng.integers(0, len(defs)))
            pooling = [oracle.SUM, oracle.MEAN, oracle.SEQUENCE][fi % 3]
            feats.append(random_feature(rng, pooling, 17, 6, 40, fi, shard, shards))
            fstore.append(t)
        for f, t in zip(feats, fstore):
            ru, ro, rc = ref.prepare(table_ids[t], f)
            ou, oo, oc = ours[t].prepare(f)
            assert np.array_equal(ru, ou) and np.array_equal(ro, oo)
            assert np.array_equal(rc.view(np.uint32), oc.view(np.uint32))
        grads = [rng.normal(0, 1e-1 if step % 2 else 3.0, (f.rows, defs[t].dim)).astype(F32)
                 for f, t in zip(feats, fstore)]
        for t in range(len(defs)):
            sel = [i for i in range(len(feats)) if fstore[i] == t]
            if not sel:
                continue
            rk, rv = ref.reduce(table_ids[t], [grads[i] if fstore[i] == t else np.zeros((feats[i].rows, defs[fstore[i]].dim), F32) for i in range(len(feats))])
            ok, ov = ours[t].reduce_gradients([feats[i] for i in sel], [grads[i] for i in sel])
            assert np.array_equal(rk, ok)
            assert np.array_equal(rv.view(np.uint32), ov.view(np.uint32))
        assert ref.push(grads) == 0
        assert oracle.push(ours, feats, fstore, grads) == 0
        for t, d in enumerate(defs):
            assert ref.powers(d.id) == ours[t].powers()
            for slot in range(ours[t].rows):
                key = ours[t].key_at(slot)
                rw, rm, rv_, ru = ref.read(d.id, key)
                w, m, v, u = ours[t].read(key)
                assert np.array_equal(rw, w) and np.array_equal(rm, m) and np.array_equal(rv_, v)
                assert ru == u


def test_overflow_rejection_matches_reference():
    defs = [oracle.table_def(**DEFS[0])]
    ref, ours = oracle.RefShard(defs), oracle.Store(defs[0])
    f = Feat(oracle.SEQUENCE, [1, 2], [0, 2], [2])
    ref.prepare(1, f)
    ours.prepare(f)
    g = np.array([[1, 1], [np.finfo(F32).max, 1]], F32)
    assert ref.push([g]) != 0
    assert oracle.push([ours], [f], [0], [g]) != 0
    for key in (1, 2):
        assert all(np.array_equal(a, b) for a, b in zip(ref.read(1, key)[:3], ours.read(key)[:3]))


def test_compact_build_and_expand_match_reference():
    rng = np.random.default_rng(3)
    d = oracle.table_def(id=2, dim=16, lr=0.01, init_min=-1, init_max=1)
    ref, ours = oracle.RefShard([d]), oracle.Store(d)
    feats = [random_feature(rng, p, 23, 7, 30, i) for i, p in
             enumerate([oracle.MEAN, oracle.SUM, oracle.SEQUENCE, oracle.MEAN])]
    for f in feats:
        ref.prepare(2, f)
        ours.prepare(f)
    grads = [rng.normal(size=(f.rows, 16)).astype(F32) for f in feats]
    keys, _ = ours.reduce_gradients(feats, grads)
    targets = keys[::2]
    r = ref.build_compact(2, grads, targets)
    o = oracle.build_compact(feats, grads, 16, targets)
    for a, b in zip(r, o):
        assert np.array_equal(np.asarray(a).view(np.uint32) if a.dtype == F32 else a,
                              np.asarray(b).view(np.uint32) if b.dtype == F32 else b)
    e_ref = oracle.ref_expand_compact(2, targets, 16, *r)
    e_our = oracle.expand_compact(targets, 16, *o)
    assert np.array_equal(e_ref.view(np.uint32), e_our.view(np.uint32))


def test_host_backend_apply_matches_oracle():
    # HostCacheBackend::ApplyHost (host_backend.cpp:119-146) with explicit
    # UpdateContext powers, bounded table, 7 steps; then an overflow rejection.
    rng = np.random.default_rng(4)
    dim, rows = 128, 4
    d = oracle.table_def(id=1, dim=dim, lr=0.01, init_min=-0.1, init_max=0.1, bounds=(-0.015, 0.015))
    hb = oracle.RefHostBackend()
    hb.define(d)
    keys = np.arange(1, rows + 1, dtype=np.uint64)
    w = (0.05 * np.sin(np.arange(rows * dim, dtype=F32))).astype(F32).reshape(rows, dim)
    m = np.tile((F32(0.001) * (np.arange(dim) % 5)).astype(F32), (rows, 1))
    v = np.tile((F32(0.002) * (1 + np.arange(dim) % 3)).astype(F32), (rows, 1))
    packed = np.concatenate([w, m, v], axis=1)
    slots = hb.load(1, dim, keys, packed, np.full(rows, 3, np.uint64))
    b1p, b2p = F32(0.9), F32(0.999)
    for step in range(7):
        g = (F32(0.03) * np.cos(np.arange(rows * dim, dtype=F32) + F32(step))).astype(F32).reshape(rows, dim)
        assert hb.apply(1, 0.01, b1p, b2p, keys, g, dim) == 0
        rc, w, m, v = oracle.adam_rows_ctx(w, m, v, g, 0.9, 0.999, 1e-8, 0.01, b1p, b2p, (-0.015, 0.015))
        assert rc == 0
        got, updates = hb.read(1, dim, keys, slots)
        assert np.array_equal(got, np.concatenate([w, m, v], axis=1))
        assert list(updates) == [4 + step] * rows
        b1p, b2p = F32(b1p * F32(0.9)), F32(b2p * F32(0.999))
    assert (np.abs(w) == F32(0.015)).any(), "clipping not exercised"
    g = np.ones((rows, dim), F32)
    g[-1, -1] = np.finfo(F32).max
    assert hb.apply(1, 0.01, b1p, b2p, keys, g, dim) != 0
    rc, *_ = oracle.adam_rows_ctx(w, m, v, g, 0.9, 0.999, 1e-8, 0.01, b1p, b2p, (-0.015, 0.015))
    assert rc != 0
    got, _ = hb.read(1, dim, keys, slots)
    assert np.array_equal(got, np.concatenate([w, m, v], axis=1))
