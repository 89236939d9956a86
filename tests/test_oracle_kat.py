"""Pins the oracle (oracle/eps_oracle.c) with the reference's own known answers.

Each test re-expresses a check that the reference's test suite holds, with its
numbers, plus closed forms and invariants that a plausible restatement mistake
(dropped term, wrong index, reversed order) would fail.
"""
import math

import numpy as np
import pytest

import oracle

F32 = np.float32


class Feat:
    def __init__(self, pooling, keys, offsets, lengths, weights=None, feature=0):
        self.pooling, self.feature = pooling, feature
        self.keys = np.asarray(keys, np.uint64)
        self.offsets = np.asarray(offsets, np.uint64)
        self.valid_lengths = np.asarray(lengths, np.uint64)
        self.weights = None if weights is None else np.asarray(weights, np.float32)


def core_table(shard_count=1, **kw):
    # tests/core_tests.cpp:43-45: {1, 2, count, 1, {0.1, 0.9, 0.999, 1e-8, 0.9, 0.999}, 0.25, 0.25, 42}
    args = dict(id=1, dim=2, shard_count=shard_count, lr=0.1, init_min=0.25, init_max=0.25, seed=42)
    args.update(kw)
    return oracle.table_def(**args)


def test_pooling_and_update_known_answers():
    # tests/core_tests.cpp:68-85
    s = oracle.Store(core_table())
    f0 = Feat(oracle.SUM, [1, 1, 2], [0, 3, 3], [3, 0], feature=0)
    f1 = Feat(oracle.MEAN, [1, 3], [0, 2], [2], feature=1)
    u0, occ0, c0 = s.prepare(f0)
    u1, occ1, c1 = s.prepare(f1)
    assert c0.shape == (2, 2)
    assert c0[0, 0] == pytest.approx(0.75, abs=1e-5)
    assert c0[1, 0] == 0.0
    assert c1[0, 0] == pytest.approx(0.5, abs=1e-5)  # unnormalised partial sum
    assert list(occ0) == [0, 0, 1] and list(u0) == [0, 1]
    assert list(u1) == [0, 2]  # key 1 is slot 0 (first touch), key 3 gets slot 2
    g0 = np.array([[1, 2], [0, 0]], F32)
    g1 = np.array([[4, 6]], F32)
    assert oracle.push([s], [f0, f1], [0, 0], [g0, g1]) == 0
    a, b, c = s.read(1), s.read(2), s.read(3)
    np.testing.assert_allclose(a[1], [0.4, 0.7], atol=1e-5)
    np.testing.assert_allclose(a[2], [0.016, 0.049], atol=1e-5)
    assert b[1][0] == pytest.approx(0.1, abs=1e-5)
    assert c[1][0] == pytest.approx(0.2, abs=1e-5)
    assert a[0][0] == pytest.approx(0.15, abs=1e-5)
    assert a[3] == 1, "repeated ID applied twice"
    b1p, b2p, seq = s.powers()
    assert seq == 1 and b1p == F32(0.9) * F32(0.9) and b2p == F32(0.999) * F32(0.999)


def test_sequence_positions_kept():
    # tests/core_tests.cpp:87-96
    s = oracle.Store(core_table(init_min=-1, init_max=1))
    _, occ, v = s.prepare(Feat(oracle.SEQUENCE, [8, 2, 8], [0, 2, 3], [2, 1]))
    assert v.shape == (3, 2)
    assert v[0, 0] == v[2, 0] and v[0, 1] == v[2, 1]
    assert list(occ) == [0, 1, 0]


def test_initializer_is_independent_of_shard_topology():
    # tests/core_tests.cpp:142-154
    even = oracle.Store(core_table(2, init_min=-1, init_max=1))
    odd = oracle.Store(oracle.table_def(id=1, dim=2, shard=1, shard_count=2, lr=0.1,
                                        init_min=-1, init_max=1, seed=42))
    with pytest.raises(ValueError):
        even.ensure(1)  # key 1 belongs to the odd shard
    even.ensure(2)
    odd.ensure(1)
    single = oracle.Store(core_table(1, init_min=-1, init_max=1))
    single.ensure(1)
    single.ensure(2)
    assert np.array_equal(single.read(1)[0], odd.read(1)[0])
    assert np.array_equal(single.read(2)[0], even.read(2)[0])


def test_initializer_closed_form():
    # shard_store.cpp:13-18,104-112 with the published SplitMix64 finaliser
    # constants; u = top 53 bits / 2^53 and a double lerp rounded once.
    d = oracle.table_def(id=7, dim=4, init_min=-0.05, init_max=0.05, seed=123)
    assert oracle.mix(0) == 0xE220A8397B1DCDAF  # SplitMix64 first output from state 0
    for key in (0, 1, 999, 2**40 + 3):
        for col in range(4):
            bits = oracle.mix(key ^ oracle.mix(123) ^ oracle.mix(7) ^ oracle.mix(col))
            u = (bits >> 11) * 2.0**-53
            assert 0.0 <= u < 1.0
            lo, hi = float(F32(-0.05)), float(F32(0.05))  # float bounds widened to double
            expect = F32((1 - u) * lo + u * hi)
            assert oracle.init_weight(d, key, col) == expect
    # All-equal bounds give the bound exactly (core_tests init 0.25/0.25).
    assert oracle.init_weight(core_table(), 5, 1) == F32(0.25)
    # Clamp applies at init (weight_bounds_tests.cpp:71-76: init 0.5 clipped to 0.2).
    b = oracle.table_def(id=1, dim=2, lr=1.0, init_min=0.5, init_max=0.5, bounds=(-0.1, 0.2))
    assert oracle.init_weight(b, 1, 0) == F32(0.2)


def test_overflow_rejects_without_partial_update():
    # tests/core_tests.cpp:214-222
    s = oracle.Store(core_table())
    f = Feat(oracle.SEQUENCE, [1, 2], [0, 2], [2])
    s.prepare(f)
    g = np.array([[1, 1], [np.finfo(np.float32).max, 1]], F32)
    assert oracle.push([s], [f], [0], [g]) != 0
    assert s.read(1)[3] == 0 and s.read(2)[3] == 0
    assert s.read(1)[0][0] == F32(0.25)
    assert s.powers()[2] == 0, "powers advanced on a rejected push"


def test_nonfinite_gradient_rejected_even_in_empty_bag():
    # batch_access.cpp:69-70: every gradient value must be finite.
    s = oracle.Store(core_table())
    f = Feat(oracle.SUM, [1], [0, 1, 1], [1, 0])
    s.prepare(f)
    g = np.array([[1, 1], [np.inf, 0]], F32)
    assert oracle.push([s], [f], [0], [g]) != 0
    assert "non-finite gradient" in oracle.last_error()


def test_bounded_adam_six_steps_closed_form():
    # tests/weight_bounds_tests.cpp:71-86: lr 1, init 0.5 clipped to [-0.1, 0.2],
    # g = +10, +10, -10, -10, -10, -10, sequence feature of key 1.
    s = oracle.Store(oracle.table_def(id=1, dim=2, lr=1.0, init_min=0.5, init_max=0.5,
                                      bounds=(-0.1, 0.2)))
    m = v = F32(0)
    w = F32(0.2)
    b1, b2 = F32(0.9), F32(0.999)
    for seq in range(1, 7):
        g = F32(10 if seq <= 2 else -10)
        m = F32(0.9) * m + (F32(1) - F32(0.9)) * g
        v = F32(0.999) * v + (F32(1) - F32(0.999)) * g * g
        step = np.sqrt(F32(1) - b2, dtype=F32) / (F32(1) - b1) * m / (np.sqrt(v, dtype=F32) + F32(1e-8))
        w = F32(np.clip(w - step, F32(-0.1), F32(0.2)))
        f = Feat(oracle.SEQUENCE, [1], [0, 1], [1])
        s.prepare(f)
        assert oracle.push([s], [f], [0], [np.full((1, 2), g, F32)]) == 0
        sw, sm, sv, _ = s.read(1)
        assert abs(sw[0] - w) < 3e-6 and abs(sm[0] - m) < 3e-6 and abs(sv[0] - v) < 3e-6
        b1, b2 = F32(b1 * F32(0.9)), F32(b2 * F32(0.999))


def test_adam_first_step_sign_and_magnitude():
    # Invariant: on the first Adam step from zero moments, |delta w| = lr_t *
    # (1-b1)|g| / (sqrt(1-b2)|g| + eps) ~= lr (bias correction cancels), with the
    # sign opposite to g.  A swapped beta or dropped bias correction fails this.
    s = oracle.Store(oracle.table_def(id=1, dim=2, lr=1e-3, init_min=0.0, init_max=0.0))
    f = Feat(oracle.SEQUENCE, [5], [0, 1], [1])
    s.prepare(f)
    assert oracle.push([s], [f], [0], [np.array([[0.5, -2.0]], F32)]) == 0
    w = s.read(5)[0]
    assert w[0] == pytest.approx(-1e-3, rel=1e-4) and w[1] == pytest.approx(1e-3, rel=1e-4)


def test_lr_t_closed_form():
    # lazy_adam.cpp:27 in float: lr * sqrt(1 - b2p) / (1 - b1p)
    for lr, b1p, b2p in [(0.1, 0.9, 0.999), (1e-3, 0.9**7, 0.999**7), (1.0, 0.0, 0.0)]:
        f = F32
        expect = f(f(lr) * np.sqrt(f(1) - f(b2p), dtype=f)) / (f(1) - f(b1p))
        assert oracle.lr_t(lr, b1p, b2p) == expect
        assert float(oracle.lr_t(lr, b1p, b2p)) == pytest.approx(lr * math.sqrt(1 - b2p) / (1 - b1p), rel=1e-4)  # float cancellation in 1 - b2p


def sin_gradients(features, dim):
    out = []
    for f in features:
        rows = len(f.keys) if f.pooling == oracle.SEQUENCE else len(f.valid_lengths)
        i = np.arange(rows * dim, dtype=np.float32) + F32(f.feature)
        out.append(np.sin(i).astype(F32).reshape(rows, dim))
    return out


def test_compact_expand_equals_reduce():
    # tests/compact_tests.cpp:13-30 (dim 128; mean, sum and sequence features).
    s = oracle.Store(oracle.table_def(id=1, dim=128, lr=0.01, init_min=0.25, init_max=0.25))
    feats = [Feat(oracle.MEAN, [1, 1, 2, 3], [0, 3, 4], [3, 1], feature=0),
             Feat(oracle.SUM, [3, 1], [0, 2], [2], feature=1),
             Feat(oracle.SEQUENCE, [2, 1], [0, 2], [2], feature=2)]
    for f in feats:
        s.prepare(f)
    grads = sin_gradients(feats, 128)
    keys, values = s.reduce_gradients(feats, grads)
    assert list(keys) == [1, 2, 3]  # first-occurrence order across features
    sv, off, src, sc = oracle.build_compact(feats, grads, 128, [3, 1])
    expanded = oracle.expand_compact([3, 1], 128, sv, off, src, sc)
    np.testing.assert_allclose(expanded[0], values[2], atol=1e-6)
    np.testing.assert_allclose(expanded[1], values[0], atol=1e-6)
    # Key 3: mean bag 1 + sum bag; key 1: mean bag 0 twice (scale 1/3), sum bag, sequence pos 1.
    assert list(off) == [0, 2, 6]
    np.testing.assert_array_equal(sc[2:4], [F32(1) / F32(3)] * 2)


def test_compact_payload_shrinks_for_long_pooled_bag():
    # tests/compact_tests.cpp:31-35
    keys = list(range(1, 65))
    f = Feat(oracle.MEAN, keys, [0, 64], [64])
    g = [np.ones((1, 128), F32)]
    sv, off, src, sc = oracle.build_compact([f], g, 128, keys)
    assert oracle.compact_bytes(64, sv.size, len(src)) < 64 * 128 * 4 / 8


def test_compact_malformed_packets_rejected():
    # tests/compact_tests.cpp:36-40
    feats = [Feat(oracle.MEAN, [1, 1, 2, 3], [0, 3, 4], [3, 1], feature=0),
             Feat(oracle.SUM, [3, 1], [0, 2], [2], feature=1)]
    grads = sin_gradients(feats, 128)
    sv, off, src, sc = oracle.build_compact(feats, grads, 128, [3, 1])
    good = dict(row_keys=[3, 1], dim=128, source_values=sv, row_offsets=off, source_rows=src, scales=sc)
    oracle.expand_compact(**good)
    bad = dict(good, source_rows=np.concatenate([[2**64 - 1], src[1:]]).astype(np.uint64))
    with pytest.raises(ValueError):
        oracle.expand_compact(**bad)
    o2 = off.copy(); o2[-1] += 1
    with pytest.raises(ValueError):
        oracle.expand_compact(**dict(good, row_offsets=o2))
    with pytest.raises(ValueError):
        oracle.expand_compact(**dict(good, row_keys=[3, 3]))
    s2 = sc.copy(); s2[0] = np.nan
    with pytest.raises(ValueError):
        oracle.expand_compact(**dict(good, scales=s2))
    v2 = sv.copy(); v2.flat[0] = np.inf
    with pytest.raises(ValueError):
        oracle.expand_compact(**dict(good, source_values=v2))


def test_gather_host_closed_form_weights():
    # tests/cuda_stress.cpp:18,89: weights 0.001*(key%17 + d%13), bags of 16,
    # pooled sums equal the float sequential sums (max error 0 observed).
    rng = np.random.default_rng(0)
    dim, bags = 128, 64
    keys = rng.integers(1, 5000, bags * 16).astype(np.uint64)
    uniq, inv = np.unique(keys, return_inverse=True)
    weight = lambda k: (F32(0.001) * (F32(k % 17) + np.arange(dim, dtype=np.uint32) % 13).astype(F32)).astype(F32)
    rows = [weight(int(k)) for k in uniq]
    f = Feat(oracle.SUM, keys, np.arange(0, bags * 16 + 1, 16), [16] * bags)
    out = oracle.gather_host(f, dim, inv.astype(np.uint64), rows)
    for b in range(bags):
        acc = np.zeros(dim, F32)
        for k in keys[b * 16:(b + 1) * 16]:
            acc = (acc + weight(int(k))).astype(F32)
        assert np.array_equal(out[b], acc)
        assert np.max(np.abs(out[b] - sum(weight(int(k)).astype(np.float64) for k in keys[b * 16:(b + 1) * 16]))) < 1e-5


def test_gather_host_layouts_with_holes():
    # tests/cuda_tests.cpp:35-45: mean (with a hole), sequence and sum layouts.
    dim = 128
    states = {k: (F32(0.05) * np.sin(np.arange(dim, dtype=F32) + F32(k * 7))).astype(F32) for k in (1, 2, 3)}
    HOLE = 2**64 - 1
    mean = Feat(oracle.MEAN, [1, 1, 999, 2], [0, 3, 4], [3, 1])
    out = oracle.gather_host(mean, dim, np.array([0, 0, HOLE, 1], np.uint64), [states[1], states[2]])
    assert np.array_equal(out[0], (states[1] + states[1]).astype(F32))
    assert np.array_equal(out[1], states[2])
    seq = Feat(oracle.SEQUENCE, [3, 1, 3], [0, 2, 3], [2, 1])
    out = oracle.gather_host(seq, dim, np.array([0, 1, 0], np.uint64), [states[3], states[1]])
    assert np.array_equal(out[0], states[3]) and np.array_equal(out[2], states[3])
    sums = Feat(oracle.SUM, [1, 2], [0, 2, 2], [2, 0])
    out = oracle.gather_host(sums, dim, np.array([0, 1], np.uint64), [states[1], states[2]])
    assert np.array_equal(out[0], (states[1] + states[2]).astype(F32)) and not out[1].any()


def test_weighted_sum_extension_reduces_to_sum_and_brute_force():
    # Weighted-sum pooling has no reference counterpart: at unit weights it must
    # equal sum pooling bit for bit, and in general a float loop of w*a then add.
    s = oracle.Store(oracle.table_def(id=3, dim=8, init_min=-1, init_max=1, seed=9))
    keys = [4, 9, 4, 11, 9]
    plain = Feat(oracle.SUM, keys, [0, 3, 5], [3, 2])
    ones = Feat(oracle.WEIGHTED_SUM, keys, [0, 3, 5], [3, 2], weights=[1] * 5)
    assert np.array_equal(s.prepare(plain)[2], s.prepare(ones)[2])
    a = np.array([0.5, 0.25, 2.0, 0.1, 3.0], F32)
    _, _, out = s.prepare(Feat(oracle.WEIGHTED_SUM, keys, [0, 3, 5], [3, 2], weights=a))
    rows = {k: s.read(k)[0] for k in set(keys)}
    for b, (lo, hi) in enumerate([(0, 3), (3, 5)]):
        acc = np.zeros(8, F32)
        for i in range(lo, hi):
            acc = (acc + (rows[keys[i]] * a[i]).astype(F32)).astype(F32)
        assert np.array_equal(out[b], acc)
    # Backward: per-occurrence scale is the weight.
    g = np.arange(16, dtype=F32).reshape(2, 8) / F32(7)
    f = Feat(oracle.WEIGHTED_SUM, keys, [0, 3, 5], [3, 2], weights=a)
    rk, rv = s.reduce_gradients([f], [g])
    assert list(rk) == [4, 9, 11]
    acc4 = (np.zeros(8, F32) + (g[0] * a[0]).astype(F32)).astype(F32)
    acc4 = (acc4 + (g[0] * a[2]).astype(F32)).astype(F32)
    assert np.array_equal(rv[0], acc4)


def test_reduce_first_occurrence_order_brute_force():
    rng = np.random.default_rng(5)
    s = oracle.Store(oracle.table_def(id=2, dim=4, init_min=-1, init_max=1))
    lengths = rng.integers(0, 6, 40)
    offsets = np.concatenate([[0], np.cumsum(lengths)])
    keys = rng.integers(0, 30, offsets[-1]).astype(np.uint64)
    f = Feat(oracle.MEAN, keys, offsets, lengths + (rng.random(40) < 0.2))
    g = rng.normal(size=(40, 4)).astype(F32)
    rk, rv = s.reduce_gradients([f], [g])
    order = []
    for k in keys:
        if k not in order:
            order.append(k)
    assert list(rk) == order
    for u, k in enumerate(order):
        acc = np.zeros(4, F32)
        for b in range(40):
            scale = F32(1) / F32(f.valid_lengths[b]) if f.valid_lengths[b] else F32(1)
            for i in range(offsets[b], offsets[b + 1]):
                if keys[i] == k:
                    acc = (acc + (g[b] * scale).astype(F32)).astype(F32)
        assert np.array_equal(rv[u], acc)


def test_mean_divide_closed_form():
    """The client's mean (distributed_client.cpp:227-232): each value is
    0.0f + partial, then divided by float(valid_length) when that is non-zero.
    IEEE division is correctly rounded, so numpy's float32 quotient is the
    closed form.  The cases fix the three ways to get it wrong: a reciprocal
    multiply (values chosen where x * (1/len) rounds differently from x / len),
    dividing an empty bag (len 0 leaves the value), and keeping -0.0 (the
    +0.0f start turns it into +0.0)."""
    x = np.array([[0.82161814, 0.3645724, 0.2941325, -1.3031572],
                  [0.34558418, 0.82161814, 0.9053559, 5.0],
                  [-0.0, 1.5, -2.25, 3.0e-38],
                  [-0.0, 0.0, -7.0, 1.0e30]], np.float32)
    lengths = np.array([3, 7, 0, 13], np.uint64)
    got = oracle.mean_divide(x, lengths)
    want = (np.float32(0.0) + x).astype(np.float32)
    for b, n in enumerate(lengths):
        if n:
            want[b] = want[b] / np.float32(n)
    assert got.tobytes() == want.tobytes()
    recip = x[:2] * (np.float32(1) / lengths[:2, None].astype(np.float32))
    assert np.any(recip != got[:2]), "the cases must separate divide from reciprocal multiply"
    assert not np.signbit(got[2, 0]) and not np.signbit(got[3, 0])  # -0.0 comes out as +0.0
    assert got[2, 1] == np.float32(1.5) and got[2, 3] == np.float32(3.0e-38)  # empty bag unchanged
