"""Full-size workload parity: the HIP pull + push against the oracle shard.

Each step: pooled pull (compared per element), device dedup + fused Adam push,
the oracle's Lookup + Push on the same inputs, then every touched row's w/m/v
compared.  Sizes are the named shapes (26 x 1M x 64 etc.); the oracle holds
only touched rows.
"""
import time

import numpy as np
import pytest

import oracle
from parity import assert_close, expected_pull, oracle_store

pytestmark = pytest.mark.gpu


def run(torch, W, H, wl, steps, explicit_state=None, compare_every=1, touched_only=False):
    """`touched_only`: compare the rows the step touched at intermediate
    compare steps (untouched rows change on neither side), every row at the end."""
    t0 = time.time()
    first = wl.batch(0)
    shard = H.DeviceShard(torch, wl.tables, max_occurrences=2 * sum(len(f.keys) for f in first))
    stores = [oracle_store(t) for t in wl.tables]
    if explicit_state is None:
        shard.init_rows()
    else:
        for t, state in enumerate(explicit_state):
            slots = torch.arange(state.shape[0], device="cuda")
            shard.load_rows(t, slots, torch.from_numpy(state).cuda())
            d = wl.tables[t].dim
            for key in range(state.shape[0]):
                stores[t].import_row(key, state[key, :d], state[key, d:2 * d], state[key, 2 * d:])
    for step in range(steps):
        feats = first if step == 0 else wl.batch(step)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        pulled = shard.lookup(dev)
        shard.prepare(dev)
        shard.push(dev)
        status = shard.status()
        assert status & H.STATUS_ERRORS == 0, f"{wl.name} step {step}: status {status:#x}"
        for f, out in zip(feats, pulled):
            want = expected_pull(stores[f.table], f)
            if step % compare_every == 0 or step == steps - 1:
                assert_close(out.cpu().numpy(), want, f"{wl.name} pull step {step} table {f.table}",
                             strict_ulp=0)
        rc = oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats])
        assert rc == 0, oracle.last_error()
        if step % compare_every == 0 or step == steps - 1:
            for t, s in enumerate(wl.tables):
                keys = stores[t].keys()
                if touched_only and step != steps - 1:
                    keys = np.unique(np.concatenate([f.keys for f in feats if f.table == t]))
                want, updates = stores[t].read_many(keys)
                got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
                assert_close(got.reshape(want.shape), want, f"{wl.name} state step {step} table {t}",
                             strict_ulp=0)
                assert tuple(shard.powers[t]) == stores[t].powers()[:2]
        print(f"{wl.name} step {step} ok ({time.time() - t0:.1f}s)", flush=True)
    return shard, stores


def test_movielens_trajectory_100_steps(torch_gpu, pkg):
    """2 tables (943, 1682) x 32, N(0, 0.01) explicit state, 128 pairs, 100 steps."""
    W, H = pkg.workloads, pkg.eps_hip
    wl = W.MovieLens()
    run(torch_gpu, W, H, wl, 100, explicit_state=wl.initial_state(), compare_every=10)


def test_criteo26_full_size_step(torch_gpu, pkg):
    """26 x 1,000,000 x 64, batch 4096, bags U{1..20}, Zipf(1.05), 13 sum + 13 mean."""
    W, H = pkg.workloads, pkg.eps_hip
    run(torch_gpu, W, H, W.Criteo26(), 2)


def test_dup10m_steps(torch_gpu, pkg):
    """10,000,000 x 128, 65,536 pairs, Zipf(1.2) (about 82% duplicates), t = 1..50:
    the pull and the step's touched rows every 5th step, and after the last step
    all 247,234 rows the 50 steps touch."""
    W, H = pkg.workloads, pkg.eps_hip
    wl = W.Dup10M()
    feats = wl.batch(0)
    dup = 1 - len(np.unique(feats[0].keys)) / len(feats[0].keys)
    print(f"duplicate fraction {dup:.3f}")
    assert dup > 0.6
    run(torch_gpu, W, H, wl, 50, compare_every=5, touched_only=True)


def test_ragged8_weighted_steps(torch_gpu, pkg):
    """8 ragged tables (dims 16..256, 100k..5M rows), weighted sum, Poisson(8) bags."""
    W, H = pkg.workloads, pkg.eps_hip
    run(torch_gpu, W, H, W.Ragged8(), 2)


def sub_feature(f, bags=None, keep_keys=None):
    """The feature restricted to some bags (pull check) or to the occurrences of
    some keys in every bag (push check).  Bag lengths for the mean stay the
    original ones, so each kept term has the scale it has in the full batch."""
    starts, ends = f.offsets[:-1].astype(np.int64), f.offsets[1:].astype(np.int64)
    if bags is not None:
        parts = [f.keys[starts[b]:ends[b]] for b in bags]
        offsets = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.uint64)
        return type(f)(f.table, f.feature, f.pooling, np.concatenate(parts).astype(np.uint64), offsets,
                       f.valid_lengths[bags], None, f.gradient[bags])
    keep = np.isin(f.keys, keep_keys)
    kept_before = np.concatenate([[0], np.cumsum(keep)])
    offsets = kept_before[np.concatenate([starts[:1], ends])].astype(np.uint64)
    return type(f)(f.table, f.feature, f.pooling, f.keys[keep], offsets, f.valid_lengths, None,
                   f.gradient)


def test_large4_full_size_sampled(torch_gpu, pkg):
    """4 x 12,500,000 x 128 (77 GB of state), 262,144 bags x 32 per table, Zipf(1.1), mean.
    The whole step runs at full size on the device; the oracle checks 1,024 sampled bags
    of the pull and, after the push, the 16 hottest and 240 random touched rows of each
    table (their reduced gradients take every occurrence of those keys, in order)."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    t0 = time.time()
    wl = W.Large4()
    feats = wl.batch(0)
    print(f"large4 batch generated ({time.time() - t0:.1f}s)", flush=True)
    shard = H.DeviceShard(torch, wl.tables, max_occurrences=sum(len(f.keys) for f in feats))
    shard.init_rows()
    dev = [H.DeviceFeature(torch, f) for f in feats]
    pulled = shard.lookup(dev)
    shard.prepare(dev)
    shard.push(dev)
    status = shard.status()
    assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
    print(f"large4 device step done ({time.time() - t0:.1f}s)", flush=True)
    rng = np.random.default_rng(44)
    for f, out in zip(feats, pulled):
        spec = wl.tables[f.table]
        bags = np.sort(rng.choice(len(f.valid_lengths), 1024, replace=False))
        sub = sub_feature(f, bags=bags)
        want = expected_pull(oracle_store(spec), sub)
        assert_close(out[torch.from_numpy(bags).cuda()].cpu().numpy(), want,
                     f"large4 pull table {f.table}", strict_ulp=0)
        uniq, counts = np.unique(f.keys, return_counts=True)
        hottest = uniq[np.argsort(-counts)[:16]]
        sample = np.union1d(hottest, rng.choice(uniq, 240, replace=False)).astype(np.uint64)
        part = sub_feature(f, keep_keys=sample)
        store = oracle_store(spec)
        store.prepare(part)
        assert oracle.push([store], [part], [0], [part.gradient]) == 0, oracle.last_error()
        keys = store.keys()
        assert len(keys) == len(sample)
        want, _ = store.read_many(keys)
        got = shard.read_rows(f.table, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
        assert_close(got.reshape(want.shape), want, f"large4 state table {f.table}", strict_ulp=0)
        assert tuple(shard.powers[f.table]) == store.powers()[:2]
        print(f"large4 table {f.table} ok ({time.time() - t0:.1f}s)", flush=True)
