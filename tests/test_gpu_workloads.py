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


def run(torch, W, H, wl, steps, explicit_state=None, compare_every=1):
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
    """10,000,000 x 128, 65,536 pairs, Zipf(1.2) (about 82% duplicates), t = 1..3."""
    W, H = pkg.workloads, pkg.eps_hip
    wl = W.Dup10M()
    feats = wl.batch(0)
    dup = 1 - len(np.unique(feats[0].keys)) / len(feats[0].keys)
    print(f"duplicate fraction {dup:.3f}")
    assert dup > 0.6
    run(torch_gpu, W, H, wl, 3)


def test_ragged8_weighted_steps(torch_gpu, pkg):
    """8 ragged tables (dims 16..256, 100k..5M rows), weighted sum, Poisson(8) bags."""
    W, H = pkg.workloads, pkg.eps_hip
    run(torch_gpu, W, H, W.Ragged8(), 2)
