"""Failure paths of the device push and update: every rejected call leaves all
rows (and the optimizer powers) unchanged, and records its failure bits in the
workspace's status history.

  * a NaN per-id weight in a weighted-sum push, and NaN, infinite or negative
    scales in a compact (CSR) update, are rejected before any write
    (ValidateCompactGradients requires finite scales >= 0,
    src/access/compact_gradients.cpp:21);
  * a hot-row hand-over that times out (driven from the host with a spin limit
    of 0, so every wait gives up at once) writes nothing and reports STALLED;
  * a rejected push does not advance the beta powers (ApplyLazyAdam advances
    them only after the update, src/update/lazy_adam.cpp:39-41).
"""
import numpy as np
import pytest

import oracle
from parity import assert_close, oracle_store

pytestmark = pytest.mark.gpu
F32 = np.float32


def hot_feature(W, rng, spec, pooling, bags=600, hot_key=5, hot_refs=900):
    """A feature whose row `hot_key` has `hot_refs` references (a hot row) among
    Zipf-distributed others."""
    lengths = rng.integers(1, 6, bags)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
    n = int(offsets[-1])
    keys = (rng.zipf(1.2, n) % spec.rows).astype(np.uint64)
    keys[rng.choice(n, min(hot_refs, n), replace=False)] = hot_key
    weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
    grad = rng.normal(0, 1e-2, (bags, spec.dim)).astype(F32)
    return W.Feature(0, 0, pooling, keys, offsets, lengths.astype(np.uint64), weights, grad)


def test_nan_weight_rejects_weighted_push(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(11)
    spec = W.TableSpec(0, 64, 3000, seed=5)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    everything = torch.arange(spec.rows, device="cuda")
    before = shard.read_rows(0, everything).clone()
    powers = shard.powers.copy()
    for value in (np.nan, np.inf):
        f = hot_feature(W, rng, spec, W.WEIGHTED_SUM)
        f.weights[17] = value
        print(f"case: weight {value}", flush=True)
        dev = [H.DeviceFeature(torch, f)]
        shard.prepare(dev)
        status = shard.push(dev)
        assert status & H.STATUS_BAD_SCALE and status & H.STATUS_REJECTED, f"{status:#x}"
        assert torch.equal(shard.read_rows(0, everything), before), "rejected push wrote rows"
        assert np.array_equal(shard.powers, powers), "rejected push advanced the powers"
        assert shard.history() & H.STATUS_BAD_SCALE


def test_bad_compact_scales_reject(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    dim = 32
    spec = W.TableSpec(0, dim, 16, seed=9)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    slots = torch.tensor([3, 9, 4], device="cuda")
    before = shard.read_rows(0, torch.arange(16, device="cuda")).clone()
    offsets = torch.tensor([0, 2, 3, 5], device="cuda")
    sources = torch.tensor([0, 1, 1, 0, 2], device="cuda")
    values = torch.from_numpy(np.random.default_rng(3).normal(0, 1e-2, (3, dim)).astype(F32)).cuda()
    for bad in (np.nan, np.inf, -0.25):
        scales = torch.tensor([0.5, 1.0, 0.25, bad, 1.0], dtype=torch.float32, device="cuda")
        print(f"case: scale {bad}", flush=True)
        st = shard.adam_compact(0, slots, offsets, sources, scales, values)
        assert st & H.STATUS_BAD_SCALE and st & H.STATUS_REJECTED, f"scale {bad}: {st:#x}"
        assert torch.equal(shard.read_rows(0, torch.arange(16, device="cuda")), before)
    # -0.0 is a valid scale (-0.0 >= 0), as in the reference.
    scales = torch.tensor([0.5, 1.0, 0.25, -0.0, 1.0], dtype=torch.float32, device="cuda")
    assert shard.adam_compact(0, slots, offsets, sources, scales, values) & H.STATUS_ERRORS == 0


def test_forced_stall_writes_nothing(torch_gpu, pkg):
    """Spin limit 0: every hot-row hand-over wait times out.  The push must
    report STALLED and leave every row unchanged (the hot-row kernel skips its
    staging, adds and stores; the row kernels after it see the stall and write
    nothing).  With the default limit the same push applies, bit-exact."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(12)
    spec = W.TableSpec(0, 64, 3000, seed=6)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    everything = torch.arange(spec.rows, device="cuda")
    before = shard.read_rows(0, everything).clone()
    f = hot_feature(W, rng, spec, W.MEAN)
    assert np.max(np.unique(f.keys, return_counts=True)[1]) > 128, "no hot row"
    dev = [H.DeviceFeature(torch, f)]
    L = H.lib()
    try:
        H.check(L.eps_hip_debug_set_spin_limit(0))
        shard.prepare(dev)
        status = shard.push(dev)
    finally:
        H.check(L.eps_hip_debug_set_spin_limit(1 << 22))
    print(f"forced stall: status {status:#x}", flush=True)
    assert status & H.STATUS_STALLED, f"{status:#x}"
    assert torch.equal(shard.read_rows(0, everything), before), "a stalled push wrote rows"
    assert shard.history() & H.STATUS_STALLED
    shard.clear_history()
    shard.prepare(dev)
    status = shard.push(dev)
    assert status & H.STATUS_ERRORS == 0, f"{status:#x}"
    assert shard.history() == 0
    store = oracle_store(spec)
    store.prepare(f)
    assert oracle.push([store], [f], [0], [f.gradient]) == 0
    keys = store.keys()
    want, _ = store.read_many(keys)
    got = shard.read_rows(0, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
    assert_close(got.reshape(want.shape), want, "push after a stalled one", strict_ulp=0)


def test_history_survives_later_pushes(torch_gpu, pkg):
    """A rejected push, then a good one in the same workspace: the good push's
    status is clean, the history keeps the rejection, the powers advanced once."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(13)
    spec = W.TableSpec(0, 32, 2000, seed=7)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    powers = shard.powers.copy()
    bad = hot_feature(W, rng, spec, W.SUM, hot_refs=10)
    bad.gradient[4, 2] = np.nan
    dev = [H.DeviceFeature(torch, bad)]
    shard.prepare(dev)
    assert shard.push(dev) & H.STATUS_NONFINITE_GRAD
    good = hot_feature(W, rng, spec, W.SUM, hot_refs=10)
    dev = [H.DeviceFeature(torch, good)]
    shard.prepare(dev)
    assert shard.push(dev) & H.STATUS_ERRORS == 0
    assert shard.history() & H.STATUS_NONFINITE_GRAD and shard.history() & H.STATUS_REJECTED
    assert np.array_equal(shard.powers, powers * np.array([[spec.beta1, spec.beta2]], F32))
    shard.clear_history()
    assert shard.history() == 0
