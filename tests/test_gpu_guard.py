"""Failure paths of the device push and update: every rejected call leaves all
rows (and the optimizer powers) unchanged, and records its failure bits in the
workspace's status history.

  * a NaN per-id weight in a weighted-sum push, and NaN, infinite or negative
    scales in a compact (CSR) update, are rejected before any write
    (ValidateCompactGradients requires finite scales >= 0,
    src/access/compact_gradients.cpp:21);
  * a hot-row hand-over that times out (driven from the host with a spin limit
    of 0, so every wait gives up at once) writes none of its hot rows and
    reports STALLED;
  * a rejected push does not advance the beta powers (ApplyLazyAdam advances
    them only after the update, src/update/lazy_adam.cpp:39-41);
  * the guard decides from a snapshot of the bounds taken before the update,
    so every block decides the same even when the update's own rows raise the
    bounds past the limit on the way (1.2 M rows, with and without the
    hot-row kernel beside the row kernel);
  * a prepared workspace damaged after preparation is never used as an
    address: a bad key rejects the push before any write, a bad reference
    word keeps its row unwritten.
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


@pytest.mark.parametrize("bags,overlap", [(24000, True), (90000, True), (24000, False), (12000, True)])
def test_forced_stall_reports_and_writes_no_hot_row(torch_gpu, pkg, bags, overlap):
    """Spin limit 0: every hand-over wait of the hot-row kernel times out (it
    runs for pushes with a table of 65,536 or more references: in 16-column
    units of 256-reference chunks under 262,144 vector references, 24,000
    bags here, else in 32-column units of 64-reference chunks, 90,000 bags; a
    push with no such table takes 64-column units beside the row kernels,
    12,000 bags).
    The push must report STALLED, in its status and in the workspace history,
    and write none of the hot rows it stalled on.  Beside the row kernels
    (`overlap`) those write theirs, so such a push is partial -- the C++
    backend stops after one (tests/cpp/hip_backend_test.cpp); on one stream
    the hot-row kernel runs first and the row kernels after it see the stall,
    so nothing is written.  From fresh state, the same push with the default
    limit applies bit-exact."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(12)
    spec = W.TableSpec(0, 64, 3000, seed=6)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    everything = torch.arange(spec.rows, device="cuda")
    before = shard.read_rows(0, everything).clone()
    f = hot_feature(W, rng, spec, W.MEAN, bags=bags, hot_refs=3000)
    if bags == 12000:
        assert len(f.keys) < 65536, len(f.keys)
    else:
        assert len(f.keys) >= 65536
        assert (len(f.keys) < 1 << 18) == (bags == 24000), len(f.keys)
    ids, counts = np.unique(f.keys, return_counts=True)
    hot = torch.from_numpy(ids[counts > 128].astype(np.int64)).cuda()
    assert hot.numel() > 0, "no hot row"
    dev = [H.DeviceFeature(torch, f)]
    L = H.lib()
    try:
        H.check(L.eps_hip_debug_set_spin_limit(0))
        shard.prepare(dev)
        status = shard.push(dev, hot_overlap=overlap)
    finally:
        H.check(L.eps_hip_debug_set_spin_limit(1 << 22))
    print(f"forced stall: bags {bags}, overlap {overlap}, status {status:#x}", flush=True)
    assert status & H.STATUS_STALLED, f"{status:#x}"
    assert shard.history() & H.STATUS_STALLED
    assert torch.equal(shard.read_rows(0, hot), before[hot]), "a stalled hot row was written"
    if not overlap:
        assert torch.equal(shard.read_rows(0, everything), before), "a row was written after the stall"
    shard.clear_history()
    shard.init_rows()  # fresh state: the stalled push was partial
    shard.prepare(dev)
    status = shard.push(dev, hot_overlap=overlap)
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


def _near_limit_shard(torch, W, H, rows, dim, x=0.7e30):
    """A table whose every row has w = v = 0 and m = m0, loaded through the
    bounds domain, with m0 chosen so that a zero-gradient first step writes
    |w'| = lr_t * m' / eps = x: the guard's w bound before the step is
    x * 1.0201 (below 1e30, so the fused pass runs), but a decision taken from
    the bounds as raised by rows already written would be 2.04 * x (checked)."""
    spec = W.TableSpec(0, dim, rows, seed=4)
    shard = H.DeviceShard(torch, [spec])
    lr = float(H.lr_t(spec.lr, spec.b1p, spec.b2p))
    m0 = F32(x * spec.eps / (spec.beta1 * lr))
    packed = torch.zeros((rows, 3 * dim), dtype=torch.float32, device="cuda")
    packed[:, dim:2 * dim] = float(m0)
    shard.load_rows(0, torch.arange(rows, device="cuda"), packed)
    del packed
    return spec, shard, m0


@pytest.mark.parametrize("hot", [False, True], ids=["rows", "rows+hot-rows-beside"])
def test_guard_decides_from_snapshot(torch_gpu, pkg, hot):
    """1.2 M distinct rows (several times the update blocks the GPU holds at
    once) whose zero-gradient step takes |w| to 0.7e30.  Every block must take
    the decision the bounds before the push allow (fused) and every row must
    be updated exactly as the CPU shard updates it (lazy_adam.cpp:7-42 applies
    the whole push: every value stays finite).  `hot` adds rows with 300
    references each on a table of more than 65,536 references, so the hot-row
    kernel runs beside the row kernel and both decide."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rows, dim = 1_200_000, 16
    spec, shard, m0 = _near_limit_shard(torch, W, H, rows, dim)
    ids = np.arange(rows, dtype=np.uint64)
    if hot:
        ids = np.concatenate([ids, np.repeat(np.arange(0, 40, dtype=np.uint64) * 7919, 300)])
    lengths = np.ones(len(ids), np.uint64)
    offsets = np.arange(len(ids) + 1, dtype=np.uint64)
    grad = np.zeros((len(ids), dim), F32)
    f = W.Feature(0, 0, W.SUM, ids, offsets, lengths, None, grad)
    dev = [H.DeviceFeature(torch, f)]
    print(f"case: snapshot guard hot={hot} rows={rows} refs={len(ids)}", flush=True)
    shard.prepare(dev)
    status = shard.push(dev)
    assert status & H.STATUS_ERRORS == 0, f"{status:#x}"
    assert not status & H.STATUS_CHECKED_PATH, f"decision should be fused: {status:#x}"
    rc, w1, m1, v1 = oracle.adam_rows_ctx(np.zeros((1, dim), F32), np.full((1, dim), m0, F32),
                                          np.zeros((1, dim), F32), np.zeros((1, dim), F32),
                                          spec.beta1, spec.beta2, spec.eps, spec.lr, spec.b1p, spec.b2p)
    assert rc == 0
    assert 0.5e30 < abs(float(w1[0, 0])) < 0.98e30
    want = np.concatenate([w1, m1, v1], axis=1)
    got = shard.read_rows(0, torch.arange(rows, device="cuda")).cpu().numpy()
    bad = np.flatnonzero(~(got == want).all(axis=1))
    assert bad.size == 0, f"{bad.size} rows differ from the CPU shard (first {bad[:5]})"
    # The bounds now hold |w| = 0.7e30: the next push must take the checked path.
    shard.prepare(dev)
    status = shard.push(dev)
    assert status & H.STATUS_CHECKED_PATH and status & H.STATUS_ERRORS == 0, f"{status:#x}"


def _find(haystack, needle):
    """Offset (in elements) of the first occurrence of array `needle` in `haystack`."""
    hb, nb = haystack.tobytes(), needle.tobytes()
    at = hb.find(nb)
    while at >= 0 and at % needle.itemsize:
        at = hb.find(nb, at + 1)
    assert at >= 0, "array not found in the workspace"
    return at // needle.itemsize


@pytest.mark.parametrize("what", ["key-table", "key-slot", "ref-feature", "ref-row"])
def test_damaged_workspace_rejects(torch_gpu, pkg, what):
    """A prepared workspace with one sorted key or reference word changed
    after preparation, naming a table, slot, feature or gradient row the push
    does not have.  A damaged key is found by the gradient scan before
    anything is written: BAD_INDEX and REJECTED, every row unchanged.  A
    damaged reference word is found where the update kernels decode it: it is
    never used as an address, BAD_INDEX is reported and the row it feeds is
    not written.  No case faults."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(21)
    spec = W.TableSpec(0, 64, 3000, seed=8)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    everything = torch.arange(spec.rows, device="cuda")
    before = shard.read_rows(0, everything).clone()
    f = hot_feature(W, rng, spec, W.MEAN)
    dev = [H.DeviceFeature(torch, f)]
    shard.prepare(dev)
    torch.cuda.synchronize()
    ws = shard.wss[0]
    host = ws.cpu().numpy().view(np.uint32)
    host = host[: len(host) // 2 * 2]
    order = np.argsort(f.keys, kind="stable")
    keys = f.keys[order].astype(np.uint32)  # one table: key == slot
    at = _find(host, keys)
    bag = np.searchsorted(f.offsets, np.arange(len(f.keys)), side="right") - 1
    scale = (F32(1) / f.valid_lengths[bag].astype(F32)).view(np.uint32).astype(np.uint64)
    words = (scale << np.uint64(32)) | bag.astype(np.uint64)
    wat = _find(host.view(np.uint64), words[order])
    k = len(keys) // 2
    print(f"case: damaged workspace {what} at sorted position {k} (row {keys[k]})", flush=True)
    flat = ws.view(torch.int32)
    if what == "key-table":   # row_bits of 3000 rows is 12: table index 1 of a one-table push
        flat[at + k] = int((1 << 12) | int(keys[k]))
    elif what == "key-slot":  # slot 3000 is inside the 12 row bits, past the table
        flat[at + k] = spec.rows
    else:
        w64 = ws[: ws.numel() // 2 * 2].view(torch.int64)
        word = int(words[order][k])
        word = (word | (5 << 27)) if what == "ref-feature" else ((word & ~((1 << 27) - 1)) | len(f.valid_lengths))
        w64[wat + k] = word - (1 << 64) if word >= 1 << 63 else word
    status = shard.push(dev)
    assert status & H.STATUS_BAD_INDEX, f"{status:#x}"
    assert shard.history() & H.STATUS_BAD_INDEX
    after = shard.read_rows(0, everything)
    if what.startswith("key"):
        assert status & H.STATUS_REJECTED, f"{status:#x}"
        assert torch.equal(after, before), "a rejected push wrote rows"
    else:
        row = int(keys[k])
        assert torch.equal(after[row], before[row]), "the row of a damaged reference was written"
