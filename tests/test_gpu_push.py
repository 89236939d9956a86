"""Device push (dedup + aggregation + fused sparse Adam) vs the oracle."""
import numpy as np
import pytest

import oracle
from parity import assert_close, oracle_store

pytestmark = pytest.mark.gpu
HOLE = np.uint64(2**64 - 1)
F32 = np.float32


def random_features(W, rng, specs, count, holes=0.0, grad_scale=1e-2, bags=200, max_len=10):
    feats = []
    for i in range(count):
        t = int(rng.integers(0, len(specs)))
        pooling = [W.SUM, W.MEAN, W.SEQUENCE, W.WEIGHTED_SUM][i % 4]
        lengths = rng.integers(0, max_len + 1, bags)
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
        n = int(offsets[-1])
        keys = (rng.zipf(1.15, n) % specs[t].rows).astype(np.uint64)
        if holes:
            keys[rng.random(n) < holes] = HOLE
        valid = (lengths + (rng.random(bags) < 0.2) * rng.integers(1, 3, bags)).astype(np.uint64)
        weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
        rows = n if pooling == W.SEQUENCE else bags
        grad = rng.normal(0, grad_scale, (rows, specs[t].dim)).astype(F32)
        feats.append(W.Feature(t, i, pooling, keys, offsets, valid, weights, grad))
    return feats


def expected_unique(feats):
    """First-occurrence order over (table, key) in feature, bag, position order."""
    index, order, occ = {}, [], []
    for f in feats:
        for k in f.keys:
            if k == HOLE:
                occ.append(int(HOLE))
                continue
            key = (f.table, int(k))
            if key not in index:
                index[key] = len(order)
                order.append(key)
            occ.append(index[key])
    return order, np.array(occ, np.uint64)


def live(f):
    """The feature restricted to its non-hole occurrences (what the CPU owner of
    those rows sees: holes are other owners' keys)."""
    keep = f.keys != HOLE
    starts = np.concatenate([[0], np.cumsum([keep[int(f.offsets[b]):int(f.offsets[b + 1])].sum()
                                            for b in range(len(f.valid_lengths))])]).astype(np.uint64)
    g = f.gradient[keep] if f.pooling == oracle.SEQUENCE else f.gradient
    w = None if f.weights is None else f.weights[keep]
    return type(f)(f.table, f.feature, f.pooling, f.keys[keep], starts, f.valid_lengths, w, g)


@pytest.mark.parametrize("dims", [(64,), (8, 64, 96), (16, 300, 6, 128)])
def test_unique_and_reduce_match_oracle(torch_gpu, pkg, dims):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(sum(dims))
    specs = [W.TableSpec(i, d, 5000 + 1000 * i, seed=20 + i) for i, d in enumerate(dims)]
    feats = random_features(W, rng, specs, 7, holes=0.05)
    print(f"case: dims={dims} occurrences={sum(len(f.keys) for f in feats)}", flush=True)
    check_unique_reduce(torch, W, H, specs, feats)


@pytest.mark.parametrize("seed", range(16))
def test_unique_and_reduce_random_sweep(torch_gpu, pkg, seed):
    """The push sweep's random layouts (sweep_case: 1-6 tables of mixed
    dimensions, every pooling, skews 1.05-1.5, 4,000-300,000 references) with
    0-10 % of the keys made holes: first-occurrence unique rows, the occurrence
    map and the reduced gradients against the oracle."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng, specs, skew, layout = sweep_case(W, 500 + seed)
    feats = sweep_features(W, rng, specs, skew, layout)
    holes = float(rng.choice([0.0, 0.03, 0.1]))
    for f in feats:
        f.keys[rng.random(len(f.keys)) < holes] = HOLE
    print(f"case: seed={seed} dims={[s.dim for s in specs]} holes={holes} "
          f"occurrences={sum(len(f.keys) for f in feats)}", flush=True)
    check_unique_reduce(torch, W, H, specs, feats)


def check_unique_reduce(torch, W, H, specs, feats):
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    dev = [H.DeviceFeature(torch, f) for f in feats]
    shard.prepare(dev)
    slots, tables, occ, count = shard.unique(dev)
    torch.cuda.synchronize()
    order, want_occ = expected_unique(feats)
    u = int(count.item())
    assert u == len(order)
    got = list(zip(tables[:u].cpu().numpy().tolist(), slots[:u].cpu().numpy().tolist()))
    assert got == order, "unique rows differ from first-occurrence order"
    assert np.array_equal(occ[:len(want_occ)].cpu().numpy().view(np.uint64), want_occ)
    values = shard.reduce(dev, occ, u).cpu().numpy()
    index = {key: i for i, key in enumerate(order)}
    for t, s in enumerate(specs):
        sel = [live(f) for f in feats if f.table == t]
        if not sel:
            continue
        store = oracle_store(s)
        keys, vals = store.reduce_gradients(sel, [f.gradient for f in sel])
        rows = [index[(t, int(k))] for k in keys]
        assert_close(values[rows, : s.dim], vals, f"reduce table {t}", strict_ulp=0)


@pytest.mark.parametrize("dims,hot_overlap", [((64,), True), ((4, 32, 192), True), ((96, 6, 256, 300), True),
                                               ((4, 32, 192), False)])
def test_push_steps_match_oracle(torch_gpu, pkg, dims, hot_overlap):
    """Zipf(1.15) keys over 4,000 rows: some rows have more than 128
    references (the hot-row kernel), on its side stream or, with hot_overlap
    False, on the push's stream."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(100 + sum(dims))
    specs = [W.TableSpec(i, d, 4000, seed=30 + i,
                         bounds=(-0.06, 0.055) if i == 1 else None) for i, d in enumerate(dims)]
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    stores = [oracle_store(s) for s in specs]
    for step in range(4):
        feats = random_features(W, rng, specs, 6, holes=0.03, grad_scale=1e-1 if step % 2 else 1.0)
        print(f"case: dims={dims} hot_overlap={hot_overlap} step={step}", flush=True)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        shard.prepare(dev)
        shard.push(dev, hot_overlap=hot_overlap)
        status = shard.status()
        assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
        cpu = [live(f) for f in feats]
        for f in cpu:
            stores[f.table].prepare(f)
        assert oracle.push(stores, cpu, [f.table for f in cpu], [f.gradient for f in cpu]) == 0
        for t, s in enumerate(specs):
            keys = stores[t].keys()
            want, _ = stores[t].read_many(keys)
            got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
            assert_close(got.reshape(want.shape), want, f"state table {t} step {step}", strict_ulp=0)
            assert tuple(shard.powers[t]) == stores[t].powers()[:2] or not any(f.table == t for f in feats)


SWEEP_DIMS = (4, 8, 12, 16, 32, 48, 64, 96, 128, 192, 256, 6, 300)


def sweep_case(W, seed):
    """A seeded random push layout: 1-6 tables of mixed dimensions (vector and
    generic), 1-8 features in every pooling, Zipf skews from 1.05 to 1.5, and
    sizes from a few thousand references up to past the 65,536-reference and
    262,144-reference thresholds of the hot-row units."""
    rng = np.random.default_rng(1000 + seed)
    n_tables = int(rng.integers(1, 7))
    specs = [W.TableSpec(i, int(rng.choice(SWEEP_DIMS)), int(rng.integers(200, 6000)), seed=200 + seed * 10 + i)
             for i in range(n_tables)]
    n_features = int(rng.integers(1, 9))
    total = int(rng.choice([4_000, 30_000, 90_000, 300_000]))
    skew = float(rng.choice([1.05, 1.2, 1.5]))
    shares = rng.dirichlet(np.ones(n_features))
    layout = []
    for f in range(n_features):
        refs = max(1, int(total * shares[f]))
        layout.append((int(rng.integers(0, n_tables)), [W.SUM, W.MEAN, W.SEQUENCE, W.WEIGHTED_SUM][int(rng.integers(0, 4))],
                       refs, int(rng.integers(1, 25))))
    return rng, specs, skew, layout


def sweep_features(W, rng, specs, skew, layout):
    feats = []
    for i, (t, pooling, refs, max_len) in enumerate(layout):
        lengths = rng.integers(0, max_len + 1, int(refs / max(1, max_len / 2)) + 1)
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
        n = int(offsets[-1])
        keys = (rng.zipf(skew, n) % specs[t].rows).astype(np.uint64)
        weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
        rows = n if pooling == W.SEQUENCE else len(lengths)
        valid = (lengths + (rng.random(len(lengths)) < 0.1)).astype(np.uint64)
        grad = rng.normal(0, 1e-2, (rows, specs[t].dim)).astype(F32)
        feats.append(W.Feature(t, i, pooling, keys, offsets, valid, weights, grad))
    return feats


@pytest.mark.parametrize("seed", range(60))
def test_push_random_sweep(torch_gpu, pkg, seed):
    """Seeded random pushes (sweep_case) over two steps, every touched row
    bit-exact against the oracle: table counts, dimensions, poolings, skews and
    sizes together, so the hot-row unit widths, both stream placements and the
    dimension classes meet in combinations no single-purpose test builds.
    Every third case runs the hot-row kernel on the push's stream."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng, specs, skew, layout = sweep_case(W, seed)
    hot_overlap = seed % 3 != 2
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    stores = [oracle_store(s) for s in specs]
    for step in range(2):
        feats = sweep_features(W, rng, specs, skew, layout)
        print(f"case: seed={seed} step={step} dims={[s.dim for s in specs]} skew={skew} "
              f"refs={[len(f.keys) for f in feats]} hot_overlap={hot_overlap}", flush=True)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        shard.prepare(dev)
        status = shard.push(dev, hot_overlap=hot_overlap)
        assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
        for f in feats:
            stores[f.table].prepare(f)
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
        for t, s in enumerate(specs):
            keys = stores[t].keys()
            if len(keys) == 0:
                continue
            want, _ = stores[t].read_many(keys)
            got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
            assert_close(got.reshape(want.shape), want, f"state table {t} step {step}", strict_ulp=0)


@pytest.mark.parametrize("refs", [128, 129])
def test_push_hot_row_boundary(torch_gpu, pkg, refs):
    """A row referenced `refs` times makes up all of its table's references:
    128 is still a row-kernel row (and no table can then hold a hot row, so no
    hot-row kernel or side stream is used), 129 is a hot row.  Other tables
    take 100 references each.  Three steps, bit-exact against the oracle."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(refs)
    specs = [W.TableSpec(i, d, 500, seed=80 + i) for i, d in enumerate((64, 32, 128))]
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    stores = [oracle_store(s) for s in specs]
    for step in range(3):
        feats = []
        for t, spec in enumerate(specs):
            n = refs if t == 0 else 100
            lengths = np.full(n // 4, 4, np.int64)
            lengths[-1] += n - int(lengths.sum())
            offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
            keys = np.full(n, 7, np.uint64) if t == 0 else (rng.zipf(1.2, n) % spec.rows).astype(np.uint64)
            pooling = [W.MEAN, W.SUM, W.WEIGHTED_SUM][t]
            weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
            grad = rng.normal(0, 1e-2, (len(lengths), spec.dim)).astype(F32)
            feats.append(W.Feature(t, t, pooling, keys, offsets, lengths.astype(np.uint64), weights, grad))
        print(f"case: refs={refs} step={step}", flush=True)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        shard.prepare(dev)
        status = shard.push(dev)
        assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
        for f in feats:
            stores[f.table].prepare(f)
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
        for t, s in enumerate(specs):
            keys = stores[t].keys()
            want, _ = stores[t].read_many(keys)
            got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
            assert_close(got.reshape(want.shape), want, f"state table {t} step {step}", strict_ulp=0)


def long_row_features(W, rng, specs, long_table, long_refs, other_refs):
    """One feature per table, Zipf(1.2) keys (hot rows everywhere); table
    `long_table` takes `long_refs` references, the others `other_refs` each."""
    feats = []
    for t, spec in enumerate(specs):
        refs = long_refs if t == long_table else other_refs
        pooling = [W.SUM, W.MEAN, W.WEIGHTED_SUM, W.SEQUENCE][t % 4]
        lengths = rng.integers(1, 9, int(refs / 4.5) + 1)
        lengths = lengths[: np.searchsorted(np.cumsum(lengths), refs) + 1]
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
        n = int(offsets[-1])
        keys = (rng.zipf(1.2, n) % spec.rows).astype(np.uint64)
        weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
        rows = n if pooling == W.SEQUENCE else len(lengths)
        grad = rng.normal(0, 1e-2, (rows, spec.dim)).astype(F32)
        feats.append(W.Feature(t, t, pooling, keys, offsets, lengths.astype(np.uint64), weights, grad))
    return feats


@pytest.mark.parametrize("other_refs", [10_000, 80_000])
def test_push_long_rows_mixed_dims(torch_gpu, pkg, other_refs):
    """A table of 70,000 references makes the hot rows narrow units: 16-column
    units while the push has fewer than 262,144 vector references (90,000),
    32-column units above (310,000).  Tables of dimensions 4, 32, 192 and 256,
    so rows have 1 to 16 units and the units past a row's dimension are
    skipped.  Two steps, every touched row bit-exact against the oracle."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(other_refs)
    specs = [W.TableSpec(i, d, 5000, seed=60 + i) for i, d in enumerate((4, 32, 192, 256))]
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    stores = [oracle_store(s) for s in specs]
    for step in range(2):
        feats = long_row_features(W, rng, specs, 2, 70_000, other_refs)
        total = sum(len(f.keys) for f in feats)
        assert (total < 262_144) == (other_refs == 10_000), total  # 16- or 32-column units
        print(f"case: other_refs={other_refs} step={step} refs={[len(f.keys) for f in feats]}", flush=True)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        shard.prepare(dev)
        status = shard.push(dev)
        assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
        for f in feats:
            stores[f.table].prepare(f)
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
        for t, s in enumerate(specs):
            keys = stores[t].keys()
            want, _ = stores[t].read_many(keys)
            got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
            assert_close(got.reshape(want.shape), want, f"state table {t} step {step}", strict_ulp=0)


@pytest.mark.parametrize("pooling", [0, 1, 3])
def test_push_with_long_runs_of_empty_bags(torch_gpu, pkg, pooling):
    """Thousands of bags and a run of 3000 empty ones: several preparation
    blocks per feature, one of which spans the empty run (its bag search
    cannot stage the run and takes the global search)."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(7 + pooling)
    specs = [W.TableSpec(0, 32, 3000, seed=41)]
    bags = 6000
    lengths = rng.integers(1, 9, bags)
    lengths[1500:4500] = 0
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
    n = int(offsets[-1])
    keys = (rng.zipf(1.1, n) % specs[0].rows).astype(np.uint64)
    valid = lengths.astype(np.uint64)
    weights = rng.random(n).astype(F32) if pooling == W.WEIGHTED_SUM else None
    grad = rng.normal(0, 1e-2, (bags, 32)).astype(F32)
    feats = [W.Feature(0, 0, pooling, keys, offsets, valid, weights, grad)]
    print(f"case: pooling={pooling} occurrences={n}", flush=True)
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    dev = [H.DeviceFeature(torch, f) for f in feats]
    shard.prepare(dev)
    shard.push(dev)
    status = shard.status()
    assert status & H.STATUS_ERRORS == 0, f"status {status:#x}"
    store = oracle_store(specs[0])
    store.prepare(feats[0])
    assert oracle.push([store], feats, [0], [grad]) == 0
    keys_done = store.keys()
    want, _ = store.read_many(keys_done)
    got = shard.read_rows(0, torch.from_numpy(keys_done.view(np.int64)).cuda()).cpu().numpy()
    assert_close(got.reshape(want.shape), want, "state after push", strict_ulp=0)


def test_overflow_rejects_whole_push(torch_gpu, pkg):
    """core_tests.cpp:214-222 / cuda_tests.cpp:131-139: an overflowing update
    leaves every row untouched; non-finite gradients and bad slots likewise."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(7)
    specs = [W.TableSpec(0, 64, 3000, seed=1), W.TableSpec(1, 32, 3000, seed=2)]
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    everything = [torch.arange(3000, device="cuda") for _ in specs]
    before = [shard.read_rows(t, everything[t]).clone() for t in range(2)]
    for case in ("flt_max", "nan_in_empty_bag", "bad_slot"):
        feats = random_features(W, rng, specs, 4)
        if case == "flt_max":
            feats[2].gradient[0, 0] = np.finfo(F32).max
            feats[2].gradient[-1, -1] = np.finfo(F32).max
        elif case == "nan_in_empty_bag":
            f = feats[1]
            empty = np.nonzero(np.diff(f.offsets) == 0)[0]
            row = int(empty[0]) if len(empty) and f.pooling != W.SEQUENCE else 0
            f.gradient[row, 3] = np.nan
        else:
            feats[3].keys[5] = np.uint64(specs[feats[3].table].rows + 7)
        dev = [H.DeviceFeature(torch, f) for f in feats]
        shard.prepare(dev)
        shard.push(dev, advance=False)
        status = shard.status()
        print(f"case {case}: status {status:#x}")
        assert status & H.STATUS_ERRORS, case
        for t in range(2):
            assert torch.equal(shard.read_rows(t, everything[t]), before[t]), f"{case}: partial update"


def test_checked_path_when_guard_cannot_prove_safety(torch_gpu, pkg):
    """Gradients of 1e17 make the guard's v' bound exceed 1e30 while no value
    overflows: the validate-then-apply path must give the oracle's result."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(8)
    specs = [W.TableSpec(0, 64, 2000, seed=3)]
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    store = oracle_store(specs[0])
    feats = random_features(W, rng, specs, 3, grad_scale=1e17)
    dev = [H.DeviceFeature(torch, f) for f in feats]
    shard.prepare(dev)
    shard.push(dev)
    status = shard.status()
    assert status & H.STATUS_CHECKED_PATH and not status & H.STATUS_ERRORS, f"{status:#x}"
    for f in feats:
        store.prepare(f)
    assert oracle.push([store], feats, [0] * 3, [f.gradient for f in feats]) == 0
    keys = store.keys()
    want, _ = store.read_many(keys)
    got = shard.read_rows(0, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
    assert_close(got.reshape(want.shape), want, "checked path state", strict_ulp=0)


def test_backend_updates_match_host_backend(torch_gpu, pkg):
    """ApplyHost (7 steps) then ApplyCompact (2 steps, CSR {0,3,4,6,7}) on a
    bounded dim-128 table, as tests/cuda_tests.cpp:104-121, against the
    HostCacheBackend arithmetic; then overflow rejections leave state unchanged."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    dim, rows = 128, 4
    spec = W.TableSpec(1, dim, 8, lr=0.01, bounds=(-0.015, 0.015), seed=42)
    shard = H.DeviceShard(torch, [spec])
    k = np.arange(1, rows + 1)
    w = (F32(0.05) * np.sin((k[:, None] * 7 + np.arange(dim)[None, :]).astype(F32))).astype(F32)
    m = np.tile((F32(0.001) * (np.arange(dim) % 5)).astype(F32), (rows, 1))
    v = np.tile((F32(0.002) * (1 + np.arange(dim) % 3)).astype(F32), (rows, 1))
    slots_np = np.array([7, 0, 3, 5], np.int64)  # arbitrary device slots for keys 1..4
    slots = torch.from_numpy(slots_np).cuda()
    shard.load_rows(0, slots, torch.from_numpy(np.concatenate([w, m, v], 1)).cuda())
    b1p, b2p = F32(0.9), F32(0.999)
    for step in range(7):
        g = (F32(0.03) * np.cos((k[:, None] + np.arange(dim)[None, :] + step).astype(F32))).astype(F32)
        opt = H.Optimizer(0.01, 0.9, 0.999, 1e-8, float(b1p), float(b2p), 1, -0.015, 0.015)
        assert shard.adam_rows(0, slots, torch.from_numpy(g).cuda(), opt) & H.STATUS_ERRORS == 0
        rc, w, m, v = oracle.adam_rows_ctx(w, m, v, g, 0.9, 0.999, 1e-8, 0.01, b1p, b2p, (-0.015, 0.015))
        assert rc == 0
        b1p, b2p = F32(b1p * F32(0.9)), F32(b2p * F32(0.999))
    got = shard.read_rows(0, slots).cpu().numpy()
    assert_close(got, np.concatenate([w, m, v], 1), "ApplyHost x7", strict_ulp=0)
    offsets = np.array([0, 3, 4, 6, 7], np.uint64)
    sources = np.array([0, 1, 0, 2, 1, 2, 0], np.uint64)
    scales = np.array([1 / 3, 0.5, 1 / 3, 1, 0.25, 0.25, 1], F32)
    sv = np.array([[F32(0.01) * np.sin(F32(s * 11 + d)) for d in range(dim)] for s in range(3)], F32)
    for step in range(2):
        opt = H.Optimizer(0.01, 0.9, 0.999, 1e-8, float(b1p), float(b2p), 1, -0.015, 0.015)
        st = shard.adam_compact(0, slots, torch.from_numpy(offsets.view(np.int64)).cuda(),
                                torch.from_numpy(sources.view(np.int64)).cuda(),
                                torch.from_numpy(scales).cuda(), torch.from_numpy(sv).cuda(), opt)
        assert st & H.STATUS_ERRORS == 0
        g = oracle.expand_compact([1, 2, 3, 4], dim, sv, offsets, sources, scales)
        rc, w, m, v = oracle.adam_rows_ctx(w, m, v, g, 0.9, 0.999, 1e-8, 0.01, b1p, b2p, (-0.015, 0.015))
        assert rc == 0
        b1p, b2p = F32(b1p * F32(0.9)), F32(b2p * F32(0.999))
    got = shard.read_rows(0, slots).cpu().numpy()
    assert_close(got, np.concatenate([w, m, v], 1), "ApplyCompact x2", strict_ulp=0)
    assert (np.abs(got[:, :dim]) == F32(0.015)).any(), "clipping not exercised"
    opt = H.Optimizer(0.01, 0.9, 0.999, 1e-8, float(b1p), float(b2p), 1, -0.015, 0.015)
    bad_sv = np.full_like(sv, np.finfo(F32).max)
    st = shard.adam_compact(0, slots, torch.from_numpy(offsets.view(np.int64)).cuda(),
                            torch.from_numpy(sources.view(np.int64)).cuda(),
                            torch.from_numpy(scales).cuda(), torch.from_numpy(bad_sv).cuda(), opt)
    assert st & H.STATUS_ERRORS
    bad = np.ones((rows, dim), F32)
    bad[-1, -1] = np.finfo(F32).max
    assert shard.adam_rows(0, slots, torch.from_numpy(bad).cuda(), opt) & H.STATUS_ERRORS
    assert np.array_equal(shard.read_rows(0, slots).cpu().numpy(), got)
