"""Pooled gather on the GPU vs the oracle (GatherHost / PrepareFeature + client mean)."""
import numpy as np
import pytest

import oracle
from parity import assert_close, oracle_store

pytestmark = pytest.mark.gpu
HOLE = np.uint64(2**64 - 1)


def random_feature(W, rng, spec, pooling, bags=300, max_len=12, holes=0.05, pad=0.2):
    lengths = rng.integers(0, max_len + 1, bags)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
    n = int(offsets[-1])
    keys = (rng.zipf(1.2, n) % spec.rows).astype(np.uint64)
    keys[rng.random(n) < holes] = HOLE
    valid = (lengths + (rng.random(bags) < pad) * rng.integers(1, 4, bags)).astype(np.uint64)
    weights = rng.random(n).astype(np.float32) if pooling == W.WEIGHTED_SUM else None
    return W.Feature(0, 0, pooling, keys, offsets, valid, weights)


def expected(store, f, dim):
    """HostCacheBackend::GatherHost over the non-hole occurrences, then the
    client mean divide."""
    live = f.keys != HOLE
    uniq, first = np.unique(f.keys[live], return_index=True)
    order = uniq[np.argsort(first)]
    index = {int(k): i for i, k in enumerate(order)}
    occ = np.array([index[int(k)] if k != HOLE else int(HOLE) for k in f.keys], np.uint64)
    rows = []
    for k in order:
        store.ensure(int(k))
        rows.append(store.read(int(k))[0])
    out = oracle.gather_host(f, dim, occ, rows)
    if f.pooling == oracle.MEAN:
        out = oracle.mean_divide(out, f.valid_lengths)
    return out


@pytest.mark.parametrize("dim", [4, 16, 32, 64, 96, 128, 192, 256, 6, 300])
@pytest.mark.parametrize("pooling", [0, 1, 2, 3])
def test_gather_matches_oracle(torch_gpu, pkg, dim, pooling):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(dim * 10 + pooling)
    spec = W.TableSpec(5, dim, 3000, seed=77 + dim)
    f = random_feature(W, rng, spec, pooling)
    print(f"case: dim={dim} pooling={pooling} occurrences={len(f.keys)}", flush=True)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = shard.lookup([H.DeviceFeature(torch, f)], status=status)[0]
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    want = expected(oracle_store(spec), f, dim)
    assert_close(out.cpu().numpy(), want, f"gather dim={dim} pooling={pooling}", strict_ulp=0)


@pytest.mark.parametrize("dim", [4, 64, 256, 300])
@pytest.mark.parametrize("pooling", [0, 1, 3])
def test_gather_long_bags(torch_gpu, pkg, dim, pooling):
    """Bags of up to 400 occurrences (sum, mean, weighted sum: the pooled
    modes, whose blocks own bags): a block's bags then hold more than the
    1,024 occurrences it stages in LDS, so their slots are resolved per
    occurrence in the summing loop (the gather's unstaged path)."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(500 + dim * 10 + pooling)
    spec = W.TableSpec(3, dim, 3000, seed=91 + dim)
    f = random_feature(W, rng, spec, pooling, bags=90, max_len=400)
    rows_per_block = 8 if dim % 4 or dim > 256 else 256 // max(4, 1 << (dim // 4 - 1).bit_length())
    per_block = [int(f.offsets[min(b + rows_per_block, len(f.valid_lengths))] - f.offsets[b])
                 for b in range(0, len(f.valid_lengths), rows_per_block)]
    assert max(per_block) > 1024, per_block  # at least one unstaged block
    print(f"case: dim={dim} pooling={pooling} occurrences={len(f.keys)} block max {max(per_block)}", flush=True)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = shard.lookup([H.DeviceFeature(torch, f)], status=status)[0]
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    want = expected(oracle_store(spec), f, dim)
    assert_close(out.cpu().numpy(), want, f"long bags dim={dim} pooling={pooling}", strict_ulp=0)


def test_gather_many_parts_one_call(torch_gpu, pkg):
    """Up to 32 features of different tables/dims in one launch, 40 -> two calls."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(1)
    dims = [4, 8, 16, 64, 96, 128, 256, 6, 300, 32]
    specs = [W.TableSpec(i, d, 2000 + 100 * i, seed=10 + i) for i, d in enumerate(dims)]
    feats = []
    for i in range(40):
        t = i % len(specs)
        f = random_feature(W, rng, specs[t], [0, 1, 2, 3][i % 4], bags=50 + 7 * (i % 20))
        f.table = t
        feats.append(f)
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    outs = shard.lookup([H.DeviceFeature(torch, f) for f in feats])
    torch.cuda.synchronize()
    stores = [oracle_store(s) for s in specs]
    for i, (f, out) in enumerate(zip(feats, outs)):
        want = expected(stores[f.table], f, specs[f.table].dim)
        assert_close(out.cpu().numpy(), want, f"part {i}", strict_ulp=0)


GATHER_SWEEP_DIMS = [1, 3, 4, 8, 12, 16, 20, 32, 48, 64, 96, 128, 160, 192, 256, 300, 520]


@pytest.mark.parametrize("seed", range(20))
def test_gather_random_sweep(torch_gpu, pkg, seed):
    """Seeded random pulls: 1-8 tables of dimensions 1-520 (vector and generic
    shapes), 1-40 features of every pooling (past 32, the pull takes two
    launches), bag counts, bag lengths (up to long bags past what a block
    stages), hole and padded-length rates all drawn per case; every output
    bit-exact against the oracle."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(7000 + seed)
    n_tables = int(rng.integers(1, 9))
    specs = [W.TableSpec(i, int(rng.choice(GATHER_SWEEP_DIMS)), int(rng.integers(50, 5000)), seed=300 + seed * 10 + i)
             for i in range(n_tables)]
    feats = []
    for i in range(int(rng.integers(1, 41))):
        t = int(rng.integers(0, n_tables))
        max_len = int(rng.choice([0, 3, 12, 40, 200]))
        f = random_feature(W, rng, specs[t], int(rng.integers(0, 4)), bags=int(rng.integers(1, 400)),
                           max_len=max_len, holes=float(rng.choice([0.0, 0.05, 0.3])),
                           pad=float(rng.choice([0.0, 0.2, 0.6])))
        f.table = t
        feats.append(f)
    print(f"case: seed={seed} dims={[s.dim for s in specs]} features={len(feats)} "
          f"occurrences={sum(len(f.keys) for f in feats)}", flush=True)
    shard = H.DeviceShard(torch, specs)
    shard.init_rows()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = shard.lookup([H.DeviceFeature(torch, f) for f in feats], status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    stores = [oracle_store(s) for s in specs]
    for i, (f, out) in enumerate(zip(feats, outs)):
        want = expected(stores[f.table], f, specs[f.table].dim)
        assert_close(out.cpu().numpy(), want, f"seed {seed} feature {i}", strict_ulp=0)


def test_gather_remap_and_transferred_vectors(torch_gpu, pkg):
    """transfer_unique route: source = unique vectors (stride dim), indices are
    unique indices mapped through `remap` (cache_backend.cu:264-300)."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    import ctypes as C
    rng = np.random.default_rng(2)
    dim, uniq = 64, 37
    vectors = rng.normal(size=(uniq, dim)).astype(np.float32)
    occ = rng.integers(0, uniq, 400).astype(np.uint64)
    occ[::17] = HOLE
    lengths = rng.multinomial(400, np.full(60, 1 / 60))
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
    perm = rng.permutation(uniq).astype(np.uint64)  # unique -> row of `vectors`
    src = torch.from_numpy(vectors).cuda()
    idx = torch.from_numpy(occ.view(np.int64)).cuda()
    remap = torch.from_numpy(perm.view(np.int64)).cuda()
    off = torch.from_numpy(offsets.view(np.int64)).cuda()
    out = torch.empty((len(lengths), dim), dtype=torch.float32, device="cuda")
    part = H.GatherPart(src.data_ptr(), idx.data_ptr(), remap.data_ptr(), off.data_ptr(), None, None,
                        out.data_ptr(), dim, len(lengths), uniq, uniq, dim, W.SUM)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    H.check(H.lib().eps_hip_gather(C.byref(part), 1, C.c_void_p(status.data_ptr()),
                                   C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    f = W.Feature(0, 0, W.SUM, np.zeros(400, np.uint64), offsets, lengths.astype(np.uint64))
    want = oracle.gather_host(f, dim, occ, [vectors[int(perm[u])] for u in range(uniq)])
    assert_close(out.cpu().numpy(), want, "remapped gather", strict_ulp=0)


def test_gather_out_of_range_slot_is_reported_and_skipped(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    spec = W.TableSpec(1, 16, 100, seed=3)
    keys = np.array([1, 2, 100, 5, 10**9], np.uint64)  # 100 and 10^9 are out of range
    f = W.Feature(0, 0, W.SUM, keys, np.array([0, 3, 5], np.uint64), np.array([3, 2], np.uint64))
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = shard.lookup([H.DeviceFeature(torch, f)], status=status)[0]
    torch.cuda.synchronize()
    assert int(status.item()) & H.STATUS_BAD_INDEX
    store = oracle_store(spec)
    ok = W.Feature(0, 0, W.SUM, np.array([1, 2, 5], np.uint64), np.array([0, 2, 3], np.uint64),
                   np.array([2, 1], np.uint64))
    _, _, want = store.prepare(ok)
    assert_close(out.cpu().numpy(), want, "skipped out-of-range slots", strict_ulp=0)


def test_empty_and_zero_length(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    spec = W.TableSpec(1, 32, 100, seed=3)
    shard = H.DeviceShard(torch, [spec])
    shard.init_rows()
    f = W.Feature(0, 0, W.MEAN, np.zeros(0, np.uint64), np.zeros(4, np.uint64), np.zeros(3, np.uint64))
    out = shard.lookup([H.DeviceFeature(torch, f)])[0]
    torch.cuda.synchronize()
    assert out.shape == (3, 32) and not out.any()


def test_state_rows_round_trip_and_pinned_admission(torch_gpu, pkg):
    """Load (ScatterState) from pinned host memory and ReadBack (ReadStateKernel)."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    rng = np.random.default_rng(9)
    for dim in (64, 6):
        spec = W.TableSpec(2, dim, 1000, seed=5)
        shard = H.DeviceShard(torch, [spec])
        shard.init_rows()
        slots = rng.choice(1000, 200, replace=False).astype(np.int64)
        packed = rng.normal(size=(200, 3 * dim)).astype(np.float32)
        packed[:, 2 * dim:] = np.abs(packed[:, 2 * dim:])
        host = torch.from_numpy(packed).pin_memory()
        s = torch.from_numpy(slots).cuda()
        shard.load_rows(0, s, host)
        back = shard.read_rows(0, s).cpu().numpy()
        assert np.array_equal(back.view(np.uint32), packed.view(np.uint32))
        pinned_out = torch.empty((200, 3 * dim), dtype=torch.float32).pin_memory()
        shard.read_rows(0, s, out=pinned_out)
        torch.cuda.synchronize()
        assert np.array_equal(pinned_out.numpy().view(np.uint32), packed.view(np.uint32))
        # Untouched slots keep the initializer's rows.
        other = np.setdiff1d(np.arange(1000), slots)[:50]
        rows = shard.read_rows(0, torch.from_numpy(other).cuda()).cpu().numpy()
        store = oracle_store(spec)
        for r, k in zip(rows, other):
            store.ensure(int(k))
            assert np.array_equal(r[:dim], store.read(int(k))[0]) and not r[dim:].any()
