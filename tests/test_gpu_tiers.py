"""Config-5 cache-tier row moves at full size, through the benchmarked pipeline.

8 ragged tables (dims 16..256, 100k..5M rows), 8192 weighted-sum bags per
table, Poisson(8) lengths, Zipf(1.05).  Every step admits 5% of its touched
rows' expected count per table from pinned host memory (w, m and v) and
writes back as many rows to pinned host memory, on two copy streams that
overlap the steps (pipeline.TierMoves; the reference's Load / ReadBack /
CommitEviction, src/cuda/cache_backend.cu:390-462,540-599).  Written-back slots
are overwritten with 7.0 until their admission, so a row that did not make
the round trip shows up.  After 6 steps, against the oracle (one CPU shard
holding every row, which the two tiers together must equal):

  * the last step's pooled outputs (0 ULP);
  * every touched row resident on the device (0 ULP);
  * every row still in host memory (written back, not yet admitted) (0 ULP).
"""
import time

import numpy as np
import pytest

import oracle
from parity import assert_close, expected_pull, oracle_store

pytestmark = pytest.mark.gpu
STEPS = 6
BATCHES = 4


def test_ragged8_tier_moves_full_size(torch_gpu, pkg):
    torch, W, H, P = torch_gpu, pkg.workloads, pkg.eps_hip, pkg.pipeline
    t0 = time.time()
    wl = W.Ragged8()
    batches = [wl.batch(i) for i in range(BATCHES)]
    touched = [[np.unique(f.keys) for f in b] for b in batches]
    admissions = wl.admissions(touched)
    counts = wl.move_counts()
    print(f"case: ragged8 tier moves, {STEPS} steps, admitted rows per step {sum(counts)} "
          f"({time.time() - t0:.1f}s)", flush=True)
    most = max(sum(len(f.keys) for f in b) for b in batches)
    shard = H.DeviceShard(torch, wl.tables, max_occurrences=most, workspaces=P.WORKSPACES)
    shard.init_rows()
    dev = [[H.DeviceFeature(torch, f) for f in b] for b in batches]
    outputs = [torch.empty((wl.bags, t.dim), dtype=torch.float32, device="cuda") for t in wl.tables]
    moves = P.TierMoves(torch, shard, admissions, wl.MOVE_LAG, poison=True)
    moves.prime()
    pipe = P.StepPipeline(torch, shard, dev, outputs, moves=moves)
    for k in range(STEPS):
        pipe.step(k)
    pipe.check()
    torch.cuda.synchronize()
    print(f"device steps done, {moves.bytes / 1e6:.1f} MB each way per step ({time.time() - t0:.1f}s)",
          flush=True)

    stores = [oracle_store(t) for t in wl.tables]
    for k in range(STEPS):
        feats = batches[k % BATCHES]
        for f in feats:
            want = expected_pull(stores[f.table], f)
            if k == STEPS - 1:
                assert_close(outputs[f.table].cpu().numpy(), want, f"pull step {k} table {f.table}",
                             strict_ulp=0)
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
    print(f"oracle done ({time.time() - t0:.1f}s)", flush=True)

    # Rows written back after the last MOVE_LAG steps wait in host memory.
    pending = {}
    for j in range(STEPS, STEPS + wl.MOVE_LAG):
        host = moves.host[j % (wl.MOVE_LAG + 1)].numpy()
        for t, spec in enumerate(wl.tables):
            keys = admissions[j % BATCHES][t]
            rows = host[int(moves.offset[t]):int(moves.offset[t + 1])].reshape(len(keys), 3 * spec.dim)
            for key, row in zip(keys, rows):
                pending[(t, int(key))] = row
    for t, spec in enumerate(wl.tables):
        keys = stores[t].keys()
        want, _ = stores[t].read_many(keys)
        want = want.reshape(len(keys), 3 * spec.dim)
        got = shard.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
        in_host = np.array([(t, int(k)) in pending for k in keys])
        for i in np.nonzero(in_host)[0]:
            got[i] = pending[(t, int(keys[i]))]
        assert in_host.sum() == sum(1 for key in pending if key[0] == t), \
            f"table {t}: a pending row was never touched"
        assert_close(got, want, f"table {t}: {len(keys)} touched rows ({int(in_host.sum())} in host memory)",
                     strict_ulp=0)
    print(f"tier parity ok ({time.time() - t0:.1f}s)", flush=True)
