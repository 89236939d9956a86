#!/usr/bin/env python3
"""Benchmark of the parameter-shard embedding step on one MI355X.

Workload: 26 fp32 tables x 1,000,000 rows x dim 64, batch 4096 bags per table,
bag length U{1..20}, ids Zipf(1.05); tables 0-12 sum pooling, 13-25 mean;
per-bag gradients N(0, 1e-2); sparse Adam lr 1e-3, betas 0.9/0.999, eps 1e-8.
One step = pooled pull of every table + device dedup of the lookup (radix sort,
on a second stream, running ahead of the pull and push) + fused duplicate-id
aggregation and Adam of every unique row.  Inputs (ids,
offsets, lengths, gradients) are resident in HBM before the timed region;
several pre-generated batches are cycled.

Prints one JSON line (rank 0).  `value` is pooled lookups/s; Adam rows/s, the
step's algorithmic HBM bandwidth and its fraction of the 8 TB/s peak ride
along.  `roofline` is the fused update kernel's own (HIP events on its stream);
`cpu_baseline` times the reference CPU shard on the host over a bounded sample.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from __graft_entry__ import package  # noqa: E402

METRIC = "pooled lookups/s + Adam rows/s on 1 GPU; achieved HBM GB/s (% of peak)"
HBM_PEAK_GBPS = 8000.0
PROFILE_SUMMARY = ROOT / "profiles" / "fused_update_criteo26.md"
COPY_BYTES = 1 << 30
FUSED_EVERY = 5  # timed steps between two timings of the fused update


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def batch_stats(wl, feats):
    unique = [len(np.unique(f.keys)) for f in feats]
    lookups = sum(len(f.keys) for f in feats)
    bags = sum(len(f.valid_lengths) for f in feats)
    pull, push = wl_bytes(wl, feats, unique)
    fused = sum(u * wl.tables[f.table].dim * 24 + f.rows * wl.tables[f.table].dim * 4
                for f, u in zip(feats, unique))
    return dict(lookups=lookups, unique=sum(unique), bags=bags, pull_bytes=pull, push_bytes=push,
                fused_bytes=fused)


def wl_bytes(wl, feats, unique):
    W = package().workloads
    return W.algorithmic_bytes(wl.tables, feats, unique)


def cpu_baseline(wl, batches, budget_s=15.0, max_steps=8):
    """Reference CPU shard (Lookup: PrepareFeature + client mean; Push:
    ReduceGradients + ValidateLazyAdam + ApplyLazyAdam) on one core."""
    import oracle

    if oracle.ref_available():
        kind = "reference"
        defs = [oracle.table_def(id=t.id, dim=t.dim, lr=t.lr, b1p=t.b1p, b2p=t.b2p,
                                 init_min=t.init_min, init_max=t.init_max, seed=t.seed)
                for t in wl.tables]
        shard = oracle.RefShard(defs)

        def step(feats):
            for f in feats:
                _, _, c = shard.prepare(wl.tables[f.table].id, f)
                if f.pooling == oracle.MEAN:
                    oracle.mean_divide(c, f.valid_lengths)
            assert shard.push([f.gradient for f in feats]) == 0
    else:
        kind = "port"
        stores = [oracle.Store(oracle.table_def(id=t.id, dim=t.dim, lr=t.lr, b1p=t.b1p, b2p=t.b2p,
                                                init_min=t.init_min, init_max=t.init_max,
                                                seed=t.seed)) for t in wl.tables]

        def step(feats):
            for f in feats:
                _, _, c = stores[f.table].prepare(f)
                if f.pooling == oracle.MEAN:
                    oracle.mean_divide(c, f.valid_lengths)
            assert oracle.push(stores, feats, [f.table for f in feats],
                               [f.gradient for f in feats]) == 0

    step(batches[0])  # first touch of the hot rows, untimed
    done, lookups, rows, t0 = 0, 0, 0, time.perf_counter()
    while done < max_steps and (time.perf_counter() - t0) < budget_s:
        feats = batches[(done + 1) % len(batches)]
        step(feats)
        lookups += sum(len(f.keys) for f in feats)
        rows += sum(len(np.unique(f.keys)) for f in feats)
        done += 1
    elapsed = time.perf_counter() - t0
    return {"value": lookups / elapsed, "unit": "lookups/s", "cores": 1, "kind": kind,
            "adam_rows_per_s": rows / elapsed, "ms_per_step": 1e3 * elapsed / done,
            "cpu": cpu_model(),
            "sample": f"{done} steps of the same workload after one untimed first-touch step, "
                      f"one shard on one thread ({'reference sources' if kind == 'reference' else 'C restatement'})"}


class _ShardFeature:
    """One shard's part of a feature: its keys (key % shards == shard) with the
    bags' offsets recounted and the original valid lengths kept, as the
    reference client routes a lookup (src/access/prepared_lookup.cpp:47-83)."""

    def __init__(self, f, shard, shards):
        keys = np.asarray(f.keys, np.uint64)
        mine = keys % np.uint64(shards) == np.uint64(shard)
        counts = np.add.reduceat(mine.astype(np.uint64), np.asarray(f.offsets[:-1], np.int64)) \
            if len(keys) else np.zeros(len(f.valid_lengths), np.uint64)
        counts[np.asarray(f.offsets[1:]) == np.asarray(f.offsets[:-1])] = 0  # empty bags
        self.keys = keys[mine]
        self.offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint64)
        self.valid_lengths = np.asarray(f.valid_lengths, np.uint64)
        self.pooling, self.feature, self.table, self.weights = f.pooling, f.feature, f.table, None
        self.gradient = f.gradient[mine] if f.pooling == 2 else f.gradient  # sequence rows follow keys

    @property
    def rows(self):
        return len(self.keys) if self.pooling == 2 else len(self.valid_lengths)


def cpu_baseline_shards(wl, batches, shards, budget_s=10.0, max_steps=8):
    """The reference's own scale-out on the host: `shards` CPU shards (the
    reference sources), one thread each, keys routed by key % shards; each
    shard runs PrepareFeature and Push on its part, the client adds the
    partial sums and divides the means.  Routing is done before timing."""
    import threading

    import oracle

    if not oracle.ref_available():
        return None
    refs = [oracle.RefShard([oracle.table_def(id=t.id, dim=t.dim, lr=t.lr, b1p=t.b1p, b2p=t.b2p,
                                              init_min=t.init_min, init_max=t.init_max, seed=t.seed,
                                              shard=i, shard_count=shards) for t in wl.tables],
                            shard=i, shard_count=shards) for i in range(shards)]
    parts = [[[_ShardFeature(f, i, shards) for f in feats] for i in range(shards)] for feats in batches]

    def step(k):
        outs, errors = [None] * shards, []

        def run(i):
            try:
                out = []
                for f in parts[k][i]:
                    out.append(refs[i].prepare(wl.tables[f.table].id, f)[2])
                if refs[i].push([f.gradient for f in parts[k][i]]) != 0:
                    raise RuntimeError(f"reference shard {i} rejected its push: {refs[i].error()}")
                outs[i] = out
            except Exception as e:  # surfaced on the calling thread
                errors.append(e)

        threads = [threading.Thread(target=run, args=(i,)) for i in range(shards)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        if errors:
            raise errors[0]
        for j, f in enumerate(batches[k]):  # client merge and mean divide
            total = outs[0][j].copy()
            for i in range(1, shards):
                total += outs[i][j]
            if f.pooling == oracle.MEAN:
                oracle.mean_divide(total, f.valid_lengths)

    step(0)  # first touch, untimed
    done, lookups, t0 = 0, 0, time.perf_counter()
    while done < max_steps and (time.perf_counter() - t0) < budget_s:
        k = (done + 1) % len(batches)
        step(k)
        lookups += sum(len(f.keys) for f in batches[k])
        done += 1
    elapsed = time.perf_counter() - t0
    return {"value": lookups / elapsed, "unit": "lookups/s", "cores": shards,
            "ms_per_step": 1e3 * elapsed / done,
            "sample": f"{done} steps after one untimed first-touch step, {shards} reference shards "
                      f"on {shards} threads, key % {shards} routing done before timing"}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batches", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run three plain 1 GiB device copies (counter calibration)")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): the parameter shard runs on a "
              "single MI355X here; multi-GPU sharding is not built.", file=sys.stderr)
        return 2

    import torch

    if args.copy_calibration:
        # A copy of known size: the FETCH_SIZE / WRITE_SIZE reading of this
        # kernel divided by 1 GiB is the counter's scale for HBM bytes.
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    pkg = package()
    W, H = pkg.workloads, pkg.eps_hip
    wl = W.Criteo26()
    batches = [wl.batch(i) for i in range(args.batches)]
    stats = [batch_stats(wl, b) for b in batches]
    shard = H.DeviceShard(torch, wl.tables, max_occurrences=max(s["lookups"] for s in stats),
                          workspaces=2)
    shard.init_rows()
    dev = [[H.DeviceFeature(torch, f) for f in b] for b in batches]
    outputs = [torch.empty((wl.batch_size, t.dim), dtype=torch.float32, device="cuda")
               for t in wl.tables]
    stream = torch.cuda.current_stream()

    # Pipeline: the push's preparation (dedup sort and hot-row list) only reads
    # the batch's ids, so it runs on a side stream ahead of the main stream
    # (pull, then push).  Two workspaces alternate: the preparation of batch k
    # waits for the push of batch k-2 (the last reader of its workspace), and
    # the push of batch k waits for its preparation.
    side = torch.cuda.Stream()
    prepared = [torch.cuda.Event() for _ in range(2)]
    pushed = [torch.cuda.Event() for _ in range(2)]

    def step(k, fused=None, phases=None):
        """One step; `fused` = two timing events around the fused update,
        `phases` = seven events for the per-phase breakdown."""
        feats = dev[k % len(dev)]
        slot = k % 2
        side.wait_event(pushed[slot])
        if phases:
            phases[0].record(stream)
            phases[5].record(side)
        shard.prepare(feats, stream=side, slot=slot)
        prepared[slot].record(side)
        if phases:
            phases[6].record(side)
        shard.lookup(feats, outputs, stream=stream)
        if phases:
            phases[1].record(stream)
        stream.wait_event(prepared[slot])
        if phases:
            phases[2].record(stream)
        shard.push(feats, stream=stream, slot=slot,
                   events=fused or (tuple(phases[3:5]) if phases else None))
        pushed[slot].record(stream)

    # Warm-up steps are issued back to back like the timed ones, so whatever
    # the runtime sets up when many launches are outstanding happens here.
    for k in range(args.warmup):
        step(k)
    for slot in range(min(2, args.warmup)):
        status = shard.status(slot=slot)
        assert status & H.STATUS_ERRORS == 0, f"warm-up push status {status:#x}"
    torch.cuda.synchronize()
    # Timed steps carry only the two events around the fused update (its
    # roofline), on every FUSED_EVERY-th step: every timing event costs GPU
    # time on its stream, and many outstanding timing events can stall the
    # host's launches.
    fused = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             if k % FUSED_EVERY == 0 else None for k in range(args.steps)]
    torch.cuda.synchronize()
    gc.disable()  # no collector pause inside the timed region
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(args.warmup + k, fused=fused[k])
    enqueued = time.perf_counter() - t0  # host time to issue the timed steps
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gc.enable()
    for slot in range(2):
        status = shard.status(slot=slot)
        assert status & H.STATUS_ERRORS == 0, f"timed push status {status:#x}"
    # Per-phase breakdown on further (untimed) steps.
    breakdown = min(args.steps, 10)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(7)] for _ in range(breakdown)]
    for k in range(breakdown):
        step(args.warmup + args.steps + k, phases=events[k])
    torch.cuda.synchronize()

    ms = elapsed * 1e3 / args.steps
    used = [stats[(args.warmup + k) % len(stats)] for k in range(args.steps)]
    mean = {key: float(np.mean([u[key] for u in used])) for key in used[0]}
    gather_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in events]))
    prepare_ms = float(np.mean([e[5].elapsed_time(e[6]) for e in events]))  # side stream
    wait_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in events]))
    fused_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in fused if e]))
    push_ms = float(np.mean([e[2].elapsed_time(e[4]) for e in events]))
    step_bytes = mean["pull_bytes"] + mean["push_bytes"]
    achieved = mean["fused_bytes"] / (fused_ms * 1e-3) / 1e9
    traffic = None
    if PROFILE_SUMMARY.exists():
        for line in PROFILE_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = float(line.split(":", 1)[1])
    result = {
        "metric": METRIC,
        "value": mean["lookups"] / (ms * 1e-3),
        "unit": "lookups/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Zipf(1.05) ids, U{1..20} bags, N(0,1e-2) gradients, "
                "reference SplitMix initializer U(-0.05,0.05); inputs resident in HBM",
        "config": {"workload": "26 tables x 1,000,000 rows x dim 64 fp32 (w|m|v AoS), batch 4096 bags "
                               "per table, bag length U{1..20}, Zipf(1.05), 13 sum + 13 mean pooling, "
                               "pull + device dedup + fused sparse Adam (lr 1e-3, 0.9/0.999, 1e-8)",
                   "tables": len(wl.tables), "rows_per_table": wl.tables[0].rows,
                   "dim": wl.tables[0].dim, "batch": wl.batch_size, "batches_cycled": len(batches)},
        "host_enqueue_ms_per_step": enqueued * 1e3 / args.steps,
        "adam_rows_per_s": mean["unique"] / (ms * 1e-3),
        "lookups_per_step": mean["lookups"],
        "adam_rows_per_step": mean["unique"],
        "step_algorithmic_bytes": step_bytes,
        "step_algorithmic_GBps": step_bytes / (ms * 1e-3) / 1e9,
        "step_frac_of_hbm_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "phases_ms": {"gather": gather_ms, "prepare": prepare_ms, "prepare_wait": wait_ms,
                      "push": push_ms, "fused_update": fused_ms,
                      "note": "gather/prepare/prepare_wait/push from untimed steps after the "
                      "timed ones (prepare runs on a side stream, ahead of the pull and push); "
                      "fused_update from every 5th timed step"},
        "roofline": {"kernel": "fused aggregation + sparse Adam (eps_hip_push_apply: "
                               "HotSliceKernel + RowRunKernel)", "bound": "hbm",
                     "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": mean["fused_bytes"],
                     # measured HBM bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)
                     # over the same duration
                     "traffic_GBps": traffic / (fused_ms * 1e-3) / 1e9 if traffic else None},
        # Occurrence-based pull rate: every pooled lookup reads one dim-wide row
        # (N x d x 4 bytes, repeats included, most served by the caches).
        "gather_effective_GBps": mean["lookups"] * wl.tables[0].dim * 4 / (gather_ms * 1e-3) / 1e9,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, batches)
        shards = min(16, os.cpu_count() or 1)  # the host share of one GPU
        if shards > 1:
            all_cores = cpu_baseline_shards(wl, batches, shards)
            if all_cores:
                result["cpu_baseline"]["all_cores"] = all_cores
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
