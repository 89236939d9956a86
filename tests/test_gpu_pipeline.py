"""The benchmarked pipeline against the serial path and the oracle.

bench.py times pipeline.StepPipeline: the push's preparation on a side stream
up to WORKSPACES - 1 batches ahead, WORKSPACES rotating workspaces, and the push split into
begin/apply/end with timing events around the fused pass.  This runs that
exact step for 8 steps of the 26 x 1,000,000 x 64 workload (4 batches cycled,
as the bench does) and requires:

  * no failure in any workspace's status history;
  * every table bit-identical to the serial path (prepare then push on one
    stream with one workspace, status read after every push), and the same
    optimizer powers;
  * the last step's pooled outputs identical to the serial path's;
  * every touched row equal to the oracle (0 ULP), with the per-element ULP
    histograms appended to $EPS_PARITY_REPORT (one JSON line) when that is set.
"""
import json
import os
import time

import numpy as np
import pytest

import oracle
from parity import assert_close, expected_pull, oracle_store, ulp_histogram

pytestmark = pytest.mark.gpu
STEPS = 8
BATCHES = 4


def test_bench_pipeline_matches_serial_and_oracle(torch_gpu, pkg):
    torch, W, H, P = torch_gpu, pkg.workloads, pkg.eps_hip, pkg.pipeline
    t0 = time.time()
    wl = W.Criteo26()
    batches = [wl.batch(i) for i in range(BATCHES)]
    most = max(sum(len(f.keys) for f in b) for b in batches)
    dev = [[H.DeviceFeature(torch, f) for f in b] for b in batches]
    print(f"case: criteo26 pipeline, {STEPS} steps ({time.time() - t0:.1f}s)", flush=True)

    piped = H.DeviceShard(torch, wl.tables, max_occurrences=most, workspaces=P.WORKSPACES)
    piped.init_rows()
    outputs = [torch.empty((wl.batch_size, t.dim), dtype=torch.float32, device="cuda") for t in wl.tables]
    pipe = P.StepPipeline(torch, piped, dev, outputs)
    for k in range(STEPS):
        pipe.step(k)
    pipe.check()
    torch.cuda.synchronize()
    print(f"pipelined steps done ({time.time() - t0:.1f}s)", flush=True)

    serial = H.DeviceShard(torch, wl.tables, max_occurrences=most)
    serial.init_rows()
    for k in range(STEPS):
        feats = dev[k % BATCHES]
        last = serial.lookup(feats)
        serial.prepare(feats)
        status = serial.push(feats)
        assert status & H.STATUS_ERRORS == 0, f"serial step {k}: {status:#x}"
    torch.cuda.synchronize()
    for t in range(len(wl.tables)):
        assert torch.equal(piped.state[t], serial.state[t]), f"table {t}: pipelined state differs"
    assert np.array_equal(piped.powers, serial.powers)
    for t, (a, b) in enumerate(zip(outputs, last)):
        assert torch.equal(a, b), f"table {t}: pipelined pull differs"
    print(f"pipelined == serial ({time.time() - t0:.1f}s)", flush=True)

    stores = [oracle_store(t) for t in wl.tables]
    report = {"workload": "criteo26 (26 x 1,000,000 x 64), 8 pipelined steps, 4 batches cycled",
              "pull_last_step": {}, "state": {}}
    for k in range(STEPS):
        feats = batches[k % BATCHES]
        for f in feats:
            want = expected_pull(stores[f.table], f)
            if k == STEPS - 1:
                got = outputs[f.table].cpu().numpy()
                hist, worst = ulp_histogram(got, want)
                report["pull_last_step"][f.table] = {"histogram": hist, "max_ulp": worst}
                assert_close(got, want, f"pull step {k} table {f.table}", strict_ulp=0)
        assert oracle.push(stores, feats, [f.table for f in feats], [f.gradient for f in feats]) == 0
    print(f"oracle done ({time.time() - t0:.1f}s)", flush=True)
    for t, spec in enumerate(wl.tables):
        keys = stores[t].keys()
        want, _ = stores[t].read_many(keys)
        got = piped.read_rows(t, torch.from_numpy(keys.view(np.int64)).cuda()).cpu().numpy()
        got = got.reshape(want.shape)
        hist, worst = ulp_histogram(got, want)
        report["state"][t] = {"rows": int(len(keys)), "histogram": hist, "max_ulp": worst}
        assert_close(got, want, f"state table {t}", strict_ulp=0)
        assert tuple(piped.powers[t]) == stores[t].powers()[:2]
    path = os.environ.get("EPS_PARITY_REPORT")
    if path:
        with open(path, "a") as out:  # one JSON line beside the per-comparison lines
            out.write(json.dumps({"what": "bench pipeline summary", **report}) + "\n")
    print(f"oracle parity ok ({time.time() - t0:.1f}s)", flush=True)
