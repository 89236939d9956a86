"""Parity helpers shared by the GPU tests (the oracle is the checker).

Floating-point results are held to the contract tolerance (1e-5 relative or
1e-6 absolute per element) and their per-element ULP histogram is reported;
integer results (slots, unique ids, occurrence maps) must be identical.
With EPS_PARITY_REPORT set to a file path, every comparison also appends one
JSON line (what, elements, histogram, worst ULP) to that file.
"""
import json
import os

import numpy as np

import oracle

RTOL, ATOL = 1e-5, 1e-6


def ordered(a):
    i = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def ulp_histogram(got, want):
    d = np.abs(ordered(got) - ordered(want)).reshape(-1)
    edges = [0, 1, 2, 4, 16, 1 << 62]
    counts = [int(np.sum((d >= lo) & (d < hi))) for lo, hi in zip(edges[:-1], edges[1:])]
    return {"0": counts[0], "1": counts[1], "2-3": counts[2], "4-15": counts[3], ">=16": counts[4]}, int(d.max(initial=0))


def assert_close(got, want, what, strict_ulp=None):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    hist, worst = ulp_histogram(got, want)
    print(f"{what}: ULP histogram {hist}")
    report = os.environ.get("EPS_PARITY_REPORT")
    if report:
        with open(report, "a") as fh:
            fh.write(json.dumps({"what": what, "elements": int(got.size), "ulp_histogram": hist,
                                 "max_ulp": worst}) + "\n")
    ok = np.abs(got.astype(np.float64) - want) <= np.maximum(ATOL, RTOL * np.abs(want.astype(np.float64)))
    assert ok.all(), f"{what}: {int((~ok).sum())} elements outside 1e-5 rel / 1e-6 abs (max ULP {worst})"
    if strict_ulp is not None:
        assert worst <= strict_ulp, f"{what}: max ULP {worst} > {strict_ulp}"
    return worst


def oracle_store(spec):
    return oracle.Store(oracle.table_def(
        id=spec.id, dim=spec.dim, lr=spec.lr, beta1=spec.beta1, beta2=spec.beta2, eps=spec.eps,
        b1p=spec.b1p, b2p=spec.b2p, bounds=spec.bounds, init_min=spec.init_min,
        init_max=spec.init_max, seed=spec.seed))


def expected_pull(store, feature):
    """Pooled output of the CPU shard + client (mean divided once)."""
    _, _, contribution = store.prepare(feature)
    if feature.pooling == oracle.MEAN:
        return oracle.mean_divide(contribution, feature.valid_lengths)
    return contribution
