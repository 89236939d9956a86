"""The allocation-free device push (eps_hip_push_static, its workspace in a
static device array of the library) against eps_hip_prepare + eps_hip_push
with a caller workspace, through the C ABI.

Two identical shards take the same two pushes in a row, the second smaller
than the first (the static array keeps the first call's contents, so what a
call needs at zero must be cleared by the call itself): statuses, every row of
every table, the bounds domain and the optimizer powers must be identical.  A
push above the static maximum (262,144 occurrences) is refused before any work
is enqueued.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def features(W, rng, specs, bags):
    out = []
    for i, pooling in enumerate((W.MEAN, W.SUM, W.WEIGHTED_SUM)):
        t = i % len(specs)
        lengths = rng.integers(1, 21, bags)
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
        n = int(offsets[-1])
        keys = (rng.zipf(1.1, n) % specs[t].rows).astype(np.uint64)  # hot rows: the sliced kernel too
        weights = rng.random(n).astype(np.float32) if pooling == W.WEIGHTED_SUM else None
        grad = rng.normal(0, 1e-2, (bags, specs[t].dim)).astype(np.float32)
        out.append(W.Feature(t, i, pooling, keys, offsets, lengths.astype(np.uint64), weights, grad))
    return out


def test_static_push_matches_workspace_push(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    L = H.lib()
    specs = [W.TableSpec(0, 64, 20000, seed=51), W.TableSpec(1, 128, 8000, seed=52, bounds=(-0.05, 0.06))]
    static, reference = H.DeviceShard(torch, specs), H.DeviceShard(torch, specs)
    static.init_rows()
    reference.init_rows()
    rng = np.random.default_rng(61)
    out = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for call, bags in enumerate((4000, 700)):
        feats = features(W, rng, specs, bags)
        n = sum(len(f.keys) for f in feats)
        print(f"case: call {call}, {bags} bags per feature, {n} occurrences", flush=True)
        assert n <= 262144
        dev = [H.DeviceFeature(torch, f) for f in feats]
        reference.prepare(dev)
        want = reference.push(dev)
        assert want & H.STATUS_ERRORS == 0, f"{want:#x}"
        arr = static._push_args(dev)
        static._opts_view["beta1_power"] = static.powers[:, 0]
        static._opts_view["beta2_power"] = static.powers[:, 1]
        H.check(L.eps_hip_push_static(static.tables, static._opts, len(specs), arr, len(dev),
                                      static.bounds.data_ptr(), out.data_ptr(), stream))
        torch.cuda.synchronize()
        got, history = (int(x) & 0xFFFFFFFF for x in out.cpu().tolist())
        assert got == want and history & H.STATUS_ERRORS == 0, f"call {call}: {got:#x} / {history:#x} vs {want:#x}"
        static.advance_powers([f.table for f in feats])
        for t in range(len(specs)):
            assert torch.equal(static.state[t], reference.state[t]), f"call {call} table {t}: states differ"
        # The bounds domain: the same maxima of |w|, |m|, v (which of its 64
        # slots holds a row's maxima follows the hot-row lists, filled by atomics).
        assert torch.equal(static.bounds.view(64, 4).max(0).values, reference.bounds.view(64, 4).max(0).values)
        assert np.array_equal(static.powers, reference.powers)
    # Above the maximum: refused, nothing enqueued.
    lengths = np.full(262145, 1, np.int64)
    big = W.Feature(0, 0, W.SUM, np.zeros(262145, np.uint64), np.arange(262146, dtype=np.uint64),
                    lengths.astype(np.uint64), None, np.zeros((262145, 64), np.float32))
    arr = (H.PushFeature * 1)(H.DeviceFeature(torch, big).push_struct(0))
    before = static.state[0].clone()
    rc = L.eps_hip_push_static(static.tables, static._opts, len(specs), arr, 1, static.bounds.data_ptr(),
                               None, stream)
    assert rc == H.CAPACITY, rc
    assert b"262144" in L.eps_hip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(static.state[0], before)
