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


def test_static_push_replays_in_a_graph(torch_gpu, pkg):
    """A static push captured in a HIP graph: every kernel runs on the
    capturing stream (no side stream or event), so the capture holds the
    whole push.  Each of three replays, with eager work and synchronisations
    between them, must leave the tables bit-identical to the same push run
    eagerly with a caller workspace (the optimizer powers are the captured
    ones, so the eager pushes keep them too), and report a clean status."""
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    L = H.lib()
    specs = [W.TableSpec(0, 64, 20000, seed=71)]
    captured, eager, warm = (H.DeviceShard(torch, specs) for _ in range(3))
    for shard in (captured, eager, warm):
        shard.init_rows()
    rng = np.random.default_rng(72)
    feats = features(W, rng, specs, 3000)
    dev = [H.DeviceFeature(torch, f) for f in feats]
    arr = captured._push_args(dev)
    out = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    # One eager call first: it looks the static array's address up on this device.
    warm_stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    H.check(L.eps_hip_push_static(warm.tables, warm._opts, len(specs), warm._push_args(dev), len(dev),
                                  warm.bounds.data_ptr(), out.data_ptr(), warm_stream))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        H.check(L.eps_hip_push_static(captured.tables, captured._opts, len(specs), arr, len(dev),
                                      captured.bounds.data_ptr(), out.data_ptr(), C.c_void_p(side.cuda_stream)))
    scratch = torch.ones(1 << 20, device="cuda")
    for replay in range(3):
        print(f"case: graph replay {replay}", flush=True)
        out.fill_(-1)
        graph.replay()
        scratch.mul_(1.5).add_(1.0)  # eager work between replays
        torch.cuda.synchronize()
        eager.prepare(dev)
        eager.push(dev, advance=False)
        want = eager.status()
        assert want & H.STATUS_ERRORS == 0, f"{want:#x}"
        got, history = (int(x) & 0xFFFFFFFF for x in out.cpu().tolist())
        assert got == want and history & H.STATUS_ERRORS == 0, f"replay {replay}: {got:#x} / {history:#x}"
        assert torch.equal(captured.state[0], eager.state[0]), f"replay {replay}: states differ"
