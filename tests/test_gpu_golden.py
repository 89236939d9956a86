"""The HIP path reproduces the golden vectors that the reference's own sources
wrote (tests/golden/), bit for bit: pooled partial sums per feature, unique rows
in first-occurrence order and their reduced gradients per table, the optimizer
powers and every touched row's w, m, v after the pushes."""
import numpy as np
import pytest

from test_golden import Feature, load, same

pytestmark = pytest.mark.gpu


def test_hip_path_reproduces_reference_trajectory(torch_gpu, pkg):
    torch, W, H = torch_gpu, pkg.workloads, pkg.eps_hip
    g = load("shard_trajectory")
    steps, features = (int(x) for x in g["steps"])
    specs = []
    for tid, dim, space, (lr, lo, hi, bounded, wmin, wmax, seed) in zip(
            g["table_ids"], g["table_dims"], g["table_space"], g["table_params"]):
        specs.append(W.TableSpec(int(tid), int(dim), int(space), lr=float(lr), init_min=float(lo),
                                 init_max=float(hi), seed=int(seed),
                                 bounds=(float(wmin), float(wmax)) if bounded else None))
    shard = H.DeviceShard(torch, specs, max_occurrences=4096)
    shard.init_rows()  # the reference initializer, key == slot
    for s in range(steps):
        print(f"case: golden step {s}", flush=True)
        feats = [Feature(g, s, f) for f in range(features)]
        dev = [H.DeviceFeature(torch, f) for f in feats]
        pooled = shard.lookup(dev, mean_divide=False)  # the shard returns partial sums
        for f, out in zip(feats, pooled):
            assert same(out.cpu().numpy(), g[f"s{s}_f{f.feature}_pooled"]), f"step {s} feature {f.feature}"
        shard.prepare(dev)
        slots, tables, occ, count = shard.unique(dev)
        u = int(count.item())
        values = shard.reduce(dev, occ, u).cpu().numpy()
        slots, tables = slots[:u].cpu().numpy().view(np.uint64), tables[:u].cpu().numpy()
        for t, spec in enumerate(specs):
            mine = tables == t
            assert same(slots[mine], g[f"s{s}_t{t}_reduce_keys"]), f"step {s} table {t}: unique rows"
            assert same(values[mine, :spec.dim], g[f"s{s}_t{t}_reduce_values"]), f"step {s} table {t}"
        shard.push(dev)
        status = shard.status()
        assert status & H.STATUS_ERRORS == 0, f"step {s}: status {status:#x}"
        for t, spec in enumerate(specs):
            assert same(np.array(shard.powers[t], np.float32), g[f"s{s}_t{t}_powers"])
            if f"s{s}_t{t}_touched" in g:
                touched = torch.from_numpy(g[f"s{s}_t{t}_touched"].view(np.int64)).cuda()
                state = shard.read_rows(t, touched).cpu().numpy()
                assert same(state, g[f"s{s}_t{t}_state"]), f"step {s} table {t}: row state"
