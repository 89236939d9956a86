"""The pipelined training step that bench.py times (and a GPU test checks).

One step over a batch of features = the pooled pull of every feature on the
main stream, then the push (gradient scan, fused aggregation + sparse Adam,
checked apply) on the main stream.  The push's preparation (device dedup sort
and hot-row lists) reads only the batch's ids, so it runs on a side stream
ahead of the pull, alternating between two workspaces:

  * batch k's preparation waits for the push of batch k-2, the last reader of
    its workspace;
  * batch k's push waits for its preparation.

Pushes are issued without reading their status (that would stall the
pipeline): optimizer powers are advanced when a push is issued and every
failure lands in the workspaces' status history, which `check()` reads once.
A run with any failure there is void (the powers of a rejected push would
have advanced).  This is the order of the reference's shard service for one
Lookup followed by one Push per step (src/server/service.cpp:137-331).
"""
from __future__ import annotations

import numpy as np

from . import eps_hip as H


class StepPipeline:
    def __init__(self, torch, shard, batches, outputs, pull=True, moves=None):
        """`shard` is an eps_hip.DeviceShard with two workspaces; `batches` a
        list of lists of DeviceFeature (cycled); `outputs` one pooled-output
        tensor per feature position.  `pull` False: the step is the push alone
        (duplicate-heavy gradient pairs).  `moves`: a TierMoves whose
        admissions run before the pull and whose write-backs run after the push."""
        if len(shard.wss) < 2:
            raise ValueError("the pipeline alternates two push workspaces")
        self.torch, self.shard, self.batches, self.outputs = torch, shard, batches, outputs
        self.pull, self.moves = pull, moves
        self.stream = torch.cuda.current_stream()
        self.side = torch.cuda.Stream()
        self.prepared = [torch.cuda.Event() for _ in range(2)]
        self.pushed = [torch.cuda.Event() for _ in range(2)]
        for slot in range(2):
            shard.clear_history(slot)

    def step(self, k, fused=None, phases=None):
        """Issues step k (batch k mod len(batches)).  `fused` = two timing
        events around the fused update; `phases` = seven events for a
        per-phase breakdown (see bench.py)."""
        feats = self.batches[k % len(self.batches)]
        slot = k % 2
        stream, side, shard = self.stream, self.side, self.shard
        side.wait_event(self.pushed[slot])
        if phases:
            phases[0].record(stream)
            phases[5].record(side)
        shard.prepare(feats, stream=side, slot=slot)
        self.prepared[slot].record(side)
        if phases:
            phases[6].record(side)
        if self.moves:
            self.moves.admit(k)
        if self.pull:
            shard.lookup(feats, self.outputs, stream=stream)
        if phases:
            phases[1].record(stream)
        stream.wait_event(self.prepared[slot])
        if phases:
            phases[2].record(stream)
        shard.push(feats, stream=stream, slot=slot, advance=False,
                   events=fused or (tuple(phases[3:5]) if phases else None))
        shard.advance_powers([f.table for f in feats])
        self.pushed[slot].record(stream)
        if self.moves:
            self.moves.write_back(k)

    def check(self):
        """Waits for the device; raises if any push of the run failed."""
        bits = [self.shard.history(slot) for slot in range(2)]
        if any(b & H.STATUS_ERRORS for b in bits):
            raise RuntimeError(f"a pipelined push failed: status history {bits[0]:#x} / {bits[1]:#x}")


class TierMoves:
    """Cache-tier row moves of a step (the device side of the reference's Move:
    Load, src/cuda/cache_backend.cu:390-462, and ReadBack + CommitEviction,
    :540-599; src/server/service.cpp:390-463).

    Batch j (of a cycle) admits the rows `admissions[j]` (per table, see
    workloads.Ragged8.admissions): their packed [w | m | v] come from pinned
    host memory and are scattered into their slots before the pull.  After the
    push, the rows that batch j + lag admits are gathered out of their slots
    and written back to pinned host memory.  The host link carries both
    directions on two copy streams, overlapped with the steps:

      * the write-back of step k is copied device -> host after step k;
      * the admission of step k + 1 is copied host -> device (into one of two
        device staging buffers) while step k runs; it is the write-back of step
        k + 1 - lag, so it never waits for the step in flight.

    Row state between a write-back and its admission lives only in host
    memory: `poison` (tests) overwrites the written-back slots so an admission
    that did not happen cannot go unseen.
    """

    def __init__(self, torch, shard, admissions, lag, poison=False):
        self.torch, self.shard, self.lag, self.poison = torch, shard, lag, poison
        self.period = len(admissions)
        dims = [s.dim for s in shard.specs]
        self.counts = [len(a) for a in admissions[0]]
        if any([len(a) for a in adm] != self.counts for adm in admissions):
            raise ValueError("every batch admits the same count per table")
        # Packed layout of one step's moved rows: table t at offset[t] floats.
        widths = [c * 3 * d for c, d in zip(self.counts, dims)]
        self.offset = np.concatenate([[0], np.cumsum(widths)]).astype(np.int64)
        total = int(self.offset[-1])
        self.bytes = total * 4  # each way, per step
        dev, f32 = "cuda", torch.float32
        self.slots = [[torch.from_numpy(np.ascontiguousarray(a).view(np.int64)).to(dev) for a in adm]
                      for adm in admissions]
        self.adm_staging = [torch.empty(total, dtype=f32, device=dev) for _ in range(2)]
        self.wb_staging = [torch.empty(total, dtype=f32, device=dev) for _ in range(2)]
        # Host copy of the rows batch j admits, for j in flight (written back lag steps before).
        self.host = [torch.empty(total, dtype=f32, pin_memory=True) for _ in range(lag + 1)]
        self.h2d, self.d2h = torch.cuda.Stream(), torch.cuda.Stream()
        ev = torch.cuda.Event
        self.staged = {}      # step -> admission copied to the device
        self.scattered = {}   # step -> admission scattered (staging free again)
        self.copied_out = {}  # step -> write-back in host memory
        self.stream = torch.cuda.current_stream()
        self._ev = ev
        self._poison_rows = None
        if poison:
            self._poison_rows = torch.full((total,), 7.0, dtype=f32, device=dev)

    def _parts(self, buf):
        return [buf[int(self.offset[t]):int(self.offset[t + 1])] for t in range(len(self.counts))]

    def prime(self):
        """Before step 0: the rows batches 0 .. lag-1 admit start in host memory
        (their current device state is written back), then the admission of
        step 0 is staged."""
        for j in range(self.lag):
            buf = self.wb_staging[0]
            for t, part in enumerate(self._parts(buf)):
                if self.counts[t]:
                    self.shard.read_rows(t, self.slots[j % self.period][t], out=part, stream=self.stream)
            self._poison_slots(j % self.period)
            self.torch.cuda.synchronize()
            self.host[j % (self.lag + 1)].copy_(buf)
        self._stage(0)

    def _poison_slots(self, j):
        if self._poison_rows is None:
            return
        for t, part in enumerate(self._parts(self._poison_rows)):
            if self.counts[t]:
                self.shard.load_rows(t, self.slots[j][t], part, stream=self.stream)

    def _stage(self, k):
        """Host -> device copy of step k's admission (copy stream)."""
        with self.torch.cuda.stream(self.h2d):
            if k - 2 in self.scattered:
                self.h2d.wait_event(self.scattered.pop(k - 2))  # staging k % 2 is free
            if k - self.lag in self.copied_out:  # the host copy of this admission is written
                self.h2d.wait_event(self.copied_out[k - self.lag])
            self.adm_staging[k % 2].copy_(self.host[k % (self.lag + 1)], non_blocking=True)
            e = self._ev()
            e.record(self.h2d)
            self.staged[k] = e

    def admit(self, k):
        """Step k, before its pull: scatter the staged rows into their slots,
        then start staging step k + 1's admission."""
        self.stream.wait_event(self.staged.pop(k))
        for t, part in enumerate(self._parts(self.adm_staging[k % 2])):
            if self.counts[t]:
                self.shard.load_rows(t, self.slots[k % self.period][t], part, stream=self.stream)
        e = self._ev()
        e.record(self.stream)
        self.scattered[k] = e
        self._stage(k + 1)

    def write_back(self, k):
        """Step k, after its push: gather the rows batch k + lag admits into
        staging, then copy them to host memory (copy stream)."""
        j = (k + self.lag) % self.period
        if k - 2 in self.copied_out:  # write-back staging k % 2 is free once copied out
            self.stream.wait_event(self.copied_out[k - 2])
        buf = self.wb_staging[k % 2]
        for t, part in enumerate(self._parts(buf)):
            if self.counts[t]:
                self.shard.read_rows(t, self.slots[j][t], out=part, stream=self.stream)
        self._poison_slots(j)
        e = self._ev()
        e.record(self.stream)
        with self.torch.cuda.stream(self.d2h):
            self.d2h.wait_event(e)
            self.host[(k + self.lag) % (self.lag + 1)].copy_(buf, non_blocking=True)
            done = self._ev()
            done.record(self.d2h)
            self.copied_out[k] = done
        self.copied_out.pop(k - self.lag - 2, None)  # no later step waits for it
