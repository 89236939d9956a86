"""The pipelined training step that bench.py times (and a GPU test checks).

One step over a batch of features = the pooled pull of every feature on the
main stream, then the push (gradient scan, fused aggregation + sparse Adam,
checked apply) on the main stream.  The push's preparation (device dedup sort
and hot-row lists) reads only the batch's ids, so it runs on a side stream,
one batch ahead: step k issues batch k+1's preparation before its own pull
and push, rotating over the shard's W push workspaces (W >= 3):

  * batch j's preparation waits for the push of batch j-W, the last reader of
    its workspace (issued two or more steps earlier);
  * batch k's push waits for its preparation (issued a step earlier).

Issued a step ahead, a preparation is on the side stream as soon as the one
before it ends, so it has a whole step's time to finish before its push
needs it, however late the host issues the step.

Pushes are issued without reading their status (that would stall the
pipeline): optimizer powers are advanced when a push is issued and every
failure lands in the workspaces' status history, which `check()` reads once.
A run with any failure there is void (the powers of a rejected push would
have advanced).  This is the order of the reference's shard service for one
Lookup followed by one Push per step (src/server/service.cpp:137-331).
"""
from __future__ import annotations

import os

import numpy as np

from . import eps_hip as H

WORKSPACES = 3  # push workspaces the timed pipeline rotates over
AHEAD = 1       # batches prepared ahead of the batch being pushed


class StepPipeline:
    def __init__(self, torch, shard, batches, outputs, pull=True, moves=None):
        """`shard` is an eps_hip.DeviceShard with two or more workspaces; `batches` a
        list of lists of DeviceFeature (cycled); `outputs` one pooled-output
        tensor per feature position.  `pull` False: the step is the push alone
        (duplicate-heavy gradient pairs).  `moves`: a TierMoves whose
        admissions run before the pull and whose write-backs run after the push."""
        if len(shard.wss) < AHEAD + 2:
            raise ValueError(f"the pipeline rotates over {AHEAD + 2} or more push workspaces")
        self.slots = len(shard.wss)
        self.torch, self.shard, self.batches, self.outputs = torch, shard, batches, outputs
        self.pull, self.moves = pull, moves
        self.stream = torch.cuda.current_stream()
        self.side = torch.cuda.Stream()
        self.prepared = [torch.cuda.Event() for _ in range(self.slots)]
        self.pushed = [torch.cuda.Event() for _ in range(self.slots)]
        for slot in range(self.slots):
            shard.clear_history(slot)
        self.next_step = 0
        self.next_prep = 0  # batches [0, next_prep) have their preparation issued
        # The pushes' hot-row kernel runs on the library's side stream only
        # while every busy stream (this one, the preparation stream, that side
        # stream and a tier-move pair's two) can have a hardware queue of its
        # own: HIP maps streams onto GPU_MAX_HW_QUEUES queues round robin, and
        # a hot-row kernel queued behind a host-link copy waits for it
        # (ragged mixed-dim step with tier moves on 4 queues: side stream
        # 0.47 ms, in-stream 0.44 ms).  More queues do not help that step:
        # with GPU_MAX_HW_QUEUES=8 (every stream on a queue of its own, the
        # hot rows beside) it ran 0.66-0.67 ms against 0.44-0.50 on 4.
        queues = int(os.environ.get("GPU_MAX_HW_QUEUES", "4"))
        self.hot_overlap = 3 + (2 if moves else 0) <= queues

    def _prepare(self, j, phases=None):
        """Issues batch j's preparation on the side stream, in workspace j mod W."""
        slot = j % self.slots
        self.side.wait_event(self.pushed[slot])
        if phases:
            phases[5].record(self.side)
        self.shard.prepare(self.batches[j % len(self.batches)], stream=self.side, slot=slot)
        self.prepared[slot].record(self.side)
        if phases:
            phases[6].record(self.side)

    def step(self, k, fused=None, phases=None):
        """Issues step k (batch k mod len(batches)); steps are issued in order
        from 0.  `fused` = two timing events around the fused update;
        `phases` = seven events for a per-phase breakdown (see bench.py; the
        preparation timed is batch k+1's, the one this step issues)."""
        if k != self.next_step:
            raise ValueError(f"steps are issued in order: expected step {self.next_step}, got {k}")
        self.next_step += 1
        feats = self.batches[k % len(self.batches)]
        slot = k % self.slots
        stream = self.stream
        shard = self.shard
        if phases:
            phases[0].record(stream)
        while self.next_prep <= k + AHEAD:
            self._prepare(self.next_prep, phases if self.next_prep == k + AHEAD else None)
            self.next_prep += 1
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
                   events=fused or (tuple(phases[3:5]) if phases else None), hot_overlap=self.hot_overlap)
        shard.advance_powers([f.table for f in feats])
        self.pushed[slot].record(stream)
        if self.moves:
            self.moves.write_back(k)

    def check(self):
        """Waits for the device; raises if any push of the run failed."""
        bits = [self.shard.history(slot) for slot in range(self.slots)]
        if any(b & H.STATUS_ERRORS for b in bits):
            raise RuntimeError("a pipelined push failed: status history " +
                               " / ".join(f"{b:#x}" for b in bits))


class TierMoves:
    """Cache-tier row moves of a step (the device side of the reference's Move:
    Load, src/cuda/cache_backend.cu:390-462, and ReadBack + CommitEviction,
    :540-599; src/server/service.cpp:390-463).

    Batch j (of a cycle) admits the rows `admissions[j]` (per table, see
    workloads.Ragged8.admissions): their packed [w | m | v] come from pinned
    host memory and land in their slots before the pull.  After the push, the
    rows that batch j + lag admits are written back to pinned host memory.
    One batched kernel per direction moves every table's rows straight between
    the slots and the pinned buffers (it reads or writes host memory over the
    host link itself: on this system a runtime copy of a pinned buffer costs
    ~0.5 ms of host time a call).  Each direction has its own stream, so the
    link carries both at once, and both overlap the steps:

      * step k + 1's admission runs during step k (its rows are not touched by
        step k: admissions avoid the rows of the previous lag - 1 batches);
      * step k's write-back runs during step k + 1 (its rows are not touched
        before their admission, lag steps later).

    Re-admitted rows carry values this shard wrote back earlier, unchanged,
    which the bounds domain already covers (it never decreases), so the
    admissions leave it alone (a push's guard decision may be reading it
    meanwhile).  Row state between a write-back and its admission lives only
    in host memory: `poison` (tests) overwrites the written-back slots so an
    admission that did not happen cannot go unseen.
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
        # Host copy of the rows batch j admits (written back lag steps before).
        self.host = [torch.empty(total, dtype=f32, pin_memory=True) for _ in range(lag + 1)]
        self.inbound, self.outbound = torch.cuda.Stream(), torch.cuda.Stream()
        self.stream = torch.cuda.current_stream()
        self._tables = [t for t, c in enumerate(self.counts) if c]
        self._args = {}  # (cycle batch, host buffer) -> batched move arguments
        ring = 8  # events are reused round robin (a wait uses the latest record)
        self._ev = {n: [torch.cuda.Event() for _ in range(ring)] for n in ("admitted", "pushed", "written")}
        self._ring = ring
        self._poison_args = None
        if poison:
            self._poison_rows = torch.full((total,), 7.0, dtype=f32, device=dev)
            self._poison_args = {j: shard.row_batches([(t, self.slots[j][t], self._parts(self._poison_rows)[t])
                                                       for t in self._tables]) for j in range(self.period)}

    def _e(self, name, k):
        return self._ev[name][k % self._ring]

    def _parts(self, buf):
        return [buf[int(self.offset[t]):int(self.offset[t + 1])] for t in range(len(self.counts))]

    def _batches(self, j):
        """Moves of the rows batch j admits, to or from host buffer j % (lag + 1)."""
        key = (j % self.period, j % (self.lag + 1))
        if key not in self._args:
            host = self._parts(self.host[key[1]])
            self._args[key] = self.shard.row_batches([(t, self.slots[key[0]][t], host[t]) for t in self._tables])
        return self._args[key]

    def _poison_slots(self, j, stream):
        if self._poison_args is not None:
            self.shard.move_rows(self._poison_args[j % self.period], False, stream=stream, bounds=False)

    def _admit(self, k):
        """Step k's admission, on the inbound stream: its host copy was written
        back at step k - lag."""
        if k >= self.lag:
            self.inbound.wait_event(self._e("written", k - self.lag))
        self.shard.move_rows(self._batches(k), False, stream=self.inbound, bounds=False)
        self._e("admitted", k).record(self.inbound)

    def prime(self):
        """Before step 0: the rows batches 0 .. lag-1 admit start in host memory
        (their current device state is written back), then step 0's admission
        is issued."""
        for j in range(self.lag):
            self.shard.move_rows(self._batches(j), True, stream=self.stream)
            self._poison_slots(j, self.stream)
        self.torch.cuda.synchronize()
        self._admit(0)

    def admit(self, k):
        """Step k, before its pull: wait for step k's admission."""
        self.stream.wait_event(self._e("admitted", k))

    def write_back(self, k):
        """Step k, after its push: issue step k + 1's admission, then (after the
        push) the write-back of the rows batch k + lag admits, into the host
        buffer step k - 1's admission read."""
        self._e("pushed", k).record(self.stream)
        self._admit(k + 1)
        self.outbound.wait_event(self._e("pushed", k))
        if k >= 1:
            self.outbound.wait_event(self._e("admitted", k - 1))
        self.shard.move_rows(self._batches(k + self.lag), True, stream=self.outbound)
        self._poison_slots(k + self.lag, self.outbound)
        self._e("written", k).record(self.outbound)
