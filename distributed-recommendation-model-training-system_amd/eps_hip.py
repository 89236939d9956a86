"""ctypes binding of libeps_hip.so (include/eps_hip.h) and a device-resident shard.

`DeviceShard` drives the C ABI the way the reference shard service drives its
backend (src/server/service.cpp Lookup/Push): lookup = pooled gather (+ the
device dedup of the lookup ticket), push = duplicate-id aggregation fused with
sparse Adam, with the per-table beta powers advanced once per applied push
(src/update/lazy_adam.cpp:39-41).  Device memory and streams come from torch
(plumbing only).  There is no CPU fallback: without the HIP library every call
raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# The in-tree build; EPS_HIP_LIBRARY names another build of the same ABI.
LIB_PATH = pathlib.Path(os.environ.get("EPS_HIP_LIBRARY", HERE / "libeps_hip.so"))

OK, INVALID_ARGUMENT, UNAVAILABLE, STALE_GENERATION, RETIRED, CAPACITY, RUN_FAILED = range(7)
SUM, MEAN, SEQUENCE, WEIGHTED_SUM = 0, 1, 2, 3
STATUS_BAD_INDEX = 0x1
STATUS_NONFINITE_GRAD = 0x2
STATUS_REDUCE_OVERFLOW = 0x4
STATUS_ADAM_OVERFLOW = 0x8
STATUS_REJECTED = 0x10
STATUS_STALLED = 0x20
STATUS_BAD_SCALE = 0x40
STATUS_CHECKED_PATH = 0x100
STATUS_ERRORS = 0xF | STATUS_REJECTED | STATUS_STALLED | STATUS_BAD_SCALE
MAX_FEATURES = 32
MAX_TABLES = 32
MAX_GATHER_PARTS = 32
HOLE = -1  # UINT64_MAX as int64


class Table(C.Structure):
    _fields_ = [("state", C.c_void_p), ("rows", C.c_uint64), ("dim", C.c_uint32), ("id", C.c_uint32)]


class Optimizer(C.Structure):
    _fields_ = [("learning_rate", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("beta1_power", C.c_float), ("beta2_power", C.c_float),
                ("bounded", C.c_int32), ("weight_min", C.c_float), ("weight_max", C.c_float)]


class GatherPart(C.Structure):
    _fields_ = [("source", C.c_void_p), ("indices", C.c_void_p), ("remap", C.c_void_p),
                ("offsets", C.c_void_p), ("valid_lengths", C.c_void_p), ("weights", C.c_void_p),
                ("output", C.c_void_p), ("stride", C.c_uint64), ("rows", C.c_uint64),
                ("source_rows", C.c_uint64), ("remap_count", C.c_uint64), ("dim", C.c_uint32),
                ("pooling", C.c_uint32)]


class RowBatch(C.Structure):
    _fields_ = [("state", C.c_void_p), ("slots", C.c_void_p), ("packed", C.c_void_p), ("count", C.c_uint64),
                ("dim", C.c_uint32), ("reserved", C.c_uint32)]


class PushFeature(C.Structure):
    _fields_ = [("indices", C.c_void_p), ("offsets", C.c_void_p), ("valid_lengths", C.c_void_p),
                ("weights", C.c_void_p), ("gradients", C.c_void_p), ("occurrences", C.c_uint64),
                ("bags", C.c_uint64), ("table", C.c_uint32), ("pooling", C.c_uint32)]


SYMBOLS = {
    "eps_hip_abi_version": (C.c_int, []),
    "eps_hip_last_error": (C.c_char_p, []),
    "eps_hip_device_check": (C.c_int, [C.c_int]),
    "eps_hip_bounds_bytes": (C.c_uint64, []),
    "eps_hip_bounds_reset": (C.c_int, [C.c_void_p, C.c_void_p]),
    "eps_hip_init_rows": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                    C.c_uint64, C.c_float, C.c_float, C.c_int32, C.c_float,
                                    C.c_float, C.c_void_p, C.c_void_p]),
    "eps_hip_scatter_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                       C.c_void_p]),
    "eps_hip_gather_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "eps_hip_move_rows": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int32, C.c_void_p, C.c_void_p]),
    "eps_hip_index_bytes": (C.c_uint64, [C.c_uint64]),
    "eps_hip_index_clear": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p]),
    "eps_hip_index_insert": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                       C.c_void_p]),
    "eps_hip_index_remove": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "eps_hip_resolve": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                  C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "eps_hip_gather": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]),
    "eps_hip_add_contribution": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                           C.c_uint32, C.c_void_p]),
    "eps_hip_normalize_mean": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32,
                                         C.c_void_p]),
    "eps_hip_push_workspace_bytes": (C.c_uint64, [C.c_uint64]),
    "eps_hip_prepare": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                  C.c_uint64, C.c_void_p]),
    "eps_hip_push": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                               C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "eps_hip_push_begin": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                     C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "eps_hip_push_apply": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                     C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "eps_hip_push_end": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                   C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "eps_hip_unique": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                 C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p]),
    "eps_hip_reduce": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                 C.c_uint64, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "eps_hip_push_static": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                      C.c_void_p, C.c_void_p]),
    "eps_hip_update_workspace_bytes": (C.c_uint64, []),
    "eps_hip_adam_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                    C.c_void_p, C.c_void_p, C.c_void_p]),
    "eps_hip_adam_compact": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64,
                                       C.c_void_p, C.c_void_p, C.c_void_p]),
    "eps_hip_status_word": (C.c_void_p, [C.c_void_p]),
    "eps_hip_status_history_word": (C.c_void_p, [C.c_void_p]),
    "eps_hip_debug_set_spin_limit": (C.c_int, [C.c_uint32]),
    "eps_hip_set_hot_row_overlap": (C.c_int, [C.c_int]),
    "eps_hip_read_status": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "eps_hip_fill_u32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint64, C.c_void_p]),
}

_lib = None


class HipError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"eps_hip error {code}: {message}")
        self.code = code


def lib():
    """The HIP library; raises if it was not built (there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int):
    if rc:
        raise HipError(rc, lib().eps_hip_last_error().decode())


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(torch, stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def lr_t(lr, b1p, b2p):
    """Bias-corrected step in float arithmetic (src/update/lazy_adam.cpp:27)."""
    f = np.float32
    return f(f(lr) * np.sqrt(f(1) - f(b2p), dtype=np.float32)) / (f(1) - f(b1p))


class DeviceFeature:
    """A feature's arrays resident on the device (int64 views of uint64 keys)."""

    def __init__(self, torch, feature, device="cuda", with_gradient=True):
        self.table = feature.table
        self.pooling = feature.pooling
        self.occurrences = len(feature.keys)
        self.bags = len(feature.valid_lengths)
        self.rows = feature.rows
        as_i64 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int64)).to(device)
        self.indices = as_i64(feature.keys)
        self.offsets = as_i64(feature.offsets)
        self.valid_lengths = as_i64(feature.valid_lengths)
        self.weights = None
        if feature.weights is not None:
            self.weights = torch.from_numpy(np.ascontiguousarray(feature.weights, np.float32)).to(device)
        self.gradient = None
        if with_gradient and feature.gradient is not None:
            self.gradient = torch.from_numpy(np.ascontiguousarray(feature.gradient, np.float32)).to(device)

    def __setattr__(self, name, value):
        # Any change of the feature's arrays or fields drops the cached struct.
        object.__setattr__(self, name, value)
        object.__setattr__(self, "_struct", None)

    def push_struct(self, table_index=None):
        if table_index is not None:
            return PushFeature(_ptr(self.indices), _ptr(self.offsets), _ptr(self.valid_lengths),
                               _ptr(self.weights), _ptr(self.gradient), self.occurrences, self.bags,
                               table_index, self.pooling)
        if self._struct is None:
            object.__setattr__(self, "_struct", self.push_struct(self.table))
        return self._struct


class DeviceShard:
    """Every row of each table resident in HBM as AoS [w|m|v] (slot == key)."""

    def __init__(self, torch, specs, max_occurrences=0, device="cuda", workspaces=1):
        self.torch = torch
        self.specs = list(specs)
        self.device = device
        L = lib()
        check(L.eps_hip_device_check(torch.device(device).index or 0))
        self.state = [torch.empty(s.rows * 3 * s.dim, dtype=torch.float32, device=device)
                      for s in self.specs]
        # Optimizer powers (beta1^t, beta2^t) per table, advanced in fp32.
        self.powers = np.array([[s.b1p, s.b2p] for s in self.specs], dtype=np.float32)
        self._betas = np.array([[s.beta1, s.beta2] for s in self.specs], dtype=np.float32)
        # One persistent optimizer array for the push calls; only its powers
        # change between pushes (written through a numpy view).
        self._opts = (Optimizer * len(self.specs))(*[self.optimizer(t) for t in range(len(self.specs))])
        self._opts_view = np.frombuffer(self._opts, dtype=np.dtype(
            [(name, np.float32 if ctype is C.c_float else np.int32) for name, ctype in Optimizer._fields_]))
        self._args_cache = {}
        self.bounds = torch.zeros(L.eps_hip_bounds_bytes() // 4, dtype=torch.int32, device=device)
        self.update_ws = torch.zeros(L.eps_hip_update_workspace_bytes() // 4, dtype=torch.int32,
                                     device=device)
        # Push workspaces: a caller that prepares the next batch while the
        # current one is pushed alternates between two of them (`slot`).
        self.wss = [None] * workspaces
        self.ws_bytes = 0
        self.reserve(max_occurrences)
        self.tables = (Table * len(self.specs))(*[
            Table(_ptr(st), s.rows, s.dim, s.id) for st, s in zip(self.state, self.specs)])

    # ---- workspace ----
    @property
    def ws(self):
        return self.wss[0]

    def reserve(self, occurrences):
        need = lib().eps_hip_push_workspace_bytes(int(occurrences))
        if need > self.ws_bytes:
            if any(w is not None for w in self.wss):
                # Work queued on any stream may still read the old workspaces:
                # drain the device before their memory can be handed out again.
                self.torch.cuda.synchronize()
            self.wss = [self.torch.zeros((need + 3) // 4, dtype=self.torch.int32, device=self.device)
                        for _ in self.wss]
            self.ws_bytes = need

    # ---- state ----
    def init_rows(self, stream=None):
        """Reference initializer for every slot (key == slot)."""
        L = lib()
        for i, s in enumerate(self.specs):
            lo, hi = s.bounds if s.bounds else (0.0, 0.0)
            check(L.eps_hip_init_rows(C.byref(self.tables[i]), 0, s.rows, 0, 1, s.seed, s.init_min,
                                      s.init_max, 1 if s.bounds else 0, lo, hi, _ptr(self.bounds),
                                      _stream(self.torch, stream)))

    def load_rows(self, table, slots, packed, stream=None):
        """Scatter packed [w|m|v] rows (device or pinned host tensor) into slots."""
        check(lib().eps_hip_scatter_rows(C.byref(self.tables[table]), _ptr(slots), _ptr(packed),
                                         slots.numel(), _ptr(self.bounds), _stream(self.torch, stream)))

    def read_rows(self, table, slots, out=None, stream=None):
        d = self.specs[table].dim
        if out is None:
            out = self.torch.empty((slots.numel(), 3 * d), dtype=self.torch.float32, device=self.device)
        check(lib().eps_hip_gather_rows(C.byref(self.tables[table]), _ptr(slots), _ptr(out),
                                        slots.numel(), _stream(self.torch, stream)))
        return out

    def row_batches(self, parts):
        """ctypes array of RowBatch for [(table, slots tensor, packed tensor), ...]."""
        return (RowBatch * len(parts))(*[RowBatch(_ptr(self.state[t]), _ptr(slots), _ptr(packed), slots.numel(),
                                                  self.specs[t].dim, 0) for t, slots, packed in parts])

    def move_rows(self, batches, write_back, stream=None, bounds=True):
        """Admit (write_back False) or write back the rows of a row_batches()
        array.  bounds=False: an admission of values the bounds domain already
        covers (rows this shard wrote back, unchanged) leaves it alone."""
        check(lib().eps_hip_move_rows(batches, len(batches), 1 if write_back else 0,
                                      _ptr(self.bounds) if bounds else None, _stream(self.torch, stream)))

    def optimizer(self, table):
        s = self.specs[table]
        b1p, b2p = self.powers[table]
        lo, hi = s.bounds if s.bounds else (0.0, 0.0)
        return Optimizer(s.lr, s.beta1, s.beta2, s.eps, float(b1p), float(b2p),
                         1 if s.bounds else 0, lo, hi)

    def advance_powers(self, tables):
        sel = list(set(tables))
        self.powers[sel] = self.powers[sel] * self._betas[sel]  # fp32 products, as the reference

    # ---- pull ----
    def gather_parts(self, feats, outputs, mean_divide=True):
        parts = []
        for f, out in zip(feats, outputs):
            s = self.specs[f.table]
            parts.append(GatherPart(
                _ptr(self.state[f.table]), _ptr(f.indices), None,
                _ptr(f.offsets) if f.pooling != SEQUENCE else None,
                _ptr(f.valid_lengths) if (f.pooling == MEAN and mean_divide) else None,
                _ptr(f.weights), _ptr(out), 3 * s.dim, f.rows, s.rows, 0, s.dim, f.pooling))
        return parts

    def lookup(self, feats, outputs=None, status=None, stream=None, mean_divide=True):
        """Pooled pull of device features into outputs (allocated if None)."""
        if outputs is None:
            outputs = [self.torch.empty((f.rows, self.specs[f.table].dim), dtype=self.torch.float32,
                                        device=self.device) for f in feats]
        def build():
            parts = self.gather_parts(feats, outputs, mean_divide)
            return [((GatherPart * len(parts[i:i + MAX_GATHER_PARTS]))(*parts[i:i + MAX_GATHER_PARTS]),
                     len(parts[i:i + MAX_GATHER_PARTS])) for i in range(0, len(parts), MAX_GATHER_PARTS)]
        chunks = self._cached("gather", list(feats) + list(outputs), build,
                              (mean_divide, tuple(o.data_ptr() for o in outputs)))
        for arr, count in chunks:
            check(lib().eps_hip_gather(arr, count, _ptr(status), _stream(self.torch, stream)))
        return outputs

    # ---- push ----
    def _cached(self, kind, objs, build, extra=()):
        """ctypes argument array for these objects, kept for the last few object
        lists seen (an entry holds its objects, so their ids stay unique while it
        lives) and rebuilt when a feature's struct or `extra` has changed."""
        key = (kind, tuple(map(id, objs)))
        hit = self._args_cache.get(key)
        if hit is not None and hit[1] == extra and all(
                getattr(a, "_struct", None) is c for a, c in zip(hit[0], hit[2])):
            return hit[3]
        arr = build()
        if len(self._args_cache) >= 16:
            self._args_cache.pop(next(iter(self._args_cache)))
        self._args_cache[key] = (list(objs), extra, [getattr(o, "_struct", None) for o in objs], arr)
        return arr

    def _push_args(self, feats):
        if len(feats) > MAX_FEATURES:
            raise ValueError("too many features for one push")
        return self._cached("push", feats, lambda: (PushFeature * len(feats))(*[f.push_struct() for f in feats]))

    def prepare(self, feats, stream=None, slot=0):
        self.reserve(sum(f.occurrences for f in feats))
        arr = self._push_args(feats)
        check(lib().eps_hip_prepare(self.tables, len(self.specs), arr, len(feats),
                                    _ptr(self.wss[slot]), self.ws_bytes, _stream(self.torch, stream)))

    def push(self, feats, stream=None, advance=True, events=None, slot=0, hot_overlap=True):
        """Fused aggregation + Adam of a prepared push.  With `advance` the call
        waits for the push, and advances the optimizer powers of the pushed
        tables only if it applied (a rejected update leaves them unchanged, as
        ApplyLazyAdam does, src/update/lazy_adam.cpp:39-41); it returns the
        status.  Callers that overlap pushes pass advance=False (asynchronous),
        advance the powers themselves and check history() afterwards.
        `events` = (start, end) torch events recorded around the fused pass;
        `slot` = the workspace the batch was prepared in; `hot_overlap` False
        runs the hot-row kernel on `stream` (eps_hip_set_hot_row_overlap)."""
        arr = self._push_args(feats)
        self._opts_view["beta1_power"] = self.powers[:, 0]
        self._opts_view["beta2_power"] = self.powers[:, 1]
        args = (self.tables, self._opts, len(self.specs), arr, len(feats), _ptr(self.wss[slot]), self.ws_bytes,
                _ptr(self.bounds), _stream(self.torch, stream))
        L = lib()
        check(L.eps_hip_push_begin(*args))
        if events:
            events[0].record(stream)
        if not hot_overlap:
            check(L.eps_hip_set_hot_row_overlap(0))
        try:
            check(L.eps_hip_push_apply(*args))
        finally:
            if not hot_overlap:
                check(L.eps_hip_set_hot_row_overlap(1))
        if events:
            events[1].record(stream)
        check(L.eps_hip_push_end(*args))
        if advance:
            status = self.status(stream, slot=slot)
            if status & STATUS_ERRORS == 0:
                self.advance_powers([f.table for f in feats])
            return status
        return None

    def status(self, stream=None, workspace=None, slot=0):
        out = C.c_uint32()
        ws = self.wss[slot] if workspace is None else workspace
        check(lib().eps_hip_read_status(_ptr(ws), C.byref(out), _stream(self.torch, stream)))
        return out.value

    def history(self, slot=0):
        """Failure bits of every push run in workspace `slot` (waits for the device)."""
        ws = self.wss[slot]
        index = (lib().eps_hip_status_history_word(_ptr(ws)) - ws.data_ptr()) // 4
        self.torch.cuda.synchronize()
        return int(ws[index].item()) & 0xFFFFFFFF

    def clear_history(self, slot=0, stream=None):
        check(lib().eps_hip_fill_u32(lib().eps_hip_status_history_word(_ptr(self.wss[slot])), 0, 1,
                                     _stream(self.torch, stream)))

    def unique(self, feats, stream=None):
        """(unique_slots, unique_tables, occurrence_to_unique, count) of a prepared push."""
        t = self.torch
        n = sum(f.occurrences for f in feats)
        slots = t.empty(max(n, 1), dtype=t.int64, device=self.device)
        tables = t.empty(max(n, 1), dtype=t.int32, device=self.device)
        occ = t.empty(max(n, 1), dtype=t.int64, device=self.device)
        count = t.zeros(1, dtype=t.int64, device=self.device)
        arr = self._push_args(feats)
        check(lib().eps_hip_unique(self.tables, len(self.specs), arr, len(feats), _ptr(self.ws),
                                   self.ws_bytes, _ptr(slots), _ptr(tables), _ptr(occ), _ptr(count),
                                   _stream(self.torch, stream)))
        return slots, tables, occ, count

    def reduce(self, feats, occ2u, rows, stream=None):
        t = self.torch
        stride = max(s.dim for s in self.specs)
        stride = (stride + 3) // 4 * 4
        values = t.zeros((max(rows, 1), stride), dtype=t.float32, device=self.device)
        arr = self._push_args(feats)
        check(lib().eps_hip_reduce(self.tables, len(self.specs), arr, len(feats), _ptr(self.ws),
                                   self.ws_bytes, _ptr(occ2u), _ptr(values), stride,
                                   _stream(self.torch, stream)))
        return values

    # ---- backend-style updates ----
    def adam_rows(self, table, slots, gradients, opt=None, stream=None):
        opt = opt or self.optimizer(table)
        check(lib().eps_hip_adam_rows(C.byref(self.tables[table]), C.byref(opt), _ptr(slots),
                                      _ptr(gradients), slots.numel(), _ptr(self.update_ws),
                                      _ptr(self.bounds), _stream(self.torch, stream)))
        return self.status(stream, self.update_ws)

    def adam_compact(self, table, slots, row_offsets, source_rows, scales, source_values, opt=None,
                     stream=None):
        opt = opt or self.optimizer(table)
        check(lib().eps_hip_adam_compact(C.byref(self.tables[table]), C.byref(opt), _ptr(slots),
                                         slots.numel(), _ptr(row_offsets), _ptr(source_rows),
                                         _ptr(scales), _ptr(source_values),
                                         source_values.shape[0], source_rows.numel(),
                                         _ptr(self.update_ws), _ptr(self.bounds),
                                         _stream(self.torch, stream)))
        return self.status(stream, self.update_ws)
