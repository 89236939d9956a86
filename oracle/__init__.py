"""Oracle: CPU restatement of the reference parameter-shard path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker (or the
timed CPU baseline).  The product path (the HIP library and the C++ backend)
never calls it.

`libeps_oracle.so` (eps_oracle.c) restates the reference algorithms in C with
the reference's floating-point operation order; see eps_oracle.h for the
per-function citations and how each is pinned.  `_ref/libeps_ref.so`, when it
was built (oracle/Makefile `ref` target, from the reference checkout), exposes
the reference's own CPU sources and is used to pin the restatement.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libeps_oracle.so"
REF_PATH = HERE / "_ref" / "libeps_ref.so"

SUM, MEAN, SEQUENCE, WEIGHTED_SUM = 0, 1, 2, 3
U64_MAX = np.uint64(0xFFFFFFFFFFFFFFFF)


class TableDef(C.Structure):
    _fields_ = [("id", C.c_uint32), ("dim", C.c_uint32), ("shard", C.c_uint32),
                ("shard_count", C.c_uint32), ("learning_rate", C.c_float),
                ("beta1", C.c_float), ("beta2", C.c_float), ("epsilon", C.c_float),
                ("initial_beta1_power", C.c_float), ("initial_beta2_power", C.c_float),
                ("bounded", C.c_int32), ("weight_min", C.c_float), ("weight_max", C.c_float),
                ("init_min", C.c_float), ("init_max", C.c_float), ("init_seed", C.c_uint64)]


class FeatureStruct(C.Structure):
    _fields_ = [("keys", C.c_void_p), ("key_count", C.c_uint64), ("offsets", C.c_void_p),
                ("valid_lengths", C.c_void_p), ("weights", C.c_void_p),
                ("bag_count", C.c_uint64), ("pooling", C.c_uint32), ("feature", C.c_uint32)]


def table_def(id=1, dim=2, shard=0, shard_count=1, lr=0.1, beta1=0.9, beta2=0.999, eps=1e-8,
              b1p=0.9, b2p=0.999, bounds=None, init_min=0.25, init_max=0.25, seed=42) -> TableDef:
    lo, hi = bounds if bounds is not None else (0.0, 0.0)
    return TableDef(id, dim, shard, shard_count, lr, beta1, beta2, eps, b1p, b2p,
                    1 if bounds is not None else 0, lo, hi, init_min, init_max, seed)


def _ptr(a):
    return None if a is None else a.ctypes.data


def _u64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class _Feature:
    """Keeps numpy arrays alive while a C struct points at them."""

    def __init__(self, f):
        self.keys = _u64(f.keys)
        self.offsets = _u64(f.offsets)
        self.valid_lengths = _u64(f.valid_lengths)
        self.weights = None if getattr(f, "weights", None) is None else _f32(f.weights)
        self.pooling = int(f.pooling)
        self.feature = int(getattr(f, "feature", 0))
        self.struct = FeatureStruct(_ptr(self.keys), len(self.keys), _ptr(self.offsets),
                                    _ptr(self.valid_lengths), _ptr(self.weights),
                                    len(self.valid_lengths), self.pooling, self.feature)

    @property
    def rows(self):
        return len(self.keys) if self.pooling == SEQUENCE else len(self.valid_lengths)


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        P, U64, U32, I32, F = C.c_void_p, C.c_uint64, C.c_uint32, C.c_int32, C.c_float
        sig = {
            "eps_or_last_error": (C.c_char_p, []),
            "eps_or_mix": (U64, [U64]),
            "eps_or_init_weight": (F, [P, U64, U32]),
            "eps_or_create": (P, [P]),
            "eps_or_destroy": (None, [P]),
            "eps_or_ensure": (C.c_int64, [P, U64]),
            "eps_or_find": (C.c_int64, [P, U64]),
            "eps_or_row_count": (U64, [P]),
            "eps_or_key_at": (U64, [P, U64]),
            "eps_or_read": (C.c_int, [P, U64, P, P, P, P]),
            "eps_or_import": (C.c_int, [P, U64, P, P, P, U64]),
            "eps_or_overwrite": (C.c_int, [P, U64, P, P, P, U64]),
            "eps_or_powers": (None, [P, P, P, P]),
            "eps_or_read_many": (C.c_int, [P, P, U64, P, P, P]),
            "eps_or_prepare_feature": (C.c_int, [P, P, P, P, P, P]),
            "eps_or_mean_divide": (None, [P, P, U64, U32]),
            "eps_or_reduce_gradients": (C.c_int, [P, P, P, U32, P, P, P]),
            "eps_or_lr_t": (F, [F, F, F]),
            "eps_or_validate_lazy_adam": (C.c_int, [P, P, P, U64]),
            "eps_or_apply_lazy_adam": (None, [P, P, P, U64]),
            "eps_or_push": (C.c_int, [P, U32, P, P, P, U32]),
            "eps_or_adam_rows_ctx": (C.c_int, [P, P, P, P, U64, U32, F, F, F, F, F, F, I32, F, F]),
            "eps_or_gather_host": (C.c_int, [P, U32, P, U64, P, P]),
            "eps_or_compact_bytes": (U64, [U64, U64, U64]),
            "eps_or_validate_compact": (C.c_int, [U64, P, U32, P, U64, P, P, P, U64]),
            "eps_or_expand_compact": (C.c_int, [U64, P, U32, P, U64, P, P, P, U64, P]),
            "eps_or_build_compact": (C.c_int, [P, P, U32, U32, P, U64, P, P, P, P, P, P]),
            "eps_or_fnv1a": (U64, [U64, P, U64]),
            "eps_or_snapshot_write": (C.c_int, [C.c_char_p, C.c_char_p, U64, U64, U64, P, U32]),
            "eps_or_snapshot_read": (C.c_int, [C.c_char_p, P, U64, P, P, P, P, P, U32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().eps_or_last_error().decode()


def mix(x: int) -> int:
    return int(lib().eps_or_mix(x))


def init_weight(defn: TableDef, key: int, d: int) -> float:
    return float(lib().eps_or_init_weight(C.byref(defn), key, d))


def lr_t(lr: float, b1p: float, b2p: float) -> np.float32:
    return np.float32(lib().eps_or_lr_t(lr, b1p, b2p))


class Store:
    """One table of a CPU shard (ShardStore restated)."""

    def __init__(self, defn: TableDef):
        self.defn = defn
        self.dim = defn.dim
        self.h = lib().eps_or_create(C.byref(defn))
        if not self.h:
            raise ValueError(last_error())

    def __del__(self):
        if getattr(self, "h", None):
            lib().eps_or_destroy(self.h)
            self.h = None

    def ensure(self, key: int) -> int:
        slot = lib().eps_or_ensure(self.h, key)
        if slot < 0:
            raise ValueError(last_error())
        return slot

    def find(self, key: int) -> int:
        return lib().eps_or_find(self.h, key)

    @property
    def rows(self) -> int:
        return int(lib().eps_or_row_count(self.h))

    def key_at(self, slot: int) -> int:
        return int(lib().eps_or_key_at(self.h, slot))

    def read(self, key: int):
        w, m, v = (np.empty(self.dim, np.float32) for _ in range(3))
        u = C.c_uint64()
        rc = lib().eps_or_read(self.h, key, _ptr(w), _ptr(m), _ptr(v), C.byref(u))
        if rc:
            raise KeyError(last_error())
        return w, m, v, u.value

    def read_many(self, keys):
        """(rows x 3 x dim state, updates) for keys."""
        keys = _u64(keys)
        out = np.empty((len(keys), 3, self.dim), np.float32)
        updates = np.empty(len(keys), np.uint64)
        rc = lib().eps_or_read_many(self.h, _ptr(keys), len(keys), _ptr(out), _ptr(updates), None)
        if rc:
            raise KeyError(last_error())
        return out, updates

    def keys(self) -> np.ndarray:
        """Row keys in slot (first-touch) order."""
        n = self.rows
        keys = np.empty(max(n, 1), np.uint64)
        lib().eps_or_read_many(self.h, None, n, None, None, _ptr(keys))
        return keys[:n]

    def import_row(self, key, w, m, v, updates=0):
        w, m, v = _f32(w), _f32(m), _f32(v)
        rc = lib().eps_or_import(self.h, key, _ptr(w), _ptr(m), _ptr(v), updates)
        if rc:
            raise ValueError(last_error())

    def overwrite(self, key, w, m, v, updates):
        w, m, v = _f32(w), _f32(m), _f32(v)
        rc = lib().eps_or_overwrite(self.h, key, _ptr(w), _ptr(m), _ptr(v), updates)
        if rc:
            raise ValueError(last_error())

    def powers(self):
        b1, b2, seq = C.c_float(), C.c_float(), C.c_uint64()
        lib().eps_or_powers(self.h, C.byref(b1), C.byref(b2), C.byref(seq))
        return np.float32(b1.value), np.float32(b2.value), seq.value

    def prepare(self, feature):
        """PrepareFeature: (unique_slots, occurrence_to_unique, contribution)."""
        f = _Feature(feature)
        n = len(f.keys)
        unique = np.empty(max(n, 1), np.uint64)
        occ = np.empty(max(n, 1), np.uint64)
        count = C.c_uint64()
        out = np.empty((f.rows, self.dim), np.float32)
        rc = lib().eps_or_prepare_feature(self.h, C.byref(f.struct), _ptr(unique), C.byref(count),
                                          _ptr(occ), _ptr(out))
        if rc:
            raise ValueError(last_error())
        return unique[:count.value].copy(), occ[:n].copy(), out

    def reduce_gradients(self, features, gradients):
        """ReduceGradients for this table: (row_keys, row_values) or raises ValueError."""
        fs = [_Feature(f) for f in features]
        arr = (FeatureStruct * len(fs))(*[f.struct for f in fs])
        grads = [_f32(g) for g in gradients]
        gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
        total = sum(len(f.keys) for f in fs)
        keys = np.empty(max(total, 1), np.uint64)
        values = np.empty((max(total, 1), self.dim), np.float32)
        count = C.c_uint64()
        rc = lib().eps_or_reduce_gradients(self.h, arr, gp, len(fs), _ptr(keys), _ptr(values),
                                           C.byref(count))
        if rc:
            raise ValueError(last_error())
        return keys[:count.value].copy(), values[:count.value].copy()

    def lazy_adam(self, keys, values):
        """ValidateLazyAdam then ApplyLazyAdam; returns 0 or the error code."""
        keys, values = _u64(keys), _f32(values)
        rc = lib().eps_or_validate_lazy_adam(self.h, _ptr(keys), _ptr(values), len(keys))
        if rc:
            return rc
        lib().eps_or_apply_lazy_adam(self.h, _ptr(keys), _ptr(values), len(keys))
        return 0


def push(stores, features, feature_store, gradients) -> int:
    """One Push over CPU-owned rows of several tables (0 = applied)."""
    fs = [_Feature(f) for f in features]
    arr = (FeatureStruct * len(fs))(*[f.struct for f in fs])
    grads = [_f32(g) for g in gradients]
    gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
    sp = (C.c_void_p * len(stores))(*[s.h for s in stores])
    fmap = np.ascontiguousarray(np.asarray(feature_store, dtype=np.uint32))
    return lib().eps_or_push(sp, len(stores), arr, _ptr(fmap), gp, len(fs))


def mean_divide(values, valid_lengths):
    values = _f32(values).copy()
    lengths = _u64(valid_lengths)
    lib().eps_or_mean_divide(_ptr(values), _ptr(lengths), len(lengths), values.shape[1])
    return values


def adam_rows_ctx(w, m, v, g, beta1, beta2, eps, lr, b1p, b2p, bounds=None):
    """HostCacheBackend::ApplyHost arithmetic; returns (rc, w, m, v)."""
    w, m, v, g = (_f32(x).copy() for x in (w, m, v, g))
    rows, dim = g.shape
    lo, hi = bounds if bounds is not None else (0.0, 0.0)
    rc = lib().eps_or_adam_rows_ctx(_ptr(w), _ptr(m), _ptr(v), _ptr(g), rows, dim, beta1, beta2,
                                    eps, lr, b1p, b2p, 1 if bounds is not None else 0, lo, hi)
    return rc, w, m, v


def gather_host(feature, dim, occurrence_to_unique, unique_weights):
    f = _Feature(feature)
    occ = _u64(occurrence_to_unique)
    rows = [_f32(r) for r in unique_weights]
    rp = (C.c_void_p * max(len(rows), 1))(*[_ptr(r) for r in rows])
    out = np.empty((f.rows, dim), np.float32)
    rc = lib().eps_or_gather_host(C.byref(f.struct), dim, _ptr(occ), len(rows), rp, _ptr(out))
    if rc:
        raise ValueError(last_error())
    return out


def expand_compact(row_keys, dim, source_values, row_offsets, source_rows, scales):
    keys, sv, off = _u64(row_keys), _f32(source_values).reshape(-1), _u64(row_offsets)
    src, sc = _u64(source_rows), _f32(scales)
    out = np.empty((len(keys), dim), np.float32)
    rc = lib().eps_or_expand_compact(len(keys), _ptr(keys), dim, _ptr(sv), sv.size, _ptr(off),
                                     _ptr(src), _ptr(sc), len(src), _ptr(out))
    if rc:
        raise ValueError(last_error())
    return out


def compact_bytes(rows, source_values, references) -> int:
    return int(lib().eps_or_compact_bytes(rows, source_values, references))


def build_compact(features, gradients, dim, row_keys):
    fs = [_Feature(f) for f in features]
    arr = (FeatureStruct * len(fs))(*[f.struct for f in fs])
    grads = [_f32(g) for g in gradients]
    gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
    keys = _u64(row_keys)
    total = sum(len(f.keys) for f in fs)
    sv = np.empty((max(total, 1), dim), np.float32)
    off = np.empty(len(keys) + 1, np.uint64)
    src = np.empty(max(total, 1), np.uint64)
    sc = np.empty(max(total, 1), np.float32)
    nsv, nref = C.c_uint64(), C.c_uint64()
    rc = lib().eps_or_build_compact(arr, gp, len(fs), dim, _ptr(keys), len(keys), _ptr(sv),
                                    C.byref(nsv), _ptr(off), _ptr(src), _ptr(sc), C.byref(nref))
    if rc:
        raise ValueError(last_error())
    return sv[: nsv.value // dim].copy(), off, src[: nref.value].copy(), sc[: nref.value].copy()


# ---------------------------------------------------------------------------
# The reference's own CPU sources (only where oracle/_ref was built).
_ref = None


FNV_OFFSET = 14695981039346656037


def fnv1a(data: bytes, start: int = FNV_OFFSET) -> int:
    buf = np.frombuffer(bytes(data), dtype=np.uint8)
    return int(lib().eps_or_fnv1a(start, buf.ctypes.data if len(buf) else None, len(buf)))


def snapshot_write(path, run: str, shard: int, shard_count: int, epoch: int, stores) -> None:
    """WriteSnapshot (format 2) of the given stores, in the given order."""
    arr = (C.c_void_p * len(stores))(*[s.h for s in stores])
    rc = lib().eps_or_snapshot_write(str(path).encode(), run.encode(), shard, shard_count, epoch,
                                     arr, len(stores))
    if rc:
        raise OSError(last_error())


class _SnapshotStore(Store):
    def __init__(self, handle, defn):  # takes ownership of a store made by the reader
        self.defn = defn
        self.dim = defn.dim
        self.h = handle


def snapshot_read(path, capacity: int = 1024) -> dict:
    """ReadSnapshot (format 1 or 2): identity, version, checksum and the tables."""
    run = C.create_string_buffer(1025)
    shard, count, epoch, checksum = C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64()
    version, tables = C.c_uint32(), C.c_uint32()
    arr = (C.c_void_p * capacity)()
    rc = lib().eps_or_snapshot_read(str(path).encode(), run, 1025, C.byref(shard), C.byref(count),
                                    C.byref(epoch), C.byref(version), arr, capacity,
                                    C.byref(tables), C.byref(checksum))
    if rc:
        raise ValueError(last_error())
    stores = []
    for i in range(tables.value):
        d = TableDef.from_address(arr[i])  # eps_or_store starts with its definition
        stores.append(_SnapshotStore(arr[i], TableDef.from_buffer_copy(d)))
    return {"run": run.value.decode(), "shard": shard.value, "shard_count": count.value,
            "epoch": epoch.value, "version": version.value, "checksum": checksum.value,
            "tables": stores}


def ref_available() -> bool:
    return REF_PATH.exists()


def ref_lib():
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise FileNotFoundError("oracle/_ref was not built (needs the reference checkout)")
        L = C.CDLL(str(REF_PATH))
        P, U64, U32, F = C.c_void_p, C.c_uint64, C.c_uint32, C.c_float
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_shard_create": (P, [U32, U32]),
            "ref_shard_destroy": (None, [P]),
            "ref_shard_create_table": (C.c_int, [P, P]),
            "ref_shard_ensure": (C.c_int, [P, U32, U64, P]),
            "ref_shard_import": (C.c_int, [P, U32, U64, P, P, P, U64]),
            "ref_shard_read": (C.c_int, [P, U32, U64, P, P, P, P]),
            "ref_shard_powers": (None, [P, U32, P, P, P]),
            "ref_shard_prepare": (C.c_int, [P, U32, P, P, P, P, P]),
            "ref_shard_clear_prepared": (None, [P]),
            "ref_shard_reduce": (C.c_int, [P, U32, P, P, P, P]),
            "ref_shard_push": (C.c_int, [P, P]),
            "ref_expand_compact": (C.c_int, [U32, U64, P, U32, P, U64, P, P, P, U64, P]),
            "ref_shard_build_compact": (C.c_int, [P, U32, P, P, U64, P, P, P, P, P, P]),
            "ref_host_backend_create": (P, [U32, U64]),
            "ref_host_backend_destroy": (None, [P]),
            "ref_host_backend_define": (C.c_int, [P, P]),
            "ref_host_backend_load": (C.c_int, [P, U32, U32, P, U64, P, P, P]),
            "ref_host_backend_apply": (C.c_int, [P, U32, F, F, F, P, U64, P, U32]),
            "ref_host_backend_read": (C.c_int, [P, U32, U32, P, P, U64, P, P]),
            "ref_shard_write_snapshot": (C.c_int, [P, C.c_char_p, C.c_char_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _ref = L
    return _ref


class RefShard:
    """A shard of the compiled reference (ShardStore + PrepareFeature + Push)."""

    def __init__(self, defs, shard=0, shard_count=1):
        self.L = ref_lib()
        self.h = self.L.ref_shard_create(shard, shard_count)
        self.dims = {}
        self.prepared = []
        for d in defs:
            rc = self.L.ref_shard_create_table(self.h, C.byref(d))
            if rc:
                raise ValueError(self.error())
            self.dims[d.id] = d.dim

    def error(self):
        return self.L.ref_last_error().decode()

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_shard_destroy(self.h)
            self.h = None

    def import_row(self, table, key, w, m, v, updates=0):
        w, m, v = _f32(w), _f32(m), _f32(v)
        rc = self.L.ref_shard_import(self.h, table, key, _ptr(w), _ptr(m), _ptr(v), updates)
        if rc:
            raise ValueError(self.error())

    def read(self, table, key):
        dim = self.dims[table]
        w, m, v = (np.empty(dim, np.float32) for _ in range(3))
        u = C.c_uint64()
        rc = self.L.ref_shard_read(self.h, table, key, _ptr(w), _ptr(m), _ptr(v), C.byref(u))
        if rc:
            raise KeyError(self.error())
        return w, m, v, u.value

    def write_snapshot(self, path, run: str) -> None:
        rc = self.L.ref_shard_write_snapshot(self.h, str(path).encode(), run.encode())
        if rc:
            raise OSError(self.error())

    def powers(self, table):
        b1, b2, seq = C.c_float(), C.c_float(), C.c_uint64()
        self.L.ref_shard_powers(self.h, table, C.byref(b1), C.byref(b2), C.byref(seq))
        return np.float32(b1.value), np.float32(b2.value), seq.value

    def prepare(self, table, feature):
        f = _Feature(feature)
        n = len(f.keys)
        unique = np.empty(max(n, 1), np.uint64)
        occ = np.empty(max(n, 1), np.uint64)
        count = C.c_uint64()
        out = np.empty((f.rows, self.dims[table]), np.float32)
        rc = self.L.ref_shard_prepare(self.h, table, C.byref(f.struct), _ptr(unique),
                                      C.byref(count), _ptr(occ), _ptr(out))
        if rc:
            raise ValueError(self.error())
        self.prepared.append(f)
        return unique[:count.value].copy(), occ[:n].copy(), out

    def reduce(self, table, gradients):
        grads = [_f32(g) for g in gradients]
        gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
        total = sum(len(f.keys) for f in self.prepared)
        keys = np.empty(max(total, 1), np.uint64)
        values = np.empty((max(total, 1), self.dims[table]), np.float32)
        count = C.c_uint64()
        rc = self.L.ref_shard_reduce(self.h, table, gp, _ptr(keys), _ptr(values), C.byref(count))
        if rc:
            raise ValueError(self.error())
        return keys[:count.value].copy(), values[:count.value].copy()

    def build_compact(self, table, gradients, row_keys):
        grads = [_f32(g) for g in gradients]
        gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
        keys = _u64(row_keys)
        dim = self.dims[table]
        total = sum(len(f.keys) for f in self.prepared)
        sv = np.empty((max(total, 1), dim), np.float32)
        off = np.empty(len(keys) + 1, np.uint64)
        src = np.empty(max(total, 1), np.uint64)
        sc = np.empty(max(total, 1), np.float32)
        nsv, nref = C.c_uint64(), C.c_uint64()
        rc = self.L.ref_shard_build_compact(self.h, table, gp, _ptr(keys), len(keys), _ptr(sv),
                                            C.byref(nsv), _ptr(off), _ptr(src), _ptr(sc),
                                            C.byref(nref))
        if rc:
            raise ValueError(self.error())
        return sv[: nsv.value // dim].copy(), off, src[: nref.value].copy(), sc[: nref.value].copy()

    def push(self, gradients) -> int:
        grads = [_f32(g) for g in gradients]
        gp = (C.c_void_p * len(grads))(*[_ptr(g) for g in grads])
        rc = self.L.ref_shard_push(self.h, gp)
        self.prepared = []
        return rc

    def clear(self):
        self.L.ref_shard_clear_prepared(self.h)
        self.prepared = []


def ref_expand_compact(table, row_keys, dim, source_values, row_offsets, source_rows, scales):
    L = ref_lib()
    keys, sv, off = _u64(row_keys), _f32(source_values).reshape(-1), _u64(row_offsets)
    src, sc = _u64(source_rows), _f32(scales)
    out = np.empty((len(keys), dim), np.float32)
    rc = L.ref_expand_compact(table, len(keys), _ptr(keys), dim, _ptr(sv), sv.size, _ptr(off),
                              _ptr(src), _ptr(sc), len(src), _ptr(out))
    if rc:
        raise ValueError(L.ref_last_error().decode())
    return out


class RefHostBackend:
    """The reference HostCacheBackend (protocol reference backend)."""

    def __init__(self, agent=0, state_bytes=1 << 30):
        self.L = ref_lib()
        self.h = self.L.ref_host_backend_create(agent, state_bytes)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_host_backend_destroy(self.h)
            self.h = None

    def error(self):
        return self.L.ref_last_error().decode()

    def define(self, d):
        rc = self.L.ref_host_backend_define(self.h, C.byref(d))
        if rc:
            raise ValueError(self.error())

    def load(self, table, dim, keys, packed, updates):
        keys, packed, updates = _u64(keys), _f32(packed), _u64(updates)
        slots = np.empty(len(keys), np.uint64)
        rc = self.L.ref_host_backend_load(self.h, table, dim, _ptr(keys), len(keys), _ptr(packed),
                                          _ptr(updates), _ptr(slots))
        if rc:
            raise ValueError(self.error())
        return slots

    def apply(self, table, lr, b1p, b2p, keys, values, dim) -> int:
        keys, values = _u64(keys), _f32(values)
        return self.L.ref_host_backend_apply(self.h, table, lr, b1p, b2p, _ptr(keys), len(keys),
                                             _ptr(values), dim)

    def read(self, table, dim, keys, slots):
        keys, slots = _u64(keys), _u64(slots)
        packed = np.empty((len(keys), 3 * dim), np.float32)
        updates = np.empty(len(keys), np.uint64)
        rc = self.L.ref_host_backend_read(self.h, table, dim, _ptr(keys), _ptr(slots), len(keys),
                                          _ptr(packed), _ptr(updates))
        if rc:
            raise ValueError(self.error())
        return packed, updates
