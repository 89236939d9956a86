"""Seeded synthetic workloads of the five embedding-shard shapes.

Inputs are generated on the host with numpy's PCG64 streams (platform
independent for a given seed) and describe one shard holding every row of each
table (keys == slots), so the same arrays drive the HIP path and the CPU
oracle.  Normal draws N(0, s) use s as the standard deviation.

Shapes (tables x rows x dim, batch):
  movielens : 2 tables (943 and 1682 rows) x 32, 128 single-hot (user, item)
              pairs per step, state initialised N(0, 0.01), 100 steps.
  criteo26  : 26 x 1,000,000 x 64, 4096 bags per table, bag length U{1..20},
              ids Zipf(1.05); tables 0-12 sum pooling, 13-25 mean pooling;
              initializer U(-0.05, 0.05).
  dup10m    : 1 x 10,000,000 x 128, 65,536 (row, gradient) pairs per step,
              ids Zipf(1.2), steps t = 1..50.
  large4    : 4 x 12,500,000 x 128, 262,144 bags x 32 per table, Zipf(1.1), mean.
  ragged8   : 8 tables, dims {16,32,64,96,128,192,256,256}, rows
              {100k,1M,5M,5M,2M,1M,500k,200k}, 8192 bags, lengths Poisson(8)
              clipped to 1..64, per-id weights U(0,1) (weighted sum), Zipf(1.05).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

SUM, MEAN, SEQUENCE, WEIGHTED_SUM = 0, 1, 2, 3


@dataclasses.dataclass
class TableSpec:
    id: int
    dim: int
    rows: int
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    b1p: float = 0.9   # initial beta powers (the powers of the first update)
    b2p: float = 0.999
    bounds: tuple | None = None
    init_min: float = -0.05
    init_max: float = 0.05
    seed: int = 42


@dataclasses.dataclass
class Feature:
    """One lookup feature (FeatureInput) on one table, with its gradient."""
    table: int            # index into the workload's table list
    feature: int
    pooling: int
    keys: np.ndarray      # uint64 row keys (== slots on a dense single shard)
    offsets: np.ndarray   # uint64, bags + 1
    valid_lengths: np.ndarray  # uint64, bags
    weights: np.ndarray | None = None   # float32 per key (weighted sum)
    gradient: np.ndarray | None = None  # float32 (rows, dim)

    @property
    def rows(self) -> int:
        return len(self.keys) if self.pooling == SEQUENCE else len(self.valid_lengths)


class Zipf:
    """Bounded Zipf(alpha) over n ranks by inverse CDF; rank r -> row
    (a * r + b) mod n with gcd(a, n) = 1, so hot rows are spread out."""

    def __init__(self, n: int, alpha: float, seed: int):
        ranks = np.arange(1, n + 1, dtype=np.float64)
        w = ranks ** (-alpha)
        self.cdf = np.cumsum(w)
        self.cdf /= self.cdf[-1]
        self.n = n
        rng = np.random.default_rng(seed)
        while True:
            a = int(rng.integers(n // 3 + 1, max(n, 2) * 2)) | 1
            if math.gcd(a, n) == 1:
                break
        self.a, self.b = a, int(rng.integers(0, n))

    def sample(self, rng: np.random.Generator, count: int) -> np.ndarray:
        u = rng.random(count)
        rank = np.searchsorted(self.cdf, u, side="right")
        rank = np.minimum(rank, self.n - 1).astype(np.uint64)
        return ((np.uint64(self.a) * rank + np.uint64(self.b)) % np.uint64(self.n)).astype(np.uint64)

    def expected_unique(self, draws: int) -> float:
        p = np.diff(np.concatenate([[0.0], self.cdf]))
        return float(np.sum(-np.expm1(draws * np.log1p(-p))))


def _bags(lengths: np.ndarray):
    offsets = np.zeros(len(lengths) + 1, np.uint64)
    np.cumsum(lengths, out=offsets[1:])
    return offsets, lengths.astype(np.uint64)


class Workload:
    name: str
    tables: list

    def batch(self, step: int) -> list:
        raise NotImplementedError

    @property
    def total_rows(self) -> int:
        return sum(t.rows for t in self.tables)


class MovieLens(Workload):
    name = "movielens"

    def __init__(self, seed: int = 1):
        self.tables = [TableSpec(0, 32, 943), TableSpec(1, 32, 1682)]
        self.seed = seed
        self.batch_size = 128

    def initial_state(self):
        """Explicit N(0, 0.01) weights, zero moments, per table (rows, 3*dim)."""
        rng = np.random.default_rng(3000 + self.seed)
        out = []
        for t in self.tables:
            s = np.zeros((t.rows, 3 * t.dim), np.float32)
            s[:, : t.dim] = rng.normal(0.0, 0.01, (t.rows, t.dim)).astype(np.float32)
            out.append(s)
        return out

    def batch(self, step: int):
        rng = np.random.default_rng((1000 + self.seed) * 100003 + step)
        g = np.random.default_rng((2000 + self.seed) * 100003 + step)
        feats = []
        for i, t in enumerate(self.tables):
            keys = rng.integers(0, t.rows, self.batch_size).astype(np.uint64)
            offsets, lengths = _bags(np.ones(self.batch_size, np.int64))
            grad = g.normal(0.0, 1e-2, (self.batch_size, t.dim)).astype(np.float32)
            feats.append(Feature(i, i, SUM, keys, offsets, lengths, None, grad))
        return feats


class Criteo26(Workload):
    name = "criteo26"

    def __init__(self, seed: int = 2, rows: int = 1_000_000, tables: int = 26, batch: int = 4096,
                 dim: int = 64, alpha: float = 1.05):
        self.tables = [TableSpec(i, dim, rows, seed=3000 + seed * 100 + i) for i in range(tables)]
        self.seed, self.batch_size, self.alpha = seed, batch, alpha
        self.zipf = [Zipf(rows, alpha, 1000 + seed * 100 + i) for i in range(tables)]

    def batch(self, step: int):
        feats = []
        for i, t in enumerate(self.tables):
            rng = np.random.default_rng(((4000 + self.seed) * 1009 + i) * 100003 + step)
            lengths = rng.integers(1, 21, self.batch_size)
            offsets, vlen = _bags(lengths)
            keys = self.zipf[i].sample(rng, int(offsets[-1]))
            g = np.random.default_rng(((2000 + self.seed) * 1009 + i) * 100003 + step)
            grad = g.normal(0.0, 1e-2, (self.batch_size, t.dim)).astype(np.float32)
            pooling = SUM if i < len(self.tables) // 2 else MEAN
            feats.append(Feature(i, i, pooling, keys, offsets, vlen, None, grad))
        return feats


class Dup10M(Workload):
    name = "dup10m"

    def __init__(self, seed: int = 3, rows: int = 10_000_000, pairs: int = 65536, dim: int = 128,
                 alpha: float = 1.2):
        self.tables = [TableSpec(0, dim, rows, seed=3000 + seed)]
        self.seed, self.pairs = seed, pairs
        self.zipf = Zipf(rows, alpha, 1000 + seed)

    def batch(self, step: int):
        rng = np.random.default_rng((1000 + self.seed) * 100003 + step)
        keys = self.zipf.sample(rng, self.pairs)
        offsets = np.array([0, self.pairs], np.uint64)
        g = np.random.default_rng((2000 + self.seed) * 100003 + step)
        grad = g.normal(0.0, 1e-2, (self.pairs, self.tables[0].dim)).astype(np.float32)
        return [Feature(0, 0, SEQUENCE, keys, offsets, np.array([self.pairs], np.uint64), None, grad)]


class Large4(Workload):
    name = "large4"

    def __init__(self, seed: int = 4, rows: int = 12_500_000, tables: int = 4, bags: int = 262144,
                 length: int = 32, dim: int = 128, alpha: float = 1.1):
        self.tables = [TableSpec(i, dim, rows, seed=3000 + seed * 100 + i) for i in range(tables)]
        self.seed, self.bags, self.length = seed, bags, length
        self.zipf = [Zipf(rows, alpha, 1000 + seed * 100 + i) for i in range(tables)]

    def batch(self, step: int):
        feats = []
        for i, t in enumerate(self.tables):
            rng = np.random.default_rng(((4000 + self.seed) * 1009 + i) * 100003 + step)
            offsets, vlen = _bags(np.full(self.bags, self.length, np.int64))
            keys = self.zipf[i].sample(rng, self.bags * self.length)
            g = np.random.default_rng(((2000 + self.seed) * 1009 + i) * 100003 + step)
            grad = g.normal(0.0, 1e-2, (self.bags, t.dim)).astype(np.float32)
            feats.append(Feature(i, i, MEAN, keys, offsets, vlen, None, grad))
        return feats


class Ragged8(Workload):
    name = "ragged8"
    DIMS = (16, 32, 64, 96, 128, 192, 256, 256)
    ROWS = (100_000, 1_000_000, 5_000_000, 5_000_000, 2_000_000, 1_000_000, 500_000, 200_000)

    def __init__(self, seed: int = 5, bags: int = 8192, alpha: float = 1.05, scale: int = 1):
        self.tables = [TableSpec(i, d, max(r // scale, 1000), seed=3000 + seed * 100 + i)
                       for i, (d, r) in enumerate(zip(self.DIMS, self.ROWS))]
        self.seed, self.bags = seed, bags
        self.zipf = [Zipf(t.rows, alpha, 1000 + seed * 100 + i) for i, t in enumerate(self.tables)]

    def batch(self, step: int):
        feats = []
        for i, t in enumerate(self.tables):
            rng = np.random.default_rng(((4000 + self.seed) * 1009 + i) * 100003 + step)
            lengths = np.clip(rng.poisson(8.0, self.bags), 1, 64)
            offsets, vlen = _bags(lengths)
            keys = self.zipf[i].sample(rng, int(offsets[-1]))
            w = np.random.default_rng(((5000 + self.seed) * 1009 + i) * 100003 + step)
            weights = w.random(len(keys)).astype(np.float32)
            g = np.random.default_rng(((2000 + self.seed) * 1009 + i) * 100003 + step)
            grad = g.normal(0.0, 1e-2, (self.bags, t.dim)).astype(np.float32)
            feats.append(Feature(i, i, WEIGHTED_SUM, keys, offsets, vlen, weights, grad))
        return feats

    # ---- cache-tier row moves ----
    MOVE_FRACTION = 0.05
    MOVE_LAG = 3  # a row written back after step k is admitted again at step k + MOVE_LAG

    def move_counts(self):
        """Rows admitted (and written back) per step and table: 5% of the
        expected touched rows."""
        return [max(1, int(round(self.MOVE_FRACTION * z.expected_unique(8 * self.bags))))
                for z in self.zipf]

    def admissions(self, touched):
        """Admission sets of a cycle of batches.  `touched[j][t]` = the unique
        keys batch j touches in table t (the batches repeat with period
        len(touched) >= MOVE_LAG).  Batch j admits A_j: a seeded sample of
        move_counts()[t] keys of batch j that neither of the previous
        MOVE_LAG - 1 batches touches.  The rows written back after batch j are
        A_{j + MOVE_LAG}: they are resident at batch j (no pending admission
        holds them), untouched while they sit in host memory, and admitted
        back, with the state they were written back with, before the batch
        that needs them."""
        period = len(touched)
        if period < self.MOVE_LAG:
            raise ValueError("tier moves need at least MOVE_LAG batches in the cycle")
        counts = self.move_counts()
        out = []
        for j in range(period):
            rng = np.random.default_rng((6000 + self.seed) * 100003 + j)
            per_table = []
            for t, count in enumerate(counts):
                recent = [touched[(j - d) % period][t] for d in range(1, self.MOVE_LAG)]
                free = np.setdiff1d(touched[j][t], np.concatenate(recent), assume_unique=False)
                if len(free) < count:
                    raise ValueError(f"batch {j} table {t}: only {len(free)} admissible rows")
                per_table.append(np.sort(rng.choice(free, count, replace=False)).astype(np.uint64))
            out.append(per_table)
        return out


def algorithmic_bytes(tables, feats, unique_rows):
    """Compulsory HBM bytes of one pull + push step (per table: unique weight rows,
    ids, offsets, pooled output; per-bag gradients, ids, offsets, w/m/v once)."""
    pull = push = 0
    for f, u in zip(feats, unique_rows):
        d = tables[f.table].dim
        n, b = len(f.keys), len(f.valid_lengths)
        extra = 4 * n if f.weights is not None else 0
        pull += u * d * 4 + n * 8 + (b + 1) * 8 + f.rows * d * 4 + extra
        push += f.rows * d * 4 + n * 8 + (b + 1) * 8 + extra + u * d * 24
    return pull, push
