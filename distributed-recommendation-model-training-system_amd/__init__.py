"""MI355X-native parameter-shard embedding path.

Pooled row gather (pull), duplicate-id aggregation of pushed gradients and the
fused sparse (Lazy)Adam update of each row's w/m/v, as hand-written gfx950 HIP
kernels behind a C ABI (include/eps_hip.h, libeps_hip.so) and a C++ backend
(host/, libeps_hip_backend.so) that restates the reference's CacheBackend /
GpuCacheAgent interface.  This Python package is a thin ctypes binding used by
tests and the benchmark.
"""
from . import eps_hip, pipeline, workloads  # noqa: F401
