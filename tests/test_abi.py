"""The C-ABI library loads and exports every symbol include/eps_hip.h declares.

No compute calls: this runs without a GPU.
"""
import ctypes
import pathlib
import re
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared(header):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eps_hip_\w+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared("eps_hip.h")
    for required in ("eps_hip_gather", "eps_hip_prepare", "eps_hip_push", "eps_hip_unique",
                     "eps_hip_reduce", "eps_hip_adam_rows", "eps_hip_adam_compact",
                     "eps_hip_scatter_rows", "eps_hip_gather_rows", "eps_hip_init_rows"):
        assert required in names


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(str(pkg.eps_hip.LIB_PATH))
    missing = [n for n in declared("eps_hip.h") if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_the_header(pkg):
    assert set(declared("eps_hip.h")) == set(pkg.eps_hip.SYMBOLS)


def test_backend_library_loads(pkg):
    """libeps_hip_backend.so (eps::HipCacheBackend) resolves against
    libeps_hip.so and the HIP runtime; its C++ entry points are exported."""
    path = pkg.eps_hip.HERE / "libeps_hip_backend.so"
    ctypes.CDLL(str(path))
    names = subprocess.run(["nm", "-DC", "--defined-only", str(path)], capture_output=True,
                           text=True, check=True).stdout
    for method in ("Define", "FreeSlots", "Load", "GatherHost", "GatherDevice", "ApplyHost",
                   "ApplyCompact", "ReadBack", "CommitEviction", "MemoryStats", "AssembleFeatures",
                   "PushDevice"):
        assert f"eps::HipCacheBackend::{method}(" in names, method


def test_host_only_queries(pkg):
    L = pkg.eps_hip.lib()
    assert L.eps_hip_abi_version() == 1
    assert L.eps_hip_bounds_bytes() == 64 * 16
    assert L.eps_hip_update_workspace_bytes() == 1024  # the control block
    small, big = L.eps_hip_push_workspace_bytes(1000), L.eps_hip_push_workspace_bytes(10**6)
    assert 1024 < small < big
    # Validation errors are reported without touching a device.
    rc = L.eps_hip_prepare(None, 0, None, 0, None, 0, None)
    assert rc == pkg.eps_hip.INVALID_ARGUMENT
    assert b"tables" in L.eps_hip_last_error()


def test_measurement_library_is_separate(pkg):
    """The row read-modify-write ceiling kernel lives in libeps_hip_measure.so,
    which only bench.py's ceiling run loads; the kernel library exports
    nothing that is not in include/eps_hip.h."""
    kernels = subprocess.run(["nm", "-D", "--defined-only", str(pkg.eps_hip.LIB_PATH)], capture_output=True,
                             text=True, check=True).stdout
    exported = set(re.findall(r"\bT (eps_\w+)", kernels))
    assert exported == set(declared("eps_hip.h")), sorted(exported ^ set(declared("eps_hip.h")))
    measure = ctypes.CDLL(str(pkg.eps_hip.HERE / "libeps_hip_measure.so"))
    measure.eps_measure_last_error.restype = ctypes.c_char_p
    fn = measure.eps_measure_row_rmw
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                   ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    assert fn(None, 64, None, 0, None, 0, 1, 1, None) == 0  # nothing to do
    assert fn(None, 64, None, 8, None, 8, 1, 1, None) == pkg.eps_hip.INVALID_ARGUMENT
    assert b"null" in measure.eps_measure_last_error()
