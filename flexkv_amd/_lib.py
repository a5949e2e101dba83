"""Loader for libflexkv_hip.so, the HIP C-ABI library (include/flexkv_hip.h).

The library is built in-tree by ``__graft_entry__.build()`` (hipcc,
--offload-arch=gfx950).  There is no fallback: if the library is missing, every
transfer raises.  torch is imported first so that torch's HIP runtime is the
one the library binds to (both use the soname libamdhip64.so.7; one process
must not hold two HIP runtimes, and ``load()`` verifies it does not).
"""
from __future__ import annotations

import atexit
import ctypes
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime before ours)

LIB_NAME = "libflexkv_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

FKV_XFER_KERNEL = 0
FKV_XFER_CE = 1
FKV_XFER_CE_PER_CHUNK = 2

FKV_HOST_DEFAULT = 0
FKV_HOST_COHERENT = 1
FKV_HOST_NONCOHERENT = 2

# Names declared in include/flexkv_hip.h; tests check the library exports all.
EXPORTED_SYMBOLS = (
    "fkv_transfer_kv_blocks",
    "fkv_transfer_kv_blocks_kv_ptrs",
    "fkv_transfer_kv_blocks_noalloc",
    "fkv_gather_kv_blocks",
    "fkv_scatter_kv_blocks",
    "fkv_transfer_kv_blocks_layerwise",
    "fkv_handle_num_groups",
    "fkv_handle_query",
    "fkv_handle_wait",
    "fkv_handle_stream_wait",
    "fkv_handle_release",
    "fkv_stream_create",
    "fkv_stream_destroy",
    "fkv_ssd_open",
    "fkv_ssd_iouring_depth",
    "fkv_ssd_stats_read",
    "fkv_ssd_close",
    "fkv_transfer_kv_blocks_ssd",
    "fkv_last_error",
    "fkv_host_alloc",
    "fkv_host_free",
    "fkv_host_register",
    "fkv_host_unregister",
    "fkv_set_staging_bytes",
    "fkv_release_staging",
    "fkv_prepare",
    "fkv_finalize",
    "fkv_profile_enable",
    "fkv_profile_read",
    "fkv_version",
)


class FkvProfile(ctypes.Structure):
    _fields_ = [
        ("kernel_launches", ctypes.c_int64),
        ("kernel_ms", ctypes.c_double),
        ("kernel_bytes", ctypes.c_int64),
        ("dma_batches", ctypes.c_int64),
        ("dma_copies", ctypes.c_int64),
        ("dma_ms", ctypes.c_double),
        ("dma_bytes", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class SsdStats(ctypes.Structure):
    """fkv_ssd_stats: cumulative I/O counters of an SSD handle."""
    _fields_ = [
        ("direct_read_bytes", ctypes.c_int64),
        ("buffered_read_bytes", ctypes.c_int64),
        ("write_bytes", ctypes.c_int64),
        ("requests", ctypes.c_int64),
        ("ring_entries", ctypes.c_int64),
        ("fallbacks", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_lock = threading.Lock()
_lib = None
# Counts finalize() calls: handles and streams made before the latest one
# are gone, and their objects skip the library call when released.
generation = 0


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_i64, c_vp, c_sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    f = lib.fkv_transfer_kv_blocks
    f.restype = c_int
    f.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
                  c_i64, c_i64, c_i64, c_vp, c_int, c_int, c_int, c_int]
    f = lib.fkv_transfer_kv_blocks_noalloc
    f.restype = c_int
    f.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
                  c_i64, c_i64, c_i64, c_vp, c_int, c_int, c_int]
    f = lib.fkv_transfer_kv_blocks_kv_ptrs
    f.restype = c_int
    f.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64,
                  c_i64, c_i64, c_vp, c_int, c_int, c_int, c_int]
    for name in ("fkv_gather_kv_blocks", "fkv_scatter_kv_blocks"):
        g = getattr(lib, name)
        g.restype = c_int
        g.argtypes = [c_int, c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_sz, c_vp, c_int]
    f = lib.fkv_transfer_kv_blocks_layerwise
    f.restype = c_int
    f.argtypes = [c_int, c_int, c_int, c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
                  c_i64, c_i64, c_i64, c_vp, c_int, c_int, c_int, c_int, ctypes.POINTER(c_vp)]
    for name, extra in (("fkv_handle_num_groups", []), ("fkv_handle_query", [c_int]),
                        ("fkv_handle_wait", [c_int]), ("fkv_handle_stream_wait", [c_int, c_vp]),
                        ("fkv_handle_release", [])):
        fn = getattr(lib, name)
        fn.restype = c_int
        fn.argtypes = [c_vp] + extra
    lib.fkv_stream_create.restype = c_int
    lib.fkv_stream_create.argtypes = [c_int, ctypes.POINTER(c_vp)]
    lib.fkv_stream_destroy.restype = c_int
    lib.fkv_stream_destroy.argtypes = [c_vp]
    lib.fkv_ssd_open.restype = c_int
    lib.fkv_ssd_open.argtypes = [ctypes.POINTER(ctypes.c_char_p), c_int, c_int, c_int, c_int,
                                 ctypes.POINTER(c_vp)]
    lib.fkv_ssd_iouring_depth.restype = c_int
    lib.fkv_ssd_iouring_depth.argtypes = [c_vp]
    lib.fkv_ssd_stats_read.restype = c_int
    lib.fkv_ssd_stats_read.argtypes = [c_vp, ctypes.POINTER(SsdStats)]
    lib.fkv_ssd_close.restype = c_int
    lib.fkv_ssd_close.argtypes = [c_vp]
    f = lib.fkv_transfer_kv_blocks_ssd
    f.restype = c_int
    f.argtypes = [c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_i64,
                  c_i64, c_i64, c_int, c_int, c_int, c_int]
    lib.fkv_last_error.restype = ctypes.c_char_p
    lib.fkv_last_error.argtypes = []
    lib.fkv_host_alloc.restype = c_int
    lib.fkv_host_alloc.argtypes = [ctypes.POINTER(c_vp), c_sz, ctypes.c_uint]
    lib.fkv_host_free.restype = c_int
    lib.fkv_host_free.argtypes = [c_vp]
    lib.fkv_host_register.restype = c_int
    lib.fkv_host_register.argtypes = [c_vp, c_sz, ctypes.c_uint]
    lib.fkv_host_unregister.restype = c_int
    lib.fkv_host_unregister.argtypes = [c_vp]
    lib.fkv_set_staging_bytes.restype = c_int
    lib.fkv_set_staging_bytes.argtypes = [c_sz]
    lib.fkv_release_staging.restype = c_int
    lib.fkv_release_staging.argtypes = []
    lib.fkv_prepare.restype = c_int
    lib.fkv_prepare.argtypes = [c_int]
    lib.fkv_finalize.restype = c_int
    lib.fkv_finalize.argtypes = []
    lib.fkv_profile_enable.restype = c_int
    lib.fkv_profile_enable.argtypes = [c_int]
    lib.fkv_profile_read.restype = c_int
    lib.fkv_profile_read.argtypes = [ctypes.POINTER(FkvProfile)]
    lib.fkv_version.restype = ctypes.c_char_p
    lib.fkv_version.argtypes = []


def hip_runtimes_loaded(name: str = "libamdhip64.so") -> list:
    """Distinct files of runtime `name` (HIP by default) mapped into this process."""
    paths = set()
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                parts = line.split()
                if len(parts) >= 6 and name in parts[-1]:
                    paths.add(os.path.realpath(parts[-1]))
    except OSError:
        pass
    return sorted(paths)


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
                    "g.build()'` from the repository root")
            lib = ctypes.CDLL(LIB_PATH)
            _declare(lib)
            # (A profiler may map a second HSA runtime for itself; the library
            # resolves its HSA calls from the one next to the HIP runtime.)
            runtimes = hip_runtimes_loaded()
            if len(runtimes) > 1:
                raise ImportError(f"two HIP runtimes are mapped into this process: {runtimes}")
            _lib = lib
            atexit.register(finalize)
    return _lib


_fast = None


def fast():
    """Load (once) and return the compiled module ``_fkv_py`` that carries the
    per-call path of c_ext.transfer_kv_blocks, bound to the functions of the
    library that load() returns; raise if it is not built."""
    global _fast
    if _fast is not None:
        return _fast
    lib = load()
    with _lock:
        if _fast is None:
            try:
                from . import _fkv_py
            except ImportError as e:
                raise ImportError(
                    f"flexkv_amd/_fkv_py is not built ({e}); run `python -c 'import "
                    "__graft_entry__ as g; g.build()'` from the repository root") from e

            def addr(fn) -> int:
                return ctypes.cast(fn, ctypes.c_void_p).value
            _fkv_py.bind(addr(lib.fkv_transfer_kv_blocks), addr(lib.fkv_transfer_kv_blocks_kv_ptrs),
                         addr(lib.fkv_last_error), FKV_XFER_KERNEL, FKV_XFER_CE)
            _fast = _fkv_py
    return _fast


def finalize() -> None:
    """Release every resource the library holds (fkv_finalize): unreleased
    layer-wise handles, streams from fkv_stream_create, copy-engine signals,
    events and staging, pinned id buffers.  Registered with atexit when the
    library loads, so these objects are destroyed while the interpreter is
    still running, before the HIP and HSA runtimes run their own exit-time
    finalizers; otherwise the runtimes would tear them down themselves, in an
    order no caller controls.  A no-op when the library was never loaded."""
    global generation
    if _lib is None:
        return
    generation += 1
    rc = _lib.fkv_finalize()
    if rc != 0:
        import sys
        print(f"flexkv: fkv_finalize failed (status {rc}): {last_error()}", file=sys.stderr)


def last_error() -> str:
    msg = load().fkv_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Raise RuntimeError(fkv_last_error()) for a non-zero status."""
    if rc != 0:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


def profile_enable(on: bool) -> None:
    check(load().fkv_profile_enable(1 if on else 0), "fkv_profile_enable")


def profile_read() -> dict:
    out = FkvProfile()
    check(load().fkv_profile_read(ctypes.byref(out)), "fkv_profile_read")
    return out.as_dict()


def set_staging_bytes(nbytes: int) -> None:
    check(load().fkv_set_staging_bytes(int(nbytes)), "fkv_set_staging_bytes")


def release_staging() -> None:
    check(load().fkv_release_staging(), "fkv_release_staging")


def prepare(device: int = -1) -> None:
    """fkv_prepare: set a device up for transfers before the first one."""
    check(load().fkv_prepare(int(device)), "fkv_prepare")
