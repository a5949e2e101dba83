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
import operator
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
    "fkv_tp_group_create",
    "fkv_tp_group_transfer",
    "fkv_tp_group_destroy",
    "fkv_last_error",
    "fkv_last_unsafe_host_blocks",
    "fkv_abandoned_copies_pending",
    "fkv_host_alloc",
    "fkv_host_free",
    "fkv_host_register",
    "fkv_host_unregister",
    "fkv_set_staging_bytes",
    "fkv_release_staging",
    "fkv_prepare",
    "fkv_set_copy_engine_policy",
    "fkv_get_copy_engine_policy",
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
        ("dma_held_copies", ctypes.c_int64),
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
    lib.fkv_tp_group_create.restype = c_int
    lib.fkv_tp_group_create.argtypes = [c_int, ctypes.POINTER(c_int), c_vp, c_int, c_vp,
                                        ctypes.POINTER(c_vp)]
    f = lib.fkv_tp_group_transfer
    f.restype = c_int
    f.argtypes = [c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_int, c_int,
                  c_int, c_int, c_int, c_int]
    lib.fkv_tp_group_destroy.restype = c_int
    lib.fkv_tp_group_destroy.argtypes = [c_vp]
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
    lib.fkv_set_copy_engine_policy.restype = c_int
    lib.fkv_set_copy_engine_policy.argtypes = [c_i64, c_int]
    lib.fkv_get_copy_engine_policy.restype = c_int
    lib.fkv_get_copy_engine_policy.argtypes = [ctypes.POINTER(c_i64), ctypes.POINTER(c_int)]
    lib.fkv_last_unsafe_host_blocks.restype = c_int
    lib.fkv_last_unsafe_host_blocks.argtypes = [c_vp, c_int]
    lib.fkv_abandoned_copies_pending.restype = c_int
    lib.fkv_abandoned_copies_pending.argtypes = [c_int]


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
_INT_MAX = 2**31 - 1


class _CtypesCalls:
    """The per-call path of c_ext.transfer_kv_blocks and
    transfer_kv_blocks_kv_ptrs over ctypes, with the compiled module's
    argument conventions: the same 16 / 15 positional arguments, False
    (nothing raised) when a tensor check fails so that c_ext names the
    argument, RuntimeError with the library's message when the transfer
    fails.  Used when _fkv_py cannot be imported (not built, or built for
    another torch or Python); each call costs a few microseconds more."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib
        self._device_visible = None

    @staticmethod
    def _i64_host(t) -> bool:
        return (isinstance(t, torch.Tensor) and t.dtype == torch.int64 and t.is_cpu
                and t.is_contiguous())

    @staticmethod
    def _mode(v) -> int:
        if isinstance(v, bool) or type(v).__name__ in ("bool_", "bool"):
            return FKV_XFER_CE if bool(v) else FKV_XFER_KERNEL
        return operator.index(v)

    @staticmethod
    def _c_int(v, what: str) -> int:
        v = operator.index(v)
        if not -_INT_MAX - 1 <= v <= _INT_MAX:
            raise OverflowError(f"{what} {v} does not fit a C int")
        return v

    def _stream(self, stream):
        if stream is not None:
            return int(stream)
        if self._device_visible is None:
            self._device_visible = torch.cuda.is_available()
        if not self._device_visible:
            return None
        return torch.cuda.current_stream().cuda_stream

    def _finish(self, rc: int) -> None:
        if rc != 0:
            msg = last_error()
            raise RuntimeError(msg or f"transfer failed ({rc})")

    def transfer_kv_blocks(self, gids, ptrs, gkv, gblk, cids, cpu, ckv, clay, cblk, chunk,
                           start, sms, h2d, mode, mla, stream):
        if not (self._i64_host(gids) and self._i64_host(ptrs) and self._i64_host(cids)
                and isinstance(cpu, torch.Tensor)) or cids.numel() != gids.numel():
            return False
        for n, what in ((gids.numel(), "block ids"), (ptrs.numel(), "layer pointers")):
            if n > _INT_MAX:
                raise RuntimeError(f"{n} {what} in one call; at most {_INT_MAX}")
        ix = operator.index
        args = (ix(gkv), ix(gblk), ix(ckv), ix(clay), ix(cblk), ix(chunk),
                self._c_int(start, "start_layer_id"), self._c_int(sms, "transfer_sms"),
                1 if h2d else 0, self._mode(mode), 1 if mla else 0)
        st = self._stream(stream)
        if st is None:
            return False
        gkv, gblk, ckv, clay, cblk, chunk, start, sms, h2d, mode, mla = args
        self._finish(self._lib.fkv_transfer_kv_blocks(
            gids.numel(), start, ptrs.numel(), gids.data_ptr(), ptrs.data_ptr(), gkv, gblk,
            cids.data_ptr(), cpu.data_ptr(), ckv, clay, cblk, 0, chunk, st, sms, h2d, mode, mla))
        return None

    def transfer_kv_blocks_kv_ptrs(self, gids, ptrs, gblk, cids, cpu, ckv, clay, cblk, chunk,
                                   start, sms, h2d, mode, mla, stream):
        if not (self._i64_host(gids) and self._i64_host(ptrs) and self._i64_host(cids)
                and isinstance(cpu, torch.Tensor)):
            return False
        for n, what in ((gids.numel(), "block ids"), (ptrs.numel(), "layer pointers")):
            if n > _INT_MAX:
                raise RuntimeError(f"{n} {what} in one call; at most {_INT_MAX}")
        ix = operator.index
        args = (ix(gblk), ix(ckv), ix(clay), ix(cblk), ix(chunk),
                self._c_int(start, "start_layer_id"), self._c_int(sms, "transfer_sms"),
                1 if h2d else 0, self._mode(mode), 1 if mla else 0)
        kv = 1 if mla else 2
        if cids.numel() != gids.numel() or ptrs.numel() % kv:
            return False
        st = self._stream(stream)
        if st is None:
            return False
        gblk, ckv, clay, cblk, chunk, start, sms, h2d, mode, mla = args
        self._finish(self._lib.fkv_transfer_kv_blocks_kv_ptrs(
            gids.numel(), start, ptrs.numel() // kv, gids.data_ptr(), ptrs.data_ptr(), gblk,
            cids.data_ptr(), cpu.data_ptr(), ckv, clay, cblk, 0, chunk, st, sms, h2d, mode, mla))
        return None


def fast():
    """Load (once) and return the per-call path of c_ext.transfer_kv_blocks:
    the compiled module ``_fkv_py`` bound to the functions of the library
    that load() returns, or, when that module cannot be imported (not built,
    or built against another torch or Python) or FLEXKV_PY_FASTCALL=0, the
    ctypes calls of _CtypesCalls (logged once)."""
    global _fast
    if _fast is not None:
        return _fast
    lib = load()
    with _lock:
        if _fast is None:
            reason = None
            if os.environ.get("FLEXKV_PY_FASTCALL", "1") == "0":
                reason = "FLEXKV_PY_FASTCALL=0"
            else:
                try:
                    from . import _fkv_py
                except ImportError as e:
                    reason = f"flexkv_amd/_fkv_py cannot be imported ({e})"
            if reason is not None:
                import logging
                logging.getLogger("flexkv").warning(
                    "%s; transfer_kv_blocks calls the library through ctypes (rebuild with "
                    "`python -c 'import __graft_entry__ as g; g.build()'`)", reason)
                _fast = _CtypesCalls(lib)
                return _fast

            def addr(fn) -> int:
                return ctypes.cast(fn, ctypes.c_void_p).value
            _fkv_py.bind(addr(lib.fkv_transfer_kv_blocks), addr(lib.fkv_transfer_kv_blocks_kv_ptrs),
                         addr(lib.fkv_last_error), FKV_XFER_KERNEL, FKV_XFER_CE)
            _fast = _fkv_py
    return _fast


def reset_fast() -> None:
    """Forget the chosen per-call path, so the next fast() chooses again
    (tests switch between the compiled module and the ctypes calls)."""
    global _fast
    import sys
    with _lock:
        _fast = None
        c_ext = sys.modules.get(__package__ + ".c_ext")
        if c_ext is not None:
            c_ext._fast = None


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


def last_unsafe_host_blocks() -> list:
    """Host block ids that copy engines may still write after this thread's
    last failed transfer (fkv_last_unsafe_host_blocks); [] when none."""
    lib = load()
    n = lib.fkv_last_unsafe_host_blocks(None, 0)
    if n <= 0:
        return []
    buf = (ctypes.c_int64 * n)()
    n = min(n, lib.fkv_last_unsafe_host_blocks(buf, n))
    return list(buf[:n])


def abandoned_copies_pending(device: int = -1) -> int:
    """Copies given up on by timed-out copy-engine waits that have not
    finished yet (fkv_abandoned_copies_pending)."""
    n = load().fkv_abandoned_copies_pending(int(device))
    if n < 0:
        raise RuntimeError(last_error() or "fkv_abandoned_copies_pending failed")
    return n


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
