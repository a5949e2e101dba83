"""Drop-in for the reference extension module ``flexkv.c_ext`` (transfer path).

``transfer_kv_blocks`` keeps the reference's 15 positional arguments
(csrc/bindings.cpp:25-32, bound without keywords at :108-109) and semantics:
it unpacks the tensors into raw pointers, runs on the *current* torch stream
(bindings.cpp:44), returns after that stream has drained (transfer.cu:131),
and raises RuntimeError on failure (bindings.cpp:51-54).  The work is done by
the HIP C-ABI entry ``fkv_transfer_kv_blocks``.
"""
from __future__ import annotations

import contextlib

import torch

from . import _lib

__all__ = ["transfer_kv_blocks", "transfer_kv_blocks_kv_ptrs", "gather_kv_blocks",
           "scatter_kv_blocks",
           "transfer_kv_blocks_layerwise", "LayerwiseTransfer", "transfer_stream",
           "release_transfer_stream", "set_copy_engine_policy", "copy_engine_policy",
           "TPTransferThreadGroup", "SSDIOCTX", "transfer_kv_blocks_ssd"]


_device_visible = None
_raw_stream = None      # torch's current-raw-stream query, once a device is seen
_current_device = None


def _stream_handle(fn_name: str) -> int:
    """Raw handle of the current torch stream of the current device.  Raises
    when no HIP device is visible (checked once per process)."""
    global _device_visible, _raw_stream, _current_device
    if _raw_stream is not None:
        return _raw_stream(_current_device())
    if _device_visible is None:
        _device_visible = torch.cuda.is_available()
    if not _device_visible:
        raise RuntimeError(f"{fn_name} needs a HIP device; none is visible")
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return torch.cuda.current_stream().cuda_stream
    _current_device = torch._C._cuda_getDevice
    _raw_stream = raw       # avoids building a Stream object per call
    return raw(_current_device())


_I64 = torch.int64


def _require_int64_host(t: torch.Tensor, name: str) -> None:
    # one combined test on the common path; the detailed checks only on failure
    if isinstance(t, torch.Tensor) and t.dtype is _I64 and t.is_cpu and t.is_contiguous():
        return
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != torch.int64:
        raise TypeError(f"{name} must be int64, got {t.dtype}")
    if t.device.type != "cpu":
        raise RuntimeError(f"{name} must be a host tensor (pinned), got device {t.device}")
    raise RuntimeError(f"{name} must be contiguous")


def transfer_kv_blocks(gpu_block_id_tensor: torch.Tensor,
                       gpu_layer_ptrs_tensor: torch.Tensor,
                       gpu_kv_stride_in_bytes: int,
                       gpu_block_stride_in_bytes: int,
                       cpu_block_id_tensor: torch.Tensor,
                       cpu_tensor: torch.Tensor,
                       cpu_kv_stride_in_bytes: int,
                       cpu_layer_stride_in_bytes: int,
                       cpu_block_stride_in_bytes: int,
                       chunk_size_in_bytes: int,
                       start_layer_id: int,
                       transfer_sms: int = -1,
                       is_host_to_device: bool = True,
                       use_ce_transfer=False,
                       is_mla: bool = False, *, stream: int = None) -> None:
    """Copy KV blocks between the per-layer GPU cache and the host cache.

    ``use_ce_transfer``: False -> zero-copy wavefront kernel; True -> copy
    engines behind an on-device gather/scatter through staging; the integer 2
    selects the reference's one-DMA-per-chunk loop (csrc/transfer.cu:97-121).
    ``transfer_sms`` bounds the compute units of the zero-copy kernel
    (-1 = automatic).  ``stream`` (keyword only, an extension) is a raw
    stream handle to run on instead of the current torch stream.

    The compiled module ``_fkv_py`` unpacks and checks the tensors, takes the
    current stream and calls ``fkv_transfer_kv_blocks`` with the GIL released;
    when a check fails, ``_explain`` raises the error that names it.
    """
    f = _fast or _load_fast()
    if f.transfer_kv_blocks(gpu_block_id_tensor, gpu_layer_ptrs_tensor, gpu_kv_stride_in_bytes,
                            gpu_block_stride_in_bytes, cpu_block_id_tensor, cpu_tensor,
                            cpu_kv_stride_in_bytes, cpu_layer_stride_in_bytes,
                            cpu_block_stride_in_bytes, chunk_size_in_bytes, start_layer_id,
                            transfer_sms, is_host_to_device, use_ce_transfer, is_mla,
                            stream) is False:
        _explain("transfer_kv_blocks", gpu_block_id_tensor, gpu_layer_ptrs_tensor,
                 "gpu_layer_ptrs_tensor", cpu_block_id_tensor, cpu_tensor, 1, stream)


def transfer_kv_blocks_kv_ptrs(gpu_block_id_tensor: torch.Tensor,
                               gpu_kv_ptrs_tensor: torch.Tensor,
                               gpu_block_stride_in_bytes: int,
                               cpu_block_id_tensor: torch.Tensor,
                               cpu_tensor: torch.Tensor,
                               cpu_kv_stride_in_bytes: int,
                               cpu_layer_stride_in_bytes: int,
                               cpu_block_stride_in_bytes: int,
                               chunk_size_in_bytes: int,
                               start_layer_id: int,
                               transfer_sms: int = -1,
                               is_host_to_device: bool = True,
                               use_ce_transfer=False,
                               is_mla: bool = False, *, stream: int = None) -> None:
    """transfer_kv_blocks for K and V held in separate allocations
    (extension): ``gpu_kv_ptrs_tensor`` is an int64 host tensor of
    ``layers * kv`` base pointers ordered [layer][K|V] (kv = 1 for MLA)."""
    f = _fast or _load_fast()
    if f.transfer_kv_blocks_kv_ptrs(gpu_block_id_tensor, gpu_kv_ptrs_tensor,
                                    gpu_block_stride_in_bytes, cpu_block_id_tensor, cpu_tensor,
                                    cpu_kv_stride_in_bytes, cpu_layer_stride_in_bytes,
                                    cpu_block_stride_in_bytes, chunk_size_in_bytes,
                                    start_layer_id, transfer_sms, is_host_to_device,
                                    use_ce_transfer, is_mla, stream) is False:
        _explain("transfer_kv_blocks_kv_ptrs", gpu_block_id_tensor, gpu_kv_ptrs_tensor,
                 "gpu_kv_ptrs_tensor", cpu_block_id_tensor, cpu_tensor, 1 if is_mla else 2,
                 stream)


_fast = None


def _load_fast():
    global _fast
    _fast = _lib.fast()
    return _fast


def _explain(fn_name: str, gpu_block_id_tensor, ptrs_tensor, ptrs_name: str,
             cpu_block_id_tensor, cpu_tensor, per_layer: int, stream) -> None:
    """Raise the error for arguments the compiled per-call path refused."""
    _require_int64_host(gpu_block_id_tensor, "gpu_block_id_tensor")
    _require_int64_host(ptrs_tensor, ptrs_name)
    _require_int64_host(cpu_block_id_tensor, "cpu_block_id_tensor")
    if not isinstance(cpu_tensor, torch.Tensor):
        raise TypeError(f"cpu_tensor must be a torch.Tensor, got {type(cpu_tensor).__name__}")
    num_blocks = gpu_block_id_tensor.numel()          # bindings.cpp:33
    if cpu_block_id_tensor.numel() != num_blocks:
        raise RuntimeError(
            f"gpu_block_id_tensor has {num_blocks} ids but cpu_block_id_tensor has "
            f"{cpu_block_id_tensor.numel()}")
    if ptrs_tensor.numel() % per_layer:
        raise RuntimeError(f"{ptrs_name} holds {ptrs_tensor.numel()} pointers, "
                           f"not a multiple of {per_layer}")
    if stream is None:
        _stream_handle(fn_name)
    raise RuntimeError(f"{fn_name}: arguments refused")


def _contiguous(fn_name: str, gpu_block_id_tensor, gpu_layer_ptrs_tensor, gpu_kv_stride_in_bytes,
                gpu_block_stride_in_bytes, chunk_size_in_bytes, buffer, is_mla) -> None:
    _require_int64_host(gpu_block_id_tensor, "gpu_block_id_tensor")
    _require_int64_host(gpu_layer_ptrs_tensor, "gpu_layer_ptrs_tensor")
    if not isinstance(buffer, torch.Tensor) or not buffer.is_contiguous():
        raise TypeError("buffer must be a contiguous torch.Tensor")
    stream = _stream_handle(fn_name)
    lib = _lib.load()
    rc = getattr(lib, fn_name)(
        int(gpu_block_id_tensor.numel()), int(gpu_layer_ptrs_tensor.numel()),
        gpu_block_id_tensor.data_ptr(), gpu_layer_ptrs_tensor.data_ptr(),
        int(gpu_kv_stride_in_bytes), int(gpu_block_stride_in_bytes), int(chunk_size_in_bytes),
        buffer.data_ptr(), buffer.numel() * buffer.element_size(), stream, 1 if is_mla else 0)
    if rc != 0:
        raise RuntimeError(_lib.last_error() or f"{fn_name} failed ({rc})")


def gather_kv_blocks(gpu_block_id_tensor: torch.Tensor, gpu_layer_ptrs_tensor: torch.Tensor,
                     gpu_kv_stride_in_bytes: int, gpu_block_stride_in_bytes: int,
                     chunk_size_in_bytes: int, buffer: torch.Tensor, is_mla: bool = False) -> None:
    """Pack the selected blocks of every layer into `buffer`, laid out
    [block][layer][K|V][chunk] (extension; no reference counterpart)."""
    _contiguous("fkv_gather_kv_blocks", gpu_block_id_tensor, gpu_layer_ptrs_tensor,
                gpu_kv_stride_in_bytes, gpu_block_stride_in_bytes, chunk_size_in_bytes, buffer,
                is_mla)


def scatter_kv_blocks(gpu_block_id_tensor: torch.Tensor, gpu_layer_ptrs_tensor: torch.Tensor,
                      gpu_kv_stride_in_bytes: int, gpu_block_stride_in_bytes: int,
                      chunk_size_in_bytes: int, buffer: torch.Tensor, is_mla: bool = False) -> None:
    """Inverse of gather_kv_blocks: unpack `buffer` into the selected blocks."""
    _contiguous("fkv_scatter_kv_blocks", gpu_block_id_tensor, gpu_layer_ptrs_tensor,
                gpu_kv_stride_in_bytes, gpu_block_stride_in_bytes, chunk_size_in_bytes, buffer,
                is_mla)


class LayerwiseTransfer:
    """Handle of an asynchronous, layer-grouped transfer
    (fkv_transfer_kv_blocks_layerwise).  Group g covers layers
    [g * granularity, (g + 1) * granularity) of the call."""

    def __init__(self, handle: int, keep_alive: tuple) -> None:
        self._h = handle
        self._keep = keep_alive
        self._gen = _lib.generation
        lib = _lib.load()
        self.num_groups = lib.fkv_handle_num_groups(handle) if handle else 0

    def _check_group(self, group: int) -> None:
        if self._h is None:
            raise RuntimeError("transfer handle already released")
        if not 0 <= group < self.num_groups:
            raise IndexError(f"group {group} out of range [0, {self.num_groups})")

    def query(self, group: int) -> bool:
        """True once every layer of `group` has landed."""
        self._check_group(group)
        rc = _lib.load().fkv_handle_query(self._h, group)
        if rc < 0:
            raise RuntimeError(_lib.last_error())
        return rc == 1

    def wait(self, group: int = None) -> None:
        """Block the host until `group` (default: the last group) is done."""
        if self.num_groups == 0:
            return
        group = self.num_groups - 1 if group is None else group
        self._check_group(group)
        _lib.check(_lib.load().fkv_handle_wait(self._h, group), "fkv_handle_wait")

    def stream_wait(self, group: int, stream: torch.cuda.Stream = None) -> None:
        """Make `stream` (default: the current stream) wait on the device
        until `group` is done; the host does not block."""
        self._check_group(group)
        st = (stream or torch.cuda.current_stream()).cuda_stream
        _lib.check(_lib.load().fkv_handle_stream_wait(self._h, group, st),
                   "fkv_handle_stream_wait")

    def release(self) -> None:
        """Wait for every group, then free the handle (idempotent; after
        the library's exit-time finalize the handle is already gone)."""
        h, self._h = self._h, None
        self._keep = ()
        if h and self._gen == _lib.generation:
            _lib.check(_lib.load().fkv_handle_release(h), "fkv_handle_release")

    def __enter__(self) -> "LayerwiseTransfer":
        return self

    def __exit__(self, *exc) -> None:
        self.release()

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass


def transfer_kv_blocks_layerwise(gpu_block_id_tensor: torch.Tensor,
                                 gpu_layer_ptrs_tensor: torch.Tensor,
                                 gpu_kv_stride_in_bytes: int, gpu_block_stride_in_bytes: int,
                                 cpu_block_id_tensor: torch.Tensor, cpu_tensor: torch.Tensor,
                                 cpu_kv_stride_in_bytes: int, cpu_layer_stride_in_bytes: int,
                                 cpu_block_stride_in_bytes: int, chunk_size_in_bytes: int,
                                 start_layer_id: int, layer_granularity: int,
                                 transfer_sms: int = -1, is_host_to_device: bool = True,
                                 is_mla: bool = False,
                                 use_ce_transfer: bool = False) -> LayerwiseTransfer:
    """Start the transfer of every layer group, after the work queued on the
    current stream, and return at once (extension; the reference issues one
    synchronous call per layer group).  Arguments as transfer_kv_blocks plus
    layer_granularity.  use_ce_transfer=False enqueues the zero-copy kernel
    of every group on the current stream; True moves a host-to-device
    transfer from block-wise host rows on the copy engines, driven by a
    library thread, with each group's event recorded once its copies have
    landed (other transfers take the kernel)."""
    import ctypes

    _require_int64_host(gpu_block_id_tensor, "gpu_block_id_tensor")
    _require_int64_host(cpu_block_id_tensor, "cpu_block_id_tensor")
    _require_int64_host(gpu_layer_ptrs_tensor, "gpu_layer_ptrs_tensor")
    if not isinstance(cpu_tensor, torch.Tensor):
        raise TypeError(f"cpu_tensor must be a torch.Tensor, got {type(cpu_tensor).__name__}")
    if cpu_block_id_tensor.numel() != gpu_block_id_tensor.numel():
        raise RuntimeError("gpu and cpu block id tensors differ in length")
    stream = _stream_handle("transfer_kv_blocks_layerwise")
    lib = _lib.load()
    out = ctypes.c_void_p()
    rc = lib.fkv_transfer_kv_blocks_layerwise(
        int(gpu_block_id_tensor.numel()), int(start_layer_id),
        int(gpu_layer_ptrs_tensor.numel()), int(layer_granularity),
        gpu_block_id_tensor.data_ptr(), gpu_layer_ptrs_tensor.data_ptr(),
        int(gpu_kv_stride_in_bytes), int(gpu_block_stride_in_bytes),
        cpu_block_id_tensor.data_ptr(), cpu_tensor.data_ptr(), int(cpu_kv_stride_in_bytes),
        int(cpu_layer_stride_in_bytes), int(cpu_block_stride_in_bytes), 0,
        int(chunk_size_in_bytes), stream, int(transfer_sms),
        1 if is_host_to_device else 0,
        _lib.FKV_XFER_CE if use_ce_transfer else _lib.FKV_XFER_KERNEL,
        1 if is_mla else 0, ctypes.byref(out))
    if rc != 0:
        raise RuntimeError(_lib.last_error() or f"fkv_transfer_kv_blocks_layerwise failed ({rc})")
    return LayerwiseTransfer(out.value, (cpu_tensor,))


_LAYERWISE_SCATTERED = {"kernel": 0, "rect_copies": 1}


def set_copy_engine_policy(min_bytes=None, layerwise_scattered=None) -> None:
    """How use_ce_transfer=True chooses its path, process-wide (extension;
    fkv_set_copy_engine_policy).  ``min_bytes``: transfers moving fewer
    bytes take the zero-copy kernel (default 32 MiB).  ``layerwise_scattered``:
    a layer-wise host cache with scattered ids moves with the zero-copy
    kernel ("kernel", the default: link rate, but it holds compute units, and
    a whole-device GEMM beside it slows 1.4-1.9x) or with one SDMA rect copy
    per block ("rect_copies": one engine, about 47 GB/s at the Llama-3-8B
    shape, compute keeps its speed).  None leaves a setting as it is; "unset"
    returns it to the FLEXKV_CE_* environment variable or the default."""
    keep = -2
    mb = keep if min_bytes is None else (-1 if min_bytes == "unset" else min_bytes)
    if not (mb in (keep, -1) or (isinstance(mb, int) and not isinstance(mb, bool) and mb >= 0)):
        raise ValueError(f"min_bytes must be a non-negative int or 'unset', got {min_bytes!r}")
    if layerwise_scattered is None:
        rc = keep
    elif layerwise_scattered == "unset":
        rc = -1
    elif layerwise_scattered in _LAYERWISE_SCATTERED:
        rc = _LAYERWISE_SCATTERED[layerwise_scattered]
    else:
        raise ValueError("layerwise_scattered must be 'kernel', 'rect_copies' or 'unset', got "
                         f"{layerwise_scattered!r}")
    _lib.check(_lib.load().fkv_set_copy_engine_policy(int(mb), int(rc)),
               "fkv_set_copy_engine_policy")


def copy_engine_policy() -> dict:
    """The copy-engine policy in force: {"min_bytes": int, "rect_copies": 0|1,
    "layerwise_scattered": "kernel"|"rect_copies"}."""
    import ctypes
    mb, rc = ctypes.c_int64(), ctypes.c_int()
    _lib.check(_lib.load().fkv_get_copy_engine_policy(ctypes.byref(mb), ctypes.byref(rc)),
               "fkv_get_copy_engine_policy")
    return {"min_bytes": mb.value, "rect_copies": rc.value,
            "layerwise_scattered": "rect_copies" if rc.value else "kernel"}


def transfer_stream(num_cus: int = 0) -> torch.cuda.ExternalStream:
    """A torch stream on its own hardware queue (fkv_stream_create) for
    transfers meant to overlap with compute; num_cus = 0 keeps every compute
    unit.  Destroy it with release_transfer_stream once no work uses it; one
    still alive at process exit is destroyed by the library's exit hook."""
    import ctypes

    lib = _lib.load()
    out = ctypes.c_void_p()
    _lib.check(lib.fkv_stream_create(int(num_cus), ctypes.byref(out)), "fkv_stream_create")
    _stream_gen[out.value] = _lib.generation
    return torch.cuda.ExternalStream(out.value)


# raw handle -> library generation of each stream made by transfer_stream
_stream_gen = {}


def release_transfer_stream(stream: torch.cuda.ExternalStream) -> None:
    """Synchronise and destroy a stream made by transfer_stream
    (fkv_stream_destroy).  The stream object must not be used afterwards."""
    gen = _stream_gen.pop(stream.cuda_stream, None)
    if gen is None:
        raise RuntimeError("not a stream made by transfer_stream, or already released")
    if gen != _lib.generation:
        return                      # the library's finalize destroyed it already
    stream.synchronize()
    _lib.check(_lib.load().fkv_stream_destroy(stream.cuda_stream), "fkv_stream_destroy")


class TPTransferThreadGroup:
    """flexkv.c_ext.TPTransferThreadGroup (csrc/bindings.cpp:144-158,
    csrc/tp_transfer_thread_group.h:30-57) over fkv_tp_group_*: the
    ``num_gpus`` ranks of data-parallel group ``dp_group_id``, each with its
    per-layer cache tensors ``gpu_blocks[rank]`` (its head slice of every
    block), sharing the host cache ``cpu_blocks``.  Rank r's device is the one
    its tensors live on (the reference computes dp_group_id * num_gpus + r),
    so ranks may share a GPU.  The library keeps one thread and one stream per
    rank until close().  Transfers run on those streams, not the current
    torch stream: work the caller queued on other streams must have finished
    (torch.cuda.synchronize()) before a transfer that reads or writes the
    same memory, as with the reference's own streams
    (csrc/tp_transfer_thread_group.cpp:39-43)."""

    def __init__(self, num_gpus: int, gpu_blocks, cpu_blocks: torch.Tensor,
                 dp_group_id: int) -> None:
        import ctypes
        import threading

        self._h = None
        self._gen = _lib.generation
        # held across each transfer and by close(), so a close() from another
        # thread cannot free the group under a running call
        self._lock = threading.Lock()
        if num_gpus < 1 or len(gpu_blocks) != num_gpus:
            raise ValueError(f"gpu_blocks needs one layer list per rank ({num_gpus})")
        num_layers = len(gpu_blocks[0])
        if num_layers == 0 or any(len(b) != num_layers for b in gpu_blocks):
            raise ValueError("every rank needs the same, non-zero number of layers")
        for r, blocks in enumerate(gpu_blocks):
            dev = blocks[0].device
            if dev.type != "cuda" or any(t.device != dev for t in blocks):
                raise ValueError(f"rank {r}: every layer tensor must be on one GPU")
        devices = (ctypes.c_int * num_gpus)(*[b[0].device.index for b in gpu_blocks])
        ptrs = (ctypes.c_void_p * (num_gpus * num_layers))(
            *[t.data_ptr() for b in gpu_blocks for t in b])
        out = ctypes.c_void_p()
        rc = _lib.load().fkv_tp_group_create(num_gpus, devices, ptrs, num_layers,
                                             cpu_blocks.data_ptr(), ctypes.byref(out))
        if rc != 0:
            raise RuntimeError(_lib.last_error() or "fkv_tp_group_create failed")
        self._h = out.value
        # the tensors must outlive the group's pointers to them
        self._keep = (list(map(list, gpu_blocks)), cpu_blocks)
        self.num_gpus = num_gpus
        self.num_layers = num_layers
        self.dp_group_id = dp_group_id

    def tp_group_transfer(self, gpu_block_id_tensor: torch.Tensor, gpu_kv_stride_in_bytes: int,
                          gpu_block_stride_in_bytes: int, gpu_chunk_size_in_bytes: int,
                          cpu_block_id_tensor: torch.Tensor, cpu_kv_stride_in_bytes: int,
                          cpu_layer_stride_in_bytes: int, cpu_block_stride_in_bytes: int,
                          cpu_chunk_size_in_bytes: int, transfer_sms: int,
                          is_host_to_device: bool, use_ce_transfer: bool, layer_id: int,
                          layer_granularity: int, is_mla: bool) -> None:
        """The reference's arguments (csrc/tp_transfer_thread_group.cpp:48-59);
        ``cpu_chunk_size_in_bytes`` only sizes the reference's log line.  Raises
        RuntimeError("tp_group_transfer failed: ...") naming the first failing
        rank, as the reference does (:107)."""
        _require_int64_host(gpu_block_id_tensor, "gpu_block_id_tensor")
        _require_int64_host(cpu_block_id_tensor, "cpu_block_id_tensor")
        n = gpu_block_id_tensor.numel()
        if cpu_block_id_tensor.numel() != n:
            raise ValueError("gpu and cpu block id tensors differ in length")
        with self._lock:
            if self._h is None:
                raise RuntimeError("TP transfer group is closed")
            rc = _lib.load().fkv_tp_group_transfer(
                self._h, n, gpu_block_id_tensor.data_ptr(), int(gpu_kv_stride_in_bytes),
                int(gpu_block_stride_in_bytes), int(gpu_chunk_size_in_bytes),
                cpu_block_id_tensor.data_ptr(), int(cpu_kv_stride_in_bytes),
                int(cpu_layer_stride_in_bytes), int(cpu_block_stride_in_bytes),
                int(transfer_sms), int(bool(is_host_to_device)), int(use_ce_transfer),
                int(layer_id), int(layer_granularity), int(bool(is_mla)))
            if rc != 0:
                raise RuntimeError("tp_group_transfer failed: " + _lib.last_error())

    def close(self) -> None:
        lock = getattr(self, "_lock", None)   # None: __init__ failed before making it
        with lock if lock is not None else contextlib.nullcontext():
            h, self._h = self._h, None
            if h and self._gen == _lib.generation:   # else finalize destroyed it already
                _lib.check(_lib.load().fkv_tp_group_destroy(h), "fkv_tp_group_destroy")

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class SSDIOCTX:
    """Open SSD cache files (csrc/transfer_ssd.h:174-204, bound at
    csrc/bindings.cpp:141-142): ``ssd_files`` maps device index -> file paths,
    every device holding the same number of files.  Each file is opened for
    buffered I/O and, where the file system allows it, O_DIRECT reads.
    ``iouring_entries > 0`` asks for an io_uring ring of that depth (created
    with ``iouring_flags``) that then carries every transfer on this context;
    when the kernel refuses the ring, transfers run pread/pwrite on threads,
    as in the reference (csrc/transfer_ssd.h:19-28).  ``iouring_depth`` is the
    ring's depth, 0 on threads."""

    def __init__(self, ssd_files, num_devices: int, iouring_entries: int = 0,
                 iouring_flags: int = 0) -> None:
        import ctypes

        self._h = None
        if num_devices <= 0:
            raise ValueError("num_devices must be positive")
        lists = [list(ssd_files[d]) for d in range(num_devices)]
        per = len(lists[0])
        if per == 0 or any(len(x) != per for x in lists):
            raise ValueError("every SSD device needs the same, non-zero number of files")
        paths = [p.encode() for x in lists for p in x]
        arr = (ctypes.c_char_p * len(paths))(*paths)
        out = ctypes.c_void_p()
        lib = _lib.load()
        if iouring_entries < 0:
            raise ValueError("iouring_entries must be >= 0")
        rc = lib.fkv_ssd_open(arr, int(num_devices), int(per), int(iouring_entries),
                              int(iouring_flags), ctypes.byref(out))
        if rc != 0:
            raise RuntimeError(_lib.last_error() or "Failed to open file")
        self._h = out.value
        self.num_devices = num_devices
        self.num_files_per_device = per
        self.iouring_depth = int(lib.fkv_ssd_iouring_depth(self._h))

    def stats(self) -> dict:
        """Cumulative I/O counters since the context was opened: bytes read
        with O_DIRECT, bytes read through the page cache, bytes written, file
        requests, io_uring entries and blocking retries."""
        import ctypes

        if self._h is None:
            raise RuntimeError("SSD context is closed")
        out = _lib.SsdStats()
        if _lib.load().fkv_ssd_stats_read(self._h, ctypes.byref(out)) != 0:
            raise RuntimeError(_lib.last_error())
        return out.as_dict()

    def close(self) -> None:
        h, self._h = self._h, None
        if h:
            _lib.load().fkv_ssd_close(h)

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def transfer_kv_blocks_ssd(ioctx: SSDIOCTX, cpu_layer_id_list: torch.Tensor, cpu_tensor_ptr: int,
                           ssd_block_ids: torch.Tensor, cpu_block_ids: torch.Tensor,
                           cpu_layer_stride_in_bytes: int, cpu_kv_stride_in_bytes: int,
                           ssd_layer_stride_in_bytes: int, ssd_kv_stride_in_bytes: int,
                           chunk_size_in_bytes: int, block_stride_in_bytes: int, is_read: bool,
                           num_blocks_per_file: int, round_robin: int = 1,
                           num_threads_per_device: int = 16, is_mla: bool = False) -> None:
    """Host cache <-> SSD files (csrc/bindings.cpp:57-76 and :110-117,
    csrc/transfer_ssd.cpp:182-285): the layers of ``cpu_layer_id_list`` (a
    contiguous int32 range) of each block pair move between the host cache at
    ``cpu_tensor_ptr`` and the files of ``ioctx``.  Blocking; raises
    RuntimeError on an I/O failure."""
    if ssd_block_ids.dtype != torch.int64:
        raise TypeError("ssd_block_ids must be int64")
    if cpu_block_ids.dtype != torch.int64:
        raise TypeError("cpu_block_ids must be int64")
    if ssd_block_ids.numel() != cpu_block_ids.numel():
        raise RuntimeError("ssd and cpu block id tensors differ in length")
    if ioctx._h is None:
        raise RuntimeError("SSD context is closed")
    layers = cpu_layer_id_list.to(torch.int64).tolist()
    if not layers:
        return
    start = int(layers[0])
    if layers != list(range(start, start + len(layers))):
        raise ValueError("cpu_layer_id_list must be a contiguous ascending range")
    sids = ssd_block_ids.contiguous().cpu()
    cids = cpu_block_ids.contiguous().cpu()
    rc = _lib.load().fkv_transfer_kv_blocks_ssd(
        ioctx._h, start, len(layers), int(cpu_tensor_ptr), sids.data_ptr(), cids.data_ptr(),
        int(sids.numel()), int(cpu_layer_stride_in_bytes), int(cpu_kv_stride_in_bytes),
        int(ssd_layer_stride_in_bytes), int(ssd_kv_stride_in_bytes), int(chunk_size_in_bytes),
        int(block_stride_in_bytes), 1 if is_read else 0, int(round_robin),
        int(num_threads_per_device), 1 if is_mla else 0)
    if rc != 0:
        raise RuntimeError(_lib.last_error() or "Failed to transfer data")
