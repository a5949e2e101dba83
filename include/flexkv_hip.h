/*
 * flexkv_hip.h - C ABI of libflexkv_hip.so, the MI355X (gfx950) GPU<->CPU
 * KV-block transfer library.
 *
 * Every entry point takes plain pointers and sizes (no torch types), returns
 * 0 on success or a non-zero status, and never lets a C++ exception cross the
 * boundary.  On failure a message describing the first error is available from
 * fkv_last_error() in the calling thread.  Status values are hipError_t codes:
 * hipErrorInvalidValue (1) for rejected arguments, other hipError_t values for
 * runtime failures.
 *
 * Reference interfaces replaced (paths are relative to the FlexKV source tree):
 *   fkv_transfer_kv_blocks   <- flexkv::transfer_kv_blocks, csrc/transfer.cu:63-132,
 *                               and its pybind wrapper transfer_kv_blocks_binding,
 *                               csrc/bindings.cpp:25-55 (+ m.def at :108-109)
 *   fkv_host_alloc/free      <- CPUAllocator.allocate(pin_memory=True),
 *                               flexkv/storage/allocator.py:93-113
 *   fkv_host_register/...    <- cudaHostRegister / cudaHostUnregister via ctypes,
 *                               flexkv/transfer/worker.py:33-47
 */
#ifndef FLEXKV_HIP_H_
#define FLEXKV_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque stream handle: a hipStream_t (0 = the legacy default stream). */
typedef void* fkv_stream_t;

/* Values of `use_ce_transfer` in fkv_transfer_kv_blocks. */
enum {
  /* Wavefront gather/scatter kernel that loads and stores pinned host memory
   * directly (zero-copy over PCIe).  Same role as the reference kernel mode,
   * csrc/transfer.cu:123-129.  Calls of at most 128 pieces (16 KiB D2H,
   * 8 KiB H2D, each within one chunk) and 4 MiB take a small-transfer kernel
   * whose arguments carry every piece's addresses (FLEXKV_SMALL_KERNEL=0
   * turns it off); larger calls take the tiled kernel. */
  FKV_XFER_KERNEL = 0,
  /* Copy-engine path: a gather kernel packs the selected chunks into a
   * contiguous HBM staging buffer and the SDMA engines move maximal
   * contiguous host runs (D2H); H2D is SDMA into staging followed by a
   * scatter kernel.  A layer-wise host cache whose ids come in runs of
   * consecutive blocks is served with one copy per (layer, K|V) run from
   * layer-major staging; with scattered ids it moves with the zero-copy
   * kernel, since the runtime runs the one SDMA rect copy per block such a
   * transfer needs on a single engine (FLEXKV_CE_RECT_COPIES=1 keeps it on
   * the engines; a transfer of rect copies runs alone).  Staging is
   * double-buffered; the PCIe copies take no compute units.  Each direction
   * has its own staging, and both take engines 0-3, the fast ones across
   * the host link (host-to-device copies shorter than 384 KiB on average
   * spread over engines 0-5, two of which wait for the scatter beside them
   * to end before taking their share); a D2H and an H2D transfer from
   * different threads run at the same time, and while both run their copies
   * split engines 0-7 (device-to-host 0-4, host-to-device 5-7;
   * FLEXKV_SDMA_DUPLEX_D2H), which balances the two.  Transfers under
   * FLEXKV_CE_MIN_BYTES (default 32 MiB; fkv_set_copy_engine_policy) or whose
   * engine copies would move under 128 KiB each move with the zero-copy
   * kernel instead, where the engines' per-copy cost would dominate, and so
   * does every transfer on a device whose engines cannot be set up (one
   * warning on stderr; FLEXKV_SDMA_ENGINES=0 turns them off) and every
   * transfer whose staging buffer cannot be allocated for want of device
   * memory (one warning; the next transfer tries again).  The pieces that
   * run without engine copies beside them (the first gather, the last
   * scatter) are cut short on transfers of FLEXKV_CE_EDGE_MIN_BYTES
   * (default 32 MiB) and more.  Same role as the reference CE mode,
   * csrc/transfer.cu:97-121. */
  FKV_XFER_CE = 1,
  /* The reference's copy-engine algorithm restated literally: one
   * hipMemcpyAsync per (layer, K|V, block) chunk, csrc/transfer.cu:97-121.
   * Kept as a comparison baseline. */
  FKV_XFER_CE_PER_CHUNK = 2
};

/*
 * Move `num_blocks` KV blocks between the per-layer GPU cache and the host
 * cache, for layers [0, num_layers) of `gpu_layer_ptrs` which correspond to
 * host layers [start_layer_id, start_layer_id + num_layers).
 *
 * For chunk (l, k, i), l < num_layers, k < (is_mla ? 1 : 2), i < num_blocks:
 *   gpu chunk = gpu_layer_ptrs[l] + k*gpu_kv_stride_bytes
 *               + gpu_block_ids[i]*gpu_block_stride_bytes
 *   cpu chunk = cpu_ptr + (l + start_layer_id)*cpu_layer_stride_bytes
 *               + k*cpu_kv_stride_bytes + cpu_block_ids[i]*cpu_block_stride_bytes
 *               + cpu_startoff_inside_chunks
 * and chunk_size_bytes bytes are copied cpu->gpu if is_host_to_device, else
 * gpu->cpu (csrc/transfer.cu:39-53).
 *
 * Arguments follow flexkv::transfer_kv_blocks (csrc/transfer.cu:63-70) one for
 * one; `transfer_cus` plays the role of `transfer_sms` (compute units the
 * zero-copy kernel may occupy; -1 = automatic: 8, or 4 for device-to-host
 * calls of 64 MiB and more whose chunks are whole multiples of 4 KiB).
 *
 * Host requirements (checked; violations return hipErrorInvalidValue):
 *   - gpu_block_ids, cpu_block_ids: host memory, num_blocks int64 each,
 *     every id >= 0; gpu_layer_ptrs: host memory, num_layers pointers.
 *   - cpu_ptr: pinned host memory (or device memory) for the kernel and CE
 *     modes; every addressed byte lies inside the allocation holding cpu_ptr,
 *     and every GPU chunk inside the allocation holding its layer pointer.
 *   - kernel mode: chunk_size_bytes, every stride, cpu_startoff and every
 *     base pointer are multiples of 16 bytes.  (The reference kernel
 *     silently drops a tail of chunk_size % 16 bytes, csrc/transfer.cu:35;
 *     this library refuses such geometry instead.)  CE mode takes any
 *     geometry: what the kernels cannot take moves on the per-chunk engine
 *     loop (FKV_XFER_CE_PER_CHUNK), as the reference CE mode moves it.
 * The call is synchronous: it returns after `stream` has drained
 * (csrc/transfer.cu:131).  Different host threads may call concurrently.
 */
int fkv_transfer_kv_blocks(int num_blocks, int start_layer_id, int num_layers,
                           const int64_t* gpu_block_ids,
                           void* const* gpu_layer_ptrs,
                           int64_t gpu_kv_stride_bytes,
                           int64_t gpu_block_stride_bytes,
                           const int64_t* cpu_block_ids, void* cpu_ptr,
                           int64_t cpu_kv_stride_bytes,
                           int64_t cpu_layer_stride_bytes,
                           int64_t cpu_block_stride_bytes,
                           int64_t cpu_startoff_inside_chunks,
                           int64_t chunk_size_bytes, fkv_stream_t stream,
                           int transfer_cus, int is_host_to_device,
                           int use_ce_transfer, int is_mla);

/* As fkv_transfer_kv_blocks, for engines that allocate K and V of a layer
 * separately (e.g. one [N, tokens, heads, dim] tensor each): gpu_kv_ptrs
 * holds num_layers * kv base pointers, [layer][K|V] (kv = 1 for MLA), and the
 * chunk of block b is at ptr + b * gpu_block_stride_bytes.  Same modes,
 * checks and semantics.  No counterpart in the reference, whose kernel needs
 * V = K + gpu_kv_stride within one allocation (csrc/transfer.cu:48-50). */
int fkv_transfer_kv_blocks_kv_ptrs(int num_blocks, int start_layer_id, int num_layers,
                                   const int64_t* gpu_block_ids, void* const* gpu_kv_ptrs,
                                   int64_t gpu_block_stride_bytes,
                                   const int64_t* cpu_block_ids, void* cpu_ptr,
                                   int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                                   int64_t cpu_block_stride_bytes,
                                   int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes,
                                   fkv_stream_t stream, int transfer_cus,
                                   int is_host_to_device, int use_ce_transfer, int is_mla);

/* As fkv_transfer_kv_blocks in kernel mode (FKV_XFER_KERNEL), for callers
 * that cannot allocate memory: tight serving loops and harnesses that forbid
 * allocation.  No counterpart in the reference.  It calls no hipMalloc,
 * hipFree, pinned or other allocating routine: fkv_transfer_kv_blocks stages
 * the id lists in pinned buffers the library allocates; this entry copies
 * them (hipMemcpyAsync on `stream`) into a fixed 1 MiB device array compiled
 * into the library, one per GPU, held until the process ends.  At most 65536
 * blocks per call; more is refused with hipErrorInvalidValue.  Transfers of
 * up to 32 blocks carry their ids in the kernel arguments instead.  Calls on
 * one GPU share that GPU's array: a call holds a per-GPU mutex from its copy
 * into the array until its kernels have finished, so concurrent calls from
 * several threads take turns.  Not for HIP graph capture: the call is
 * synchronous and resolves ids and addresses on the host, so a stream under
 * capture is refused with hipErrorStreamCaptureUnsupported before anything is
 * queued.  Same arguments (without use_ce_transfer), checks and synchronous
 * return as fkv_transfer_kv_blocks; library profiling does not see these
 * calls. */
int fkv_transfer_kv_blocks_noalloc(int num_blocks, int start_layer_id, int num_layers,
                                   const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                                   int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                                   const int64_t* cpu_block_ids, void* cpu_ptr,
                                   int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                                   int64_t cpu_block_stride_bytes,
                                   int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes,
                                   fkv_stream_t stream, int transfer_cus, int is_host_to_device,
                                   int is_mla);

/* Device-side gather / scatter between the per-layer GPU cache and one
 * contiguous buffer laid out [num_blocks][num_layers][K|V][chunk] (block i of
 * the id list at byte offset i * num_layers * kv * chunk).  This is the
 * on-device half of FKV_XFER_CE exposed on its own, for callers that move the
 * packed blocks themselves (RDMA, file I/O, peer GPUs).  The buffer may be
 * device or pinned host memory; buffer_bytes must cover every block.  Same
 * checks and synchronous return as fkv_transfer_kv_blocks.  No counterpart in
 * the reference, which only ever copies between the two caches. */
int fkv_gather_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                         void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                         int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes,
                         void* buffer, size_t buffer_bytes, fkv_stream_t stream, int is_mla);
int fkv_scatter_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                          void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                          int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes,
                          const void* buffer, size_t buffer_bytes, fkv_stream_t stream,
                          int is_mla);

/* Asynchronous, layer-grouped transfer.  Layers [0, num_layers) move in
 * groups of `layer_granularity` consecutive layers, in order, after the work
 * already queued on `stream`; an event marks the end of each group.  The
 * call returns at once, with a handle the caller polls or waits on per
 * group: on the host (fkv_handle_query / fkv_handle_wait) or on the device
 * (fkv_handle_stream_wait makes another stream, e.g. the one running layer l
 * of the model, wait for group g).
 *
 * use_ce_transfer = FKV_XFER_KERNEL: the zero-copy kernel, every group
 * enqueued on `stream` before the call returns; fkv_handle_stream_wait makes
 * the other stream wait on the device, without a host round trip.
 * transfer_cus = -1 selects 2 compute units for host-to-device transfers
 * (enough for the link; the rest of the chip stays with the compute the
 * transfer overlaps) and 8 for device-to-host.
 * use_ce_transfer = FKV_XFER_CE (host to device from block-wise host rows;
 * other transfers take the kernel): the copy engines, so the transfer holds
 * no compute unit while its bytes cross the link.  A library thread moves
 * windows of consecutive groups: one SDMA copy per block and window into
 * double-buffered staging, then, once they have landed, the window's
 * scatter on a library stream with a hardware queue of its own, where the
 * events of the window's groups are recorded.  Windows grow 1, 2, 4, ...
 * groups up to FLEXKV_LAYERWISE_CE_MIN_COPY_BYTES per block (default
 * 256 KiB) and near the end hold at most half of the groups left, so the
 * first group arrives early and the compute a window releases ends while
 * the rest arrive.  Every window spreads its copies over the wide engine
 * set, FLEXKV_SDMA_ENGINES_WIDE engines (default 8, engines 0-7:
 * host-to-device copies on engines 8-15 slow compute kernels running beside
 * them about twofold).  FLEXKV_LAYERWISE_CE_KERNEL_GROUPS=n (default 0)
 * moves the first n groups with the zero-copy kernel before the engines
 * start, so the first group lands sooner.
 * fkv_handle_stream_wait and fkv_handle_wait first wait on the host until
 * the group's event exists (its copies have landed), fkv_handle_query
 * reports 0 until then.
 *
 * Arguments and checks as in fkv_transfer_kv_blocks; the id lists and layer
 * pointers are copied before the call returns.  The caller keeps the GPU
 * cache and host cache alive until the handle is released;
 * fkv_handle_release waits for all groups and frees the handle.  A handle
 * may be waited on and queried from several threads, but its release must
 * not overlap another call on it, and no call may follow it.
 *
 * The reference reaches the same layer-wise schedule with one synchronous
 * call per layer group (worker.py:293-295, layer-wise ops of
 * flexkv/cache/transfer_pattern.py:370-428) and host polling
 * (kvmanager.py:480 wait_at_layer_group). */
typedef struct fkv_transfer_handle_s* fkv_transfer_handle;
int fkv_transfer_kv_blocks_layerwise(
    int num_blocks, int start_layer_id, int num_layers, int layer_granularity,
    const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
    int64_t gpu_block_stride_bytes, const int64_t* cpu_block_ids, void* cpu_ptr,
    int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
    int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes, fkv_stream_t stream,
    int transfer_cus, int is_host_to_device, int use_ce_transfer, int is_mla,
    fkv_transfer_handle* out);
int fkv_handle_num_groups(fkv_transfer_handle h);             /* groups, or -1 */
int fkv_handle_query(fkv_transfer_handle h, int group);       /* 1 done, 0 pending, <0 error */
int fkv_handle_wait(fkv_transfer_handle h, int group);        /* host blocks until done */
int fkv_handle_stream_wait(fkv_transfer_handle h, int group, fkv_stream_t other);
int fkv_handle_release(fkv_transfer_handle h);

/* A stream on its own hardware queue, for transfers that must overlap with
 * compute.  The HIP runtime spreads ordinary streams over a small pool of
 * hardware queues (4 per process by default), so a transfer stream and a
 * compute stream can land on the same queue and run one after the other; a
 * stream created with a CU mask gets a queue of its own.  num_cus = 0 keeps
 * every compute unit; num_cus = n confines the stream's kernels to the first
 * n.  No counterpart in the reference (its worker uses torch.cuda.Stream(),
 * worker.py:253). */
int fkv_stream_create(int num_cus, fkv_stream_t* out);
int fkv_stream_destroy(fkv_stream_t s);

/* Host cache <-> SSD files (host code, no device work).  Same file layout,
 * block mapping and thread fan-out as the reference SSD tier
 * (csrc/transfer_ssd.cpp:17-285 transfer_kv_blocks_ssd, SSDIOCTX at
 * csrc/transfer_ssd.h:174-242): `paths` lists num_devices * files_per_device
 * files, device-major.  SSD block b maps to device (b/rr) % D, device block
 * ((b/rr)/D)*rr + b%rr, file (device block) % F, in-file block
 * (device block) / F; chunk (l, k) of a block sits at
 * in_file*block_stride + l*ssd_layer_stride + k*ssd_kv_stride in the file and
 * at cpu_id*block_stride + l*cpu_layer_stride + k*cpu_kv_stride in host
 * memory.  Layers [start_layer, start_layer + num_layers) move.  Reads use
 * O_DIRECT when chunk_size is a multiple of 4096, into page-aligned bounce
 * buffers that are then copied to host memory.
 * Chunks adjacent in both the file and host memory merge into one request of
 * at most FLEXKV_SSD_MAX_REQUEST_BYTES (default and maximum 1 GiB).
 * Synchronous; returns 0 or 1 with fkv_last_error() set. */
typedef struct fkv_ssd_s* fkv_ssd_t;
/* iouring_entries / iouring_flags are the reference's SSDIOCTX arguments
 * (csrc/transfer_ssd.h:177-178, CacheConfig.ssd_cache_iouring_entries/_flags):
 * entries > 0 asks for an io_uring submission ring of that depth, created
 * with io_uring_setup(entries, flags); every transfer on the handle then
 * queues its requests on the ring from the calling thread (one caller at a
 * time per handle) instead of fanning out over threads.  A ring the kernel
 * refuses leaves the handle on threads, with a warning on stderr, as in the
 * reference (transfer_ssd.h:19-28). */
int fkv_ssd_open(const char* const* paths, int num_devices, int files_per_device,
                 int iouring_entries, int iouring_flags, fkv_ssd_t* out);
/* Depth of the handle's io_uring ring, 0 when transfers use threads (no ring
 * asked for, or the kernel refused it), -1 for a null handle
 * (IOUring::enabled, csrc/transfer_ssd.h:40). */
int fkv_ssd_iouring_depth(fkv_ssd_t h);
/* Cumulative I/O counters of a handle since it was opened, in the spirit of
 * the reference's IOUring::dump (csrc/transfer_ssd.h:124-134): bytes read
 * with O_DIRECT (through the library's page-aligned bounce buffers; O_DIRECT
 * cannot target HIP-pinned host memory), bytes read through the page cache,
 * bytes written, file requests after merging, io_uring entries completed,
 * and requests or ring entries redone with blocking page-cache I/O after
 * O_DIRECT or the ring could not complete them. */
typedef struct {
  int64_t direct_read_bytes;
  int64_t buffered_read_bytes;
  int64_t write_bytes;
  int64_t requests;
  int64_t ring_entries;
  int64_t fallbacks;
} fkv_ssd_stats;
int fkv_ssd_stats_read(fkv_ssd_t h, fkv_ssd_stats* out);
/* Closes the files and frees the context: no transfer on it may be running
 * or start afterwards (transfers on one context from several threads are
 * fine; they take turns on its ring). */
int fkv_ssd_close(fkv_ssd_t h);
int fkv_transfer_kv_blocks_ssd(fkv_ssd_t h, int start_layer, int num_layers, void* cpu_ptr,
                               const int64_t* ssd_block_ids, const int64_t* cpu_block_ids,
                               int num_blocks, int64_t cpu_layer_stride_bytes,
                               int64_t cpu_kv_stride_bytes, int64_t ssd_layer_stride_bytes,
                               int64_t ssd_kv_stride_bytes, int64_t chunk_size_bytes,
                               int64_t block_stride_bytes, int is_read, int round_robin,
                               int num_threads_per_device, int is_mla);

/* Tensor-parallel transfer group: the ranks of one data-parallel group, each
 * holding its own head slice (gpu chunk) of every block, move the same
 * blocks at once, rank r into or out of bytes [r * gpu_chunk, (r + 1) *
 * gpu_chunk) of each host chunk.  Replaces flexkv::TPTransferThreadGroup
 * (csrc/tp_transfer_thread_group.h:30-57, .cpp:23-109).
 *
 * fkv_tp_group_create: `devices[r]` is rank r's device (ranks may share one);
 * `gpu_layer_ptrs` holds num_ranks * num_layers per-layer cache pointers,
 * [rank][layer], each layer laid out as for fkv_transfer_kv_blocks; the host
 * cache `cpu_ptr` is shared.  The group keeps one host thread and one stream
 * per rank until fkv_tp_group_destroy (or fkv_finalize).
 *
 * fkv_tp_group_transfer: tp_group_transfer's arguments
 * (csrc/tp_transfer_thread_group.cpp:48-59) without the host chunk size,
 * which only sizes the reference's log line.  Every rank makes one
 * fkv_transfer_kv_blocks call on its own stream, host layers [layer_id,
 * layer_id + layer_granularity) from rank r's pointers r * num_layers +
 * layer_id onward, at cpu_startoff_inside_chunks = r * gpu_chunk_size_bytes.
 * Synchronous: returns when every rank's call has; on failure, the first
 * failing rank's status and message (fkv_last_error names the rank), and
 * fkv_last_unsafe_host_blocks gathers every rank's.  Differences from the
 * reference: rank r's layer pointers start at r * num_layers (the
 * reference uses r * layer_granularity, which is another rank's table when
 * the window is not every layer); under MLA (every rank holds the same
 * latent) device-to-host is moved by rank 0 alone instead of every rank
 * writing the same bytes, and host-to-device by every rank; devices come
 * from the caller instead of dp_group_id * num_ranks + r.  One transfer of a
 * group runs at a time; transfers of different groups may overlap.  Each
 * rank runs on the group's own stream, so work the caller queued elsewhere on
 * the same memory must be finished first.
 *
 * fkv_tp_group_destroy: waits for a transfer of the group that is running,
 * then stops the rank threads and destroys their streams.  The handle is
 * gone when it returns: no call on it may start during or after it. */
typedef struct fkv_tp_group_s* fkv_tp_group_t;
int fkv_tp_group_create(int num_ranks, const int* devices, void* const* gpu_layer_ptrs,
                        int num_layers, void* cpu_ptr, fkv_tp_group_t* out);
int fkv_tp_group_transfer(fkv_tp_group_t group, int num_blocks, const int64_t* gpu_block_ids,
                          int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                          int64_t gpu_chunk_size_bytes, const int64_t* cpu_block_ids,
                          int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                          int64_t cpu_block_stride_bytes, int transfer_cus,
                          int is_host_to_device, int use_ce_transfer, int layer_id,
                          int layer_granularity, int is_mla);
int fkv_tp_group_destroy(fkv_tp_group_t group);

/* How copy-engine mode (use_ce_transfer = FKV_XFER_CE) chooses between the
 * SDMA engines and the zero-copy kernel, process-wide.  No counterpart in
 * the reference, whose CE mode always copies on the engines.
 *   min_bytes: transfers that move fewer bytes take the zero-copy kernel
 *     (default 32 MiB: below it the kernel is as fast, and holds its compute
 *     units for at most about 0.6 ms); 0 sends every transfer the engines can
 *     take to them.
 *   rect_copies: a layer-wise host cache with scattered ids (no contiguous
 *     host run longer than one chunk) moves with one SDMA rect copy per
 *     block when 1 (the one engine the runtime assigns per direction: about
 *     0.8 of the host link, and compute beside it keeps its speed), with the
 *     zero-copy kernel when 0 (the default: the link's full rate, but any
 *     kernel resident on the compute units slows a whole-device GEMM beside
 *     it).  profiles/results.md holds the measured rates of both.
 * -1 for either unsets it (FLEXKV_CE_MIN_BYTES / FLEXKV_CE_RECT_COPIES, else
 * the default, apply again); -2 keeps it as it is.  fkv_get_copy_engine_policy
 * reads the values in force. */
int fkv_set_copy_engine_policy(int64_t min_bytes, int rect_copies);
int fkv_get_copy_engine_policy(int64_t* min_bytes, int* rect_copies);

/* Message of the last failed call made by this thread ("" if none). */
const char* fkv_last_error(void);

/* Host block ids (cpu_block_ids values) of this thread's last
 * fkv_transfer_kv_blocks or fkv_transfer_kv_blocks_kv_ptrs call whose
 * device-to-host copy-engine copies were given up on: a wait on the copy
 * engines timed out (FLEXKV_SDMA_TIMEOUT_MS), so an engine may still write
 * those blocks' rows of the host cache after the call returned its error.
 * Writes up to `cap` ids to `out` (which may be null when cap is 0) and
 * returns how many there are; 0 after a call that left no copy behind.
 * Such a call fails; its caller must not read those host blocks, nor write
 * them through another path, until the engines are known to be done (the
 * process ends, or fkv_abandoned_copies_pending returns 0).  No counterpart
 * in the reference, whose copy-engine path waits without a bound
 * (csrc/transfer.cu:131). */
int fkv_last_unsafe_host_blocks(int64_t* out, int cap);

/* Copies on device `device` given up on by timed-out copy-engine waits whose
 * completion signals have not yet reached zero (0: every such copy has
 * finished, and the host blocks fkv_last_unsafe_host_blocks named are safe
 * again); negative on error.  No counterpart in the reference. */
int fkv_abandoned_copies_pending(int device);

/* Pinned, device-mapped host allocation (hipHostMalloc).  flags: 0 = runtime
 * default, FKV_HOST_COHERENT / FKV_HOST_NONCOHERENT select the coherence
 * mode explicitly.  Replaces the pinned torch.empty of CPUAllocator. */
enum { FKV_HOST_DEFAULT = 0, FKV_HOST_COHERENT = 1, FKV_HOST_NONCOHERENT = 2 };
int fkv_host_alloc(void** out_ptr, size_t bytes, unsigned flags);
int fkv_host_free(void* ptr);

/* Check that [ptr, ptr+bytes) is pinned host memory usable by the transfer
 * kernels (worker.py:35-41 registers the host cache at worker start).  This
 * library never page-locks existing pageable memory: allocate the host cache
 * with fkv_host_alloc instead.  Returns 0 if the range is pinned, else
 * hipErrorInvalidValue.  fkv_host_unregister is the matching no-op. */
int fkv_host_register(void* ptr, size_t bytes, unsigned flags);
int fkv_host_unregister(void* ptr);

/* Staging buffer used by FKV_XFER_CE on each device, one per direction
 * (bytes, split in two halves).  Takes effect at the next allocation; 0 =
 * default (1 GiB).  fkv_release_staging frees every device's buffers. */
int fkv_set_staging_bytes(size_t bytes);
int fkv_release_staging(void);

/* Set up `device` (-1: the current one) for transfers before the first one:
 * loads the library's kernels, allocates both directions' copy-engine
 * staging, sets up the SDMA engines, creates completion signals and the
 * layer-wise pipeline's stream, and runs one small copy on each engine the
 * library may use, so work the driver queued there (clearing the new staging
 * memory) is done.  Without it the first
 * copy-engine transfer of each direction pays this, 25-50 ms on MI355X.
 * Copy engines that cannot be set up, or staging that does not fit in device
 * memory, are not errors: transfers then use the zero-copy kernel, as they
 * would have.  No counterpart in the reference; for callers that want their
 * first transfer to cost what later ones do (a server before its first
 * request; GPUCPUTransferWorker calls it when it uses the copy engines). */
int fkv_prepare(int device);

/* Release everything the library holds for the process: waits for and frees
 * layer-wise handles never released, synchronises and destroys streams made
 * by fkv_stream_create, waits for queued copy-engine copies and destroys
 * their completion signals and events, frees the staging buffers and the
 * pinned id buffers.  Meant for process exit (the Python loader calls it from
 * an atexit hook), so these objects are gone before the HIP and HSA runtimes
 * run their own exit-time finalizers; the library stays usable afterwards and
 * re-creates what it needs.  Handles released here are invalid afterwards
 * (the handle calls refuse them).  Must not race with transfers on other
 * threads.  No counterpart in the reference, whose extension holds no such
 * resources (csrc/transfer.cu keeps only a cached occupancy). */
int fkv_finalize(void);

/* Optional per-process timing of the library's kernels and DMA batches,
 * measured with HIP events on the stream each one runs on. */
typedef struct fkv_profile {
  int64_t kernel_launches;   /* gather/scatter/zero-copy kernel launches */
  double kernel_ms;          /* sum of their event-measured durations */
  int64_t kernel_bytes;      /* algorithmic bytes they moved */
  int64_t dma_batches;       /* DMA batches issued by FKV_XFER_CE */
  int64_t dma_copies;        /* individual contiguous DMA copies */
  double dma_ms;             /* sum of event-measured DMA batch durations */
  int64_t dma_bytes;
  int64_t dma_held_copies;   /* DMA copies queued only after the scatter beside them ended */
} fkv_profile;
int fkv_profile_enable(int on);     /* also clears the counters */
int fkv_profile_read(fkv_profile* out);

/* Library version string, e.g. "flexkv_hip 0.1 gfx950". */
const char* fkv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLEXKV_HIP_H_ */
