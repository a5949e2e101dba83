// kv_internal.h - declarations shared by the library's translation units:
// kv_transfer.hip (kernels and transfer paths), kv_host.cpp (errors, pointer
// checks, validation, id staging, host-only entry points) and kv_sdma.cpp
// (copy engines through HSA).  Not installed; not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "flexkv_hip.h"
#include "fkv_error.h"
#include "kv_wait.h"

namespace fkv_detail {
#pragma GCC visibility push(hidden)

constexpr int kMaxLayersPerLaunch = 128;    // layer pointers in kernel args
constexpr int kMaxDevices = 64;
// Staging per device and direction (two halves).  Launch size sets the
// gather/scatter rate (MI355X, in a copy-engine transfer at the Llama-3-8B
// shape: gather 4.95 / 5.46 / 5.78 TB/s and scatter 3.58 / 4.32 / 4.78 TB/s
// with 256 MiB / 512 MiB / 1 GiB of staging); 1 GiB is 0.35% of the
// device's 288 GB.
constexpr size_t kDefaultStagingBytes = size_t(1) << 30;
constexpr int kInval = static_cast<int>(hipErrorInvalidValue);

// Set the calling thread's error message; returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define FKV_HIP(call)                                                          \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess) {                                                    \
      return ::fkv_detail::fail(static_cast<int>(e_), "%s failed: %s (%s:%d)", \
                                #call, hipGetErrorString(e_), __FILE__,        \
                                __LINE__);                                     \
    }                                                                          \
  } while (0)

// ---------------------------------------------------------------------------
// Pointer classification and bounds

struct PtrInfo {
  bool host = false;     // pinned host memory
  bool device = false;   // device memory
  char* dev_ptr = nullptr;  // device-visible address of the queried pointer
  char* base = nullptr;     // allocation start (host address space)
  size_t size = 0;          // allocation size
};

// Returns 0 and fills `out` if p lies in memory known to the HIP runtime.
int query_ptr(const void* p, PtrInfo* out);
// [p + lo, p + hi) must lie inside the allocation described by info.
bool range_inside(const char* p, __int128 lo, __int128 hi, const PtrInfo& info);

// ---------------------------------------------------------------------------
// Per-device state: copy-engine lanes, copy engines, occupancy.

// One direction's copy-engine transfers: its staging buffer (two halves),
// per half the completion signals of the queued copies and one event (the
// gather/scatter kernel that last used the half, on the caller's stream).
// Every copy has a signal of its own.  Each engine's last copy of a half
// signals an interrupt signal (`wake`), the host's blocking wait; the others
// signal polled signals (GPU-only consumers: the host reads their values but
// never waits on them), which add no interrupt to the engine's work (small
// copies run 5-25% faster on MI355X).  The two directions have a lane each,
// so a device-to-host and a host-to-device transfer run at the same time.
struct CopyLane {
  std::mutex mu;            // serialises this direction's copy-engine transfers
  char* staging = nullptr;
  size_t staging_bytes = 0;
  std::vector<hsa_signal_t> polled_pool[2], irq_pool[2];   // created on demand, kept
  std::vector<hsa_signal_t> queued[2];   // signal of every copy queued on the half
  std::vector<hsa_signal_t> wake[2];     // the interrupt signals among them
  // pool signals the half's queued copies use (issue_sdma appends after them)
  size_t used_polled[2] = {0, 0}, used_irq[2] = {0, 0};
  hipEvent_t ev_compute[2] = {nullptr, nullptr};
  // A wait on this lane timed out: an engine may still write its staging
  // buffer or decrement its signals, so neither is freed or reused again
  // (the device's copy-engine transfers use the zero-copy kernel from then
  // on).  The signals of the copies given up on are kept here, never destroyed.
  bool stalled = false;
  std::vector<hsa_signal_t> abandoned;
  // host block ids the device-to-host copies of each half write, and those
  // of halves given up on (the device-to-host lane only)
  HostRowLedger rows;
  // stream (own hardware queue) of the copy-engine layer-wise pipeline's
  // scatter kernels, made on first use under stream_mu
  std::mutex stream_mu;
  hipStream_t pipeline_stream = nullptr;
};

struct DeviceState {
  bool init = false;
  int num_cus = 0;
  int occ_zero_copy[2] = {0, 0};
  int occ_staged[2] = {0, 0};   // row-by-row staging kernels, per direction
  int occ_small[2] = {1, 1};   // kv_small_copy_kernel, D2H / H2D
  int occ_whole[2] = {0, 0};    // whole-group staging kernels, per direction
  // Copy engines: the HSA agents of this GPU and of the host and the SDMA
  // engines each direction pins its copies to (disjoint sets where the device
  // has enough engines).
  std::mutex sdma_mu;       // guards the set-up below
  bool sdma_init = false;
  // set-up failed: copy-engine transfers on this device use the zero-copy
  // kernel from then on
  std::atomic<bool> sdma_failed{false};
  // a staging allocation failed for want of device memory (warned once)
  std::atomic<bool> staging_oom_warned{false};
  hsa_agent_t gpu_agent{}, cpu_agent{};
  std::vector<hsa_amd_sdma_engine_id_t> engines[2];   // [D2H, H2D]
  // host-to-device engines of the copy-engine layer-wise pipeline: every
  // engine device-to-host did not take, up to FLEXKV_SDMA_ENGINES_LAYERWISE
  std::vector<hsa_amd_sdma_engine_id_t> engines_wide;
  // the first few of them: short host-to-device copies of synchronous
  // transfers (FLEXKV_SDMA_ENGINES_WIDE_SYNC)
  std::vector<hsa_amd_sdma_engine_id_t> engines_wide_sync;
  // Engines each direction takes while the other direction's copy-engine
  // transfer is in flight (FLEXKV_SDMA_DUPLEX_D2H of engines 0-7 for
  // device-to-host, the rest of 0-7 for host-to-device); empty: no split.
  std::vector<hsa_amd_sdma_engine_id_t> engines_duplex[2];
  // copy-engine transfers in flight per direction [D2H, H2D]
  std::atomic<int> busy[2] = {0, 0};
  CopyLane lane[2];                                    // [D2H, H2D]
};

// Counts a copy-engine transfer of one direction as in flight on a device
// for its lifetime (DeviceState::busy), so the other direction's copies take
// the duplex engine split meanwhile.
struct BusyMark {
  std::atomic<int>& n;
  explicit BusyMark(std::atomic<int>& c) : n(c) { n.fetch_add(1, std::memory_order_relaxed); }
  ~BusyMark() { n.fetch_sub(1, std::memory_order_relaxed); }
  BusyMark(const BusyMark&) = delete;
  BusyMark& operator=(const BusyMark&) = delete;
};

extern DeviceState g_dev[kMaxDevices];
// staging bytes per device and direction asked for with
// fkv_set_staging_bytes (0: default)
extern std::atomic<size_t> g_staging_request;

// Makes a device current for the guard's lifetime.
struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  int set(int dev) {
    FKV_HIP(hipGetDevice(&prev));
    if (prev != dev) {
      FKV_HIP(hipSetDevice(dev));
      changed = true;
    }
    return 0;
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// ---------------------------------------------------------------------------
// Geometry validated on the host before anything is launched.

struct Geometry {
  int num_blocks, start_layer, num_layers, kv;
  const int64_t* gids;
  const int64_t* cids;
  void* const* layer_ptrs;   // num_layers * ptrs_per_layer entries
  int ptrs_per_layer = 1;    // kv when K and V are separate allocations (gks = 0)
  int64_t gks, gbs, cks, cls, cbs, startoff, chunk;
  char* cpu_ptr;
  PtrInfo cpu_info;
  int64_t min_gid, max_gid, min_cid, max_cid;

  // Base address of half k of call layer l (block 0).
  char* gpu_base(int l, int k) const {
    const int64_t i = static_cast<int64_t>(l) * ptrs_per_layer + (ptrs_per_layer > 1 ? k : 0);
    return static_cast<char*>(layer_ptrs[i]) + k * gks;
  }
  // Layers whose pointers fit one launch's kernel arguments.
  int layers_per_launch() const { return kMaxLayersPerLaunch / ptrs_per_layer; }
};

// Check ids, strides, alignment and that every byte the transfer touches lies
// inside the host and device allocations; fills the id ranges and cpu_info.
int validate(Geometry& g, int mode);
// Whether the chunk size, every stride, the start offset, cpu_ptr and every
// layer pointer are multiples of 16 bytes, as the kernels' 16-byte accesses
// need.  Null pointers pass (validate reports them).
bool geometry_vec16(const Geometry& g);

// Profiling (fkv_profile_enable / fkv_profile_read)
extern std::atomic<bool> g_prof_on;
void prof_add_kernel(double ms, int64_t bytes);
void prof_add_dma(double ms, int64_t copies, int64_t bytes, int64_t held_copies = 0);

// Event pairs recorded around launches when profiling is on; read after the
// final synchronisation.
struct ProfSpan {
  hipEvent_t a, b;
  int64_t bytes;
  int64_t copies;
  bool dma;
};

struct ProfRecorder {
  bool on = g_prof_on.load(std::memory_order_relaxed);
  std::vector<ProfSpan> spans;
  int begin(hipStream_t s, hipEvent_t* a) {
    if (!on) return 0;
    FKV_HIP(hipEventCreate(a));
    FKV_HIP(hipEventRecord(*a, s));
    return 0;
  }
  int end(hipStream_t s, hipEvent_t a, int64_t bytes, int64_t copies, bool dma) {
    if (!on) return 0;
    hipEvent_t b;
    FKV_HIP(hipEventCreate(&b));
    FKV_HIP(hipEventRecord(b, s));
    spans.push_back({a, b, bytes, copies, dma});
    return 0;
  }
  // A pair of events for one kernel launched with hipExtLaunchKernelGGL,
  // which stamps the kernel's own start and end into them: no marker packets
  // on the stream, so the span is the kernel alone.  Both null when off.
  int kernel_events(hipEvent_t* a, hipEvent_t* b) {
    *a = *b = nullptr;
    if (!on) return 0;
    FKV_HIP(hipEventCreate(a));
    const hipError_t e = hipEventCreate(b);
    if (e != hipSuccess) {
      (void)hipEventDestroy(*a);
      *a = nullptr;
      return fail(static_cast<int>(e), "hipEventCreate: %s", hipGetErrorString(e));
    }
    return 0;
  }
  void kernel_span(hipEvent_t a, hipEvent_t b, int64_t bytes) {
    if (a && b) spans.push_back({a, b, bytes, 0, false});
  }
  void flush() {
    for (auto& sp : spans) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, sp.a, sp.b) == hipSuccess) {
        if (sp.dma)
          prof_add_dma(ms, sp.copies, sp.bytes);
        else
          prof_add_kernel(ms, sp.bytes);
      }
      (void)hipEventDestroy(sp.a);
      (void)hipEventDestroy(sp.b);
    }
    spans.clear();
  }
  ~ProfRecorder() {
    for (auto& sp : spans) {
      (void)hipEventDestroy(sp.a);
      (void)hipEventDestroy(sp.b);
    }
  }
};

// Pinned, device-mapped id buffers (the packed (gpu_id, cpu_id) pairs the
// kernels read) come from one process-wide pool: a call takes a buffer of at
// least `bytes` and gives it back once its kernels have finished (synchronous
// calls: at return; layer-wise handles: at release).  fkv_finalize frees the
// pool.
struct IdBuf {
  int64_t* host = nullptr;
  char* dev = nullptr;
  size_t cap = 0;
};
int ids_acquire(size_t bytes, IdBuf* out);
void ids_release(const IdBuf& b);
// Frees every buffer in the pool.  A buffer on loan at that moment goes back
// into the pool when its call ends and stays there until the next free.
int ids_pool_free();
// Holds a pool buffer for the scope of a synchronous call.  Declare it before
// the call's DrainOnError, so the drain runs first and no kernel still reads
// the buffer when it goes back to the pool.
struct IdLease {
  IdBuf buf;
  IdLease() = default;
  IdLease(const IdLease&) = delete;
  IdLease& operator=(const IdLease&) = delete;
  ~IdLease() {
    if (buf.host) ids_release(buf);
  }
};
// Device-memory id buffers for the staging kernels, one pool per device
// (hipMalloc, power-of-two capacities from 64 KiB).  A staging transfer
// copies its id pairs into one with a small kernel, so every workgroup reads
// its tile's ids from HBM instead of over PCIe from the pinned buffer.
// Freed by dev_ids_pool_free (fkv_finalize).
int dev_ids_acquire(int dev, size_t bytes, IdBuf* out);
void dev_ids_release(int dev, const IdBuf& b);
int dev_ids_pool_free();
// Holds a device id buffer for the scope of a synchronous call (declare it
// before the call's DrainOnError).
struct DevIdLease {
  int dev = -1;
  IdBuf buf;
  DevIdLease() = default;
  DevIdLease(const DevIdLease&) = delete;
  DevIdLease& operator=(const DevIdLease&) = delete;
  ~DevIdLease() {
    if (buf.dev) dev_ids_release(dev, buf);
  }
};
// Synchronises and destroys every stream made by fkv_stream_create and not
// destroyed yet (fkv_finalize).
int streams_destroy_all();
// Stops and frees every TP transfer group not yet destroyed (kv_tp_group.cpp).
int tp_groups_destroy_all();
// The ids as (gpu_id, cpu_id) pairs.
void pack_ids_into(const Geometry& g, int64_t* h);
// Pack ids into a pool buffer held by `lease` as (gpu_id, cpu_id) pairs.
int pack_ids(const Geometry& g, IdLease& lease);
// The device a stream belongs to (the current device for the null stream).
int stream_device(hipStream_t s, int* dev);

// ---------------------------------------------------------------------------
// Copy engines (kv_sdma.cpp)

// One DMA between staging and the host cache: `bytes` contiguous bytes or,
// with slices > 0, `slices` pieces of `bytes` each, back to back in staging
// and `host_pitch` apart in the host cache (one rect copy).
struct Run {
  int64_t staging_off;
  char* host;
  int64_t bytes;
  int32_t slices = 0;
  int64_t host_pitch = 0;
};

// The host-side distance between consecutive (layer, K|V) chunks of a block
// when an `nl`-layer window of the block is not one contiguous run but its
// chunks still lie at one stride (layer-wise host layouts
// [layer][K|V][block][chunk], MLA), so one rect copy moves the window; else 0.
inline int64_t host_slice_pitch(const Geometry& g, int nl) {
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) && (nl == 1 || g.cls == g.kv * g.chunk);
  if (row_contig) return 0;
  int64_t pitch = 0;
  if (g.kv == 1)
    pitch = g.cls;                      // slice = layer
  else if (nl == 1)
    pitch = g.cks;                      // slice = K|V
  else if (g.cls == g.kv * g.cks)
    pitch = g.cks;                      // slice = layer * kv + K|V
  return pitch >= g.chunk ? pitch : 0;
}

// Whether a layer-wise host cache's ids come in runs of consecutive blocks
// long enough that staging the blocks layer-major ([layer][K|V][block][chunk])
// and copying each (layer, K|V) run linearly beats one rect copy per block:
// the host block stride is one chunk and the average run moves at least
// `min_run_bytes`.
bool layer_major_pays_off(const Geometry& g, int64_t min_run_bytes);

// Host runs for blocks [b0, b0+nb) of a piece over `nl` layers starting at
// `l0`.  Staging block-major ([block][layer][K|V][chunk]): maximal contiguous
// runs when block rows are contiguous in the host cache, one rect copy per
// block when `rect` and host_slice_pitch() allows it, else one run per chunk.
// Staging layer-major ([layer][K|V][block][chunk], `layer_major`): for each
// (layer, K|V), maximal runs of consecutive host blocks.
void build_runs(const Geometry& g, int b0, int nb, int l0, int nl, bool rect, bool layer_major,
                std::vector<Run>& runs);
// Whether the HSA runtime offers rect copies (after ensure_sdma).
bool sdma_rect_available();
// HSA agents and SDMA engines for the copy-engine path on device `dev`, found
// through `hip_ptr`, a device allocation HIP made on `dev`.
int ensure_sdma(DeviceState& d, int dev, const void* hip_ptr);
// A lane staging buffer of at least two halves of `need_half` bytes, and the
// lane's events.
int ensure_staging(CopyLane& lane, size_t need_half);
// Queue the copies of `runs` between the host cache and staging half `half`
// of `lane` on the direction's SDMA engines (`wide`: the layer-wise
// pipeline's wider host-to-device set), round robin, each with its own
// completion signal.  The half must have no copies queued (sdma_wait).
// Engine sets issue_sdma may take: the direction's own, or for host-to-device
// copies the synchronous transfers' wide set or the layer-wise pipeline's.
enum EngineSet { kEnginesOwn = 0, kEnginesWideSync = 1, kEnginesWide = 2 };
// A half's copies whose first stretch runs beside a scatter kernel can hold
// back the engines of the set beyond its first kHoldKeepEngines: issue_sdma
// then queues only the kept engines' share of `runs` and leaves the held
// engines' share, the tail of `runs`, in `deferred`, sized so that held
// engines starting `held_fraction` of the half's time late finish with the
// others.  The caller queues `deferred` (issue_sdma with `held_part`) once the
// scatter is done.  A set of at most kHoldKeepEngines engines holds nothing.
constexpr size_t kHoldKeepEngines = 4;
struct SdmaHold {
  double held_fraction = 0;
  std::vector<Run> deferred;
};
// `held_part`: queue `runs` (a `deferred` list) on the held engines of the set,
// after the copies already queued on the half (on every engine of the set when
// it has no held engines now).
int issue_sdma(DeviceState& d, CopyLane& lane, const std::vector<Run>& runs, char* staging,
               bool h2d, int half, hsa_agent_t host_agent, int wide = kEnginesOwn,
               SdmaHold* hold = nullptr, bool held_part = false);
// Wait until every copy queued on a staging half has finished: block on the
// interrupt signals of the engines' last copies, then check every copy's own
// signal.  An engine runs its copies in order, so the check normally finds
// them done; if one is not, the check reloads it until it is.  A counted signal
// shared by many copies would instead depend on every layer between here and
// the engines decrementing it by exactly one.  `spin` waits actively instead
// of sleeping: for the last wait of a call, where the host's wake-up from a
// sleep that lasted the whole transfer (15-30 us measured) would add to the
// call's time; a wait overlapped with the other half's copies sleeps.
// Bounded: after FLEXKV_SDMA_TIMEOUT_MS (default 20 s) it gives up, marks the
// lane stalled and the device's engines failed, and returns
// hipErrorLaunchTimeOut with the error message set; otherwise 0.
int sdma_wait(DeviceState& d, CopyLane& lane, int half, bool spin = false);
// Readies a lane (its mutex held, its staging allocated, the engines set up)
// before its first transfer: polled completion signals for `copies_per_half`
// copies on each staging half (the pools grow on demand beyond that), and
// one 4 KiB copy between `host` (pinned, at least 64 KiB) and staging on each
// engine the direction may take, waited for, so work the driver queued on
// those engines (clearing newly allocated device memory) is done first.
int sdma_prepare_lane(DeviceState& d, CopyLane& lane, bool h2d, size_t copies_per_half,
                      char* host, size_t host_bytes);
// Waits for a lane's queued copies, then destroys its pooled signals and
// events and frees its staging buffer (a stalled lane keeps its staging and
// signals).  The lane's mutex must be held.
int lane_release(DeviceState& d, CopyLane& lane);

// When a transfer fails after enqueueing work, wait for that work before the
// call returns: a copy must not land in the caller's buffers, or read the
// reused id and staging buffers, after the error has been reported.
// The message of the error being reported is kept: the drain's own waits
// must not replace it.
struct DrainOnError {
  hipStream_t stream;
  DeviceState* dev = nullptr;
  CopyLane* lane = nullptr;
  bool armed = true;
  ~DrainOnError() {
    if (!armed) return;
    const std::string msg = last_error();
    (void)hipStreamSynchronize(stream);
    if (lane && dev)
      for (int h = 0; h < 2; ++h) (void)sdma_wait(*dev, *lane, h);
    (void)hipGetLastError();
    last_error() = msg;
  }
};

#pragma GCC visibility pop
}  // namespace fkv_detail
