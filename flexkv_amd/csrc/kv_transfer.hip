// kv_transfer.hip - GPU<->CPU KV-block transfer for MI355X (gfx950).
//
// One kernel template moves "chunks": the (layer, K|V, block) pieces of the
// KV cache, each `chunk_size` contiguous bytes on both sides
// (csrc/transfer.cu:39-53 gives the reference addressing).  It is used twice:
//   * zero-copy mode: the "CPU side" is the pinned host cache itself and the
//     kernel's 16-byte loads/stores travel over PCIe;
//   * copy-engine mode: the "CPU side" is a contiguous HBM staging buffer laid
//     out [block][layer][K|V][chunk]; the SDMA engines (queued through HSA)
//     then move maximal contiguous host runs between staging and the host
//     cache.
//
// Work decomposition: a workgroup (4 wavefronts) owns a tile of consecutive
// blocks; it stages the tile's (gpu_id, cpu_id) pairs in LDS, then its
// wavefronts stream the tile's rows (64 lanes x 16 B = 1 KiB) in groups of
// kUnroll rows, issuing all loads of a group before any store.  Rows are
// ordered block -> layer -> K|V -> offset, which is host-address order for the
// block-wise host layout.  Layer base pointers travel in the kernel argument
// block (scalar loads, no PCIe round trip per chunk).

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "flexkv_hip.h"
#include "fkv_error.h"

namespace {

// Rows (64 lanes x 16 B) each wavefront keeps in flight: the zero-copy
// kernel is PCIe bound, the staging gather/scatter HBM bound.  Measured on
// MI355X at the Llama-3-8B shape with 8 CUs: D2H best at 8 rows, H2D at 4.
#ifndef FKV_UNROLL_ZC_D2H
#define FKV_UNROLL_ZC_D2H 8
#endif
#ifndef FKV_UNROLL_ZC_H2D
#define FKV_UNROLL_ZC_H2D 4
#endif
#ifndef FKV_UNROLL_HBM
#define FKV_UNROLL_HBM 32
#endif
// Wave issue priority (s_setprio, 0-3) of the zero-copy kernel, which shares
// compute units with the caller's kernels when transfers overlap compute.
#ifndef FKV_ZC_PRIO
#define FKV_ZC_PRIO 0
#endif
// Staging gather/scatter launch shape: 1 = one workgroup per tile (grid =
// tiles), 0 = an occupancy-sized grid looping over tiles.
#ifndef FKV_HBM_ONEPASS
#define FKV_HBM_ONEPASS 1
#endif
// Tiles per occupancy slot the tiling aims for (zero-copy / staging).
#ifndef FKV_TILE_FACTOR
#define FKV_TILE_FACTOR 4
#endif
#ifndef FKV_TILE_FACTOR_HBM
#define FKV_TILE_FACTOR_HBM 16
#endif
// Cache hints: loads are non-temporal everywhere; stores are non-temporal
// into HBM but plain into pinned host memory (about 2% faster D2H over PCIe).
#ifndef FKV_NT_LOAD
#define FKV_NT_LOAD 1
#endif
#ifndef FKV_NT_STORE_HBM
#define FKV_NT_STORE_HBM 1
#endif
#ifndef FKV_NT_STORE_HOST
#define FKV_NT_STORE_HOST 0
#endif
// The staging scatter (packed HBM -> scattered chunks) has its own knobs.
#ifndef FKV_UNROLL_SCATTER
#define FKV_UNROLL_SCATTER FKV_UNROLL_HBM
#endif
#ifndef FKV_TILE_FACTOR_SCATTER
#define FKV_TILE_FACTOR_SCATTER FKV_TILE_FACTOR_HBM
#endif
#ifndef FKV_NT_LOAD_SCATTER
#define FKV_NT_LOAD_SCATTER FKV_NT_LOAD
#endif
#ifndef FKV_NT_STORE_SCATTER
#define FKV_NT_STORE_SCATTER FKV_NT_STORE_HBM
#endif

constexpr int kThreads = 256;               // 4 wavefronts of 64 lanes
constexpr int kWaves = kThreads / 64;
constexpr int kUnrollHbm = FKV_UNROLL_HBM;
constexpr int kMaxLayersPerLaunch = 128;    // layer pointers in kernel args
constexpr int kMaxTileBlocks = 64;
constexpr int kMaxDevices = 64;
// SDMA engines the copy-engine path spreads its copies over: measured on
// MI355X with 2 MiB copies, one engine moves 45 GB/s, four 56 GB/s in either
// direction, all sixteen 46 GB/s device-to-host.
constexpr int kDefaultSdmaEngines = 4;
// Compute units of the zero-copy kernel when the caller passes -1: enough
// loads/stores in flight to saturate the PCIe Gen5 x16 link (measured on
// MI355X: 8 CUs reach the link's copy rate; more add contention).
constexpr int kAutoZeroCopyCus = 8;
// Layer-wise host-to-device transfers run beside the caller's compute.  Two
// CUs still fill the link for reads from host memory (56.9 vs 57.2 GB/s with
// 8) and leave the rest of the chip to the compute kernels: a 32-layer
// Llama-3-8B load overlapped with per-layer GEMMs finishes in 42.8 ms on 2
// CUs against 46.1 ms on 8.
constexpr int kAutoLayerwiseH2DCus = 2;
constexpr size_t kDefaultStagingBytes = size_t(256) << 20;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Every address the kernel touches is global memory (HBM or mapped pinned
// host memory); saying so lets the compiler emit global_* instead of flat_*.
typedef __attribute__((address_space(1))) u32x4 gvec;

struct CopyArgs {
  const int64_t* ids;        // device-visible (gpu_id, cpu_id) pairs
  char* cpu_base;            // CPU side of launch layer 0, block index 0
  int64_t gpu_kv_stride;
  int64_t gpu_block_stride;
  int64_t cpu_kv_stride;
  int64_t cpu_layer_stride;
  int64_t cpu_block_stride;
  int64_t chunk_vec;         // 16-byte vectors per chunk
  int32_t rows_per_chunk;    // ceil(chunk_vec / 64)
  int32_t num_blocks;
  int32_t num_layers;        // layers in this launch (<= kMaxLayersPerLaunch)
  int32_t kv_dim;
  int32_t tile_blocks;       // a tile is tile_blocks blocks x tile_layers layers
  int32_t tile_layers;
  int32_t tiles_b;           // tiles along the block axis
  int32_t num_tiles;
  int32_t ptrs_per_layer;    // 1: layer_ptr[l] + k*gpu_kv_stride; kv: layer_ptr[l*kv + k]
  uint64_t layer_ptr[kMaxLayersPerLaunch];
};

// A value every lane of the wavefront holds, moved to a scalar register.
__device__ inline int64_t wave_uniform(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// kH2D: copy CPU side -> GPU side.  kIotaCpu: the CPU side is staging and
// block i of the launch sits at CPU-side block index i (ids[2i+1] unused).
// Row addresses are wave-uniform (scalar registers); each lane adds its own
// 16-byte slot, so one 32-bit lane offset serves every access.
template <bool kH2D, bool kIotaCpu>
__global__ __launch_bounds__(kThreads) void kv_chunk_copy_kernel(CopyArgs a) {
  constexpr bool kScatter = kIotaCpu && kH2D;
  constexpr int kUnroll = kIotaCpu ? (kScatter ? FKV_UNROLL_SCATTER : kUnrollHbm)
                                   : (kH2D ? FKV_UNROLL_ZC_H2D : FKV_UNROLL_ZC_D2H);
  // only the zero-copy D2H instantiation stores into host memory
  constexpr bool kNtStore = kScatter ? FKV_NT_STORE_SCATTER
                                     : ((kIotaCpu || kH2D) ? FKV_NT_STORE_HBM : FKV_NT_STORE_HOST);
  constexpr bool kNtLoad = kScatter ? FKV_NT_LOAD_SCATTER : FKV_NT_LOAD;
  __shared__ int64_t s_gid[kMaxTileBlocks];
  __shared__ int64_t s_cid[kMaxTileBlocks];

  if (!kIotaCpu && FKV_ZC_PRIO > 0) __builtin_amdgcn_s_setprio(FKV_ZC_PRIO);
  const int lane = threadIdx.x & 63;
  const uint32_t lane_off = static_cast<uint32_t>(lane) * 16;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kv = static_cast<uint32_t>(a.kv_dim);
  const uint32_t rpc = static_cast<uint32_t>(a.rows_per_chunk);
  const uint32_t ppl = static_cast<uint32_t>(a.ptrs_per_layer);
  // true when every row of a chunk is a full 64-lane row
  const bool full_rows = (a.chunk_vec & 63) == 0;

  for (int tile = blockIdx.x; tile < a.num_tiles; tile += gridDim.x) {
    const int tb = tile % a.tiles_b;
    const int tl = tile / a.tiles_b;
    const int b0 = tb * a.tile_blocks;
    const int nb = min(a.tile_blocks, a.num_blocks - b0);
    const int l0 = tl * a.tile_layers;
    const uint32_t nl = static_cast<uint32_t>(min(a.tile_layers, a.num_layers - l0));
    const uint32_t items_per_block = nl * kv;
    __syncthreads();  // previous tile's readers are done with the LDS ids
    if (threadIdx.x < nb) {
      const int64_t* pr = a.ids + 2 * static_cast<int64_t>(b0 + threadIdx.x);
      s_gid[threadIdx.x] = pr[0];
      s_cid[threadIdx.x] = kIotaCpu ? static_cast<int64_t>(b0 + threadIdx.x) : pr[1];
    }
    __syncthreads();

    const uint32_t rows = static_cast<uint32_t>(nb) * items_per_block * rpc;
    for (uint32_t g = static_cast<uint32_t>(wave) * kUnroll; g < rows;
         g += kWaves * kUnroll) {
      // Decompose the group's first row once; later rows advance a cursor
      // over (block, layer, K|V, row) in that order.
      uint32_t item = g / rpc;
      uint32_t rr = g - item * rpc;
      uint32_t bi = item / items_per_block;
      uint32_t rem = item - bi * items_per_block;
      uint32_t l = rem / kv;
      uint32_t k = rem - l * kv;

      const char* src[kUnroll];
      char* dst[kUnroll];
      bool live[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t bsafe = min(bi, static_cast<uint32_t>(nb - 1));
        const uint32_t layer = static_cast<uint32_t>(l0) + min(l, nl - 1);
        const int64_t gid = wave_uniform(s_gid[bsafe]);
        const int64_t cid = wave_uniform(s_cid[bsafe]);
        const int64_t row_off = static_cast<int64_t>(rr) * (64 * 16);
        char* gpu = reinterpret_cast<char*>(a.layer_ptr[layer * ppl + k * (ppl - 1)]) +
                    static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride + row_off;
        char* cpu = a.cpu_base + static_cast<int64_t>(layer) * a.cpu_layer_stride +
                    static_cast<int64_t>(k) * a.cpu_kv_stride + cid * a.cpu_block_stride + row_off;
        live[u] = (g + u < rows) &&
                  (full_rows || static_cast<int64_t>(rr) * 64 + lane < a.chunk_vec);
        src[u] = kH2D ? cpu : gpu;
        dst[u] = kH2D ? gpu : cpu;
        // advance the cursor by one row
        if (++rr == rpc) {
          rr = 0;
          if (++k == kv) {
            k = 0;
            if (++l == nl) {
              l = 0;
              ++bi;
            }
          }
        }
      }
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (live[u]) {
          const gvec* p = (const gvec*)(src[u] + lane_off);
          if (kNtLoad)
            v[u] = __builtin_nontemporal_load(p);
          else
            v[u] = *p;
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (live[u]) {
          gvec* p = (gvec*)(dst[u] + lane_off);
          if (kNtStore)
            __builtin_nontemporal_store(v[u], p);
          else
            *p = v[u];
        }
      }
    }
  }
}

// A system-scope acquire in every workgroup.  Launched with a workgroup per
// compute unit (so every XCD's L2 takes part) before a kernel reads memory
// the copy engines wrote outside any HIP stream: no stale line survives it.
__global__ __launch_bounds__(64) void acquire_system_kernel() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
}

// ---------------------------------------------------------------------------
// Errors

}  // namespace

namespace fkv_detail {
std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}
}  // namespace fkv_detail

namespace {

#define t_err (::fkv_detail::last_error())

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  t_err = buf;
  return code;
}

#define FKV_HIP(call)                                                          \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess) {                                                    \
      return fail(static_cast<int>(e_), "%s failed: %s (%s:%d)", #call,        \
                  hipGetErrorString(e_), __FILE__, __LINE__);                  \
    }                                                                          \
  } while (0)

constexpr int kInval = static_cast<int>(hipErrorInvalidValue);

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
int query_ptr(const void* p, PtrInfo* out) {
  hipPointerAttribute_t at;
  memset(&at, 0, sizeof(at));
  hipError_t e = hipPointerGetAttributes(&at, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return kInval;
  }
  if (at.type == hipMemoryTypeHost) {
    out->host = true;
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, const_cast<void*>(p), 0) != hipSuccess || dp == nullptr) {
      (void)hipGetLastError();
      return kInval;
    }
    out->dev_ptr = static_cast<char*>(dp);
  } else if (at.type == hipMemoryTypeDevice) {
    out->device = true;
    out->dev_ptr = static_cast<char*>(const_cast<void*>(p));
  } else {
    return kInval;
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
  if (e != hipSuccess || base == nullptr) {
    (void)hipGetLastError();
    return kInval;
  }
  out->base = static_cast<char*>(base);
  out->size = size;
  return 0;
}

// [p + lo, p + hi) must lie inside the allocation described by info.
bool range_inside(const char* p, __int128 lo, __int128 hi, const PtrInfo& info) {
  const __int128 start = static_cast<__int128>(reinterpret_cast<uintptr_t>(p)) + lo;
  const __int128 end = static_cast<__int128>(reinterpret_cast<uintptr_t>(p)) + hi;
  const __int128 a0 = static_cast<__int128>(reinterpret_cast<uintptr_t>(info.base));
  const __int128 a1 = a0 + static_cast<__int128>(info.size);
  return lo <= hi && start >= a0 && end <= a1;
}

// ---------------------------------------------------------------------------
// Per-device state: staging buffer, side stream, events, occupancy.

struct DeviceState {
  std::mutex mu;            // serialises copy-engine transfers on the device
  bool init = false;
  int num_cus = 0;
  int occ_zero_copy[2] = {0, 0};
  int occ_staged[2] = {0, 0};
  char* staging = nullptr;
  size_t staging_bytes = 0;
  // Copy engines: the HSA agents of this GPU and of the host, the SDMA
  // engines usable in each direction, and per staging half a pool of
  // completion signals (one per queued copy, `in_flight` of them in use) and
  // one event (the gather/scatter kernel that last used the half, on the
  // caller's stream).
  bool sdma_init = false;
  hsa_agent_t gpu_agent{}, cpu_agent{};
  std::vector<hsa_amd_sdma_engine_id_t> engines[2];   // [D2H, H2D]
  std::vector<hsa_signal_t> sigs[2];
  size_t in_flight[2] = {0, 0};
  hipEvent_t ev_compute[2] = {nullptr, nullptr};
};

DeviceState g_dev[kMaxDevices];
std::mutex g_init_mu;
std::atomic<size_t> g_staging_request{0};

// Profiling
std::atomic<bool> g_prof_on{false};
std::mutex g_prof_mu;
fkv_profile g_prof{};

template <bool H, bool I>
void* kernel_ptr() {
  return reinterpret_cast<void*>(&kv_chunk_copy_kernel<H, I>);
}

int ensure_device_basics(int dev) {
  DeviceState& d = g_dev[dev];
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (d.init) return 0;
  FKV_HIP(hipDeviceGetAttribute(&d.num_cus, hipDeviceAttributeMultiprocessorCount, dev));
  int o = 0;
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<false, false>(), kThreads, 0));
  d.occ_zero_copy[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<true, false>(), kThreads, 0));
  d.occ_zero_copy[1] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<false, true>(), kThreads, 0));
  d.occ_staged[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<true, true>(), kThreads, 0));
  d.occ_staged[1] = std::max(1, o);
  d.init = true;
  return 0;
}

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

// Thread-local pinned buffer holding the packed (gpu_id, cpu_id) pairs the
// kernels read.  Calls are synchronous, so the previous call's kernels have
// finished before the buffer is rewritten or regrown.  Buffers are not freed
// at thread exit (the runtime may already be gone at process exit).
struct PinnedIds {
  int64_t* p = nullptr;
  char* dev = nullptr;
  size_t cap = 0;  // bytes
};
thread_local PinnedIds t_ids;

int pinned_ids(size_t bytes, int64_t** host, char** dev) {
  if (bytes > t_ids.cap) {
    if (t_ids.p) FKV_HIP(hipHostFree(t_ids.p));
    t_ids.p = nullptr;
    t_ids.cap = 0;
    size_t cap = std::max<size_t>(bytes, 64 << 10);
    void* p = nullptr;
    FKV_HIP(hipHostMalloc(&p, cap, hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent));
    void* dp = nullptr;
    FKV_HIP(hipHostGetDevicePointer(&dp, p, 0));
    t_ids.p = static_cast<int64_t*>(p);
    t_ids.dev = static_cast<char*>(dp);
    t_ids.cap = cap;
  }
  *host = t_ids.p;
  *dev = t_ids.dev;
  return 0;
}

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

int validate(Geometry& g, int mode) {
  if (g.num_blocks < 0 || g.num_layers < 0 || g.start_layer < 0)
    return fail(kInval, "negative count: num_blocks=%d num_layers=%d start_layer_id=%d",
                g.num_blocks, g.num_layers, g.start_layer);
  if (!g.gids || !g.cids || !g.layer_ptrs || !g.cpu_ptr)
    return fail(kInval, "null pointer argument");
  if (g.chunk <= 0) return fail(kInval, "chunk_size_in_bytes must be positive, got %lld", (long long)g.chunk);
  if (g.gks < 0 || g.gbs < 0 || g.cks < 0 || g.cls < 0 || g.cbs < 0 || g.startoff < 0)
    return fail(kInval, "strides and cpu_startoff_inside_chunks must be non-negative");
  const bool vec_mode = (mode == FKV_XFER_KERNEL || mode == FKV_XFER_CE);
  if (vec_mode) {
    const int64_t vals[] = {g.chunk, g.gks, g.gbs, g.cks, g.cls, g.cbs, g.startoff};
    for (int64_t v : vals)
      if (v % 16 != 0)
        return fail(kInval,
                    "kernel/CE transfer needs chunk size, strides and start offset in "
                    "multiples of 16 bytes (chunk=%lld gkv=%lld gblk=%lld ckv=%lld "
                    "clayer=%lld cblk=%lld startoff=%lld)",
                    (long long)g.chunk, (long long)g.gks, (long long)g.gbs, (long long)g.cks,
                    (long long)g.cls, (long long)g.cbs, (long long)g.startoff);
    if (reinterpret_cast<uintptr_t>(g.cpu_ptr) % 16 != 0)
      return fail(kInval, "cpu_ptr is not 16-byte aligned");
  }
  // Host must be able to read ids and the layer table.
  g.min_gid = g.min_cid = INT64_MAX;
  g.max_gid = g.max_cid = -1;
  for (int i = 0; i < g.num_blocks; ++i) {
    const int64_t a = g.gids[i], b = g.cids[i];
    if (a < 0 || b < 0)
      return fail(kInval, "negative block id at position %d (gpu %lld, cpu %lld)", i,
                  (long long)a, (long long)b);
    g.min_gid = std::min(g.min_gid, a);
    g.max_gid = std::max(g.max_gid, a);
    g.min_cid = std::min(g.min_cid, b);
    g.max_cid = std::max(g.max_cid, b);
  }
  if (query_ptr(g.cpu_ptr, &g.cpu_info) != 0)
    return fail(kInval, "cpu_ptr %p is not pinned host or device memory known to HIP "
                "(allocate the host cache with fkv_host_alloc / pin_memory=True)", g.cpu_ptr);
  const __int128 lo = static_cast<__int128>(g.start_layer) * g.cls +
                      static_cast<__int128>(g.min_cid) * g.cbs + g.startoff;
  const __int128 hi = static_cast<__int128>(g.start_layer + g.num_layers - 1) * g.cls +
                      static_cast<__int128>(g.kv - 1) * g.cks +
                      static_cast<__int128>(g.max_cid) * g.cbs + g.startoff + g.chunk;
  if (!range_inside(g.cpu_ptr, lo, hi, g.cpu_info))
    return fail(kInval,
                "cpu block ids [%lld, %lld] with layers [%d, %d) address bytes outside the "
                "host cache allocation (%zu bytes)",
                (long long)g.min_cid, (long long)g.max_cid, g.start_layer,
                g.start_layer + g.num_layers, g.cpu_info.size);
  const __int128 glo = static_cast<__int128>(g.min_gid) * g.gbs;
  const __int128 ghi = static_cast<__int128>(g.kv - 1) * g.gks +
                       static_cast<__int128>(g.max_gid) * g.gbs + g.chunk;
  // Every layer (or K/V) pointer is its own allocation as a rule; query each.
  if (g.ptrs_per_layer != 1 && (g.ptrs_per_layer != g.kv || g.gks != 0))
    return fail(kInval, "separate K/V pointers need kv pointers per layer and no kv stride");
  const int64_t nptr = static_cast<int64_t>(g.num_layers) * g.ptrs_per_layer;
  for (int64_t i = 0; i < nptr; ++i) {
    const char* p = static_cast<const char*>(g.layer_ptrs[i]);
    if (!p) return fail(kInval, "gpu layer pointer %lld is null", (long long)i);
    if (vec_mode && reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(kInval, "gpu layer pointer %lld is not 16-byte aligned", (long long)i);
    PtrInfo pi;
    if (query_ptr(p, &pi) != 0 || !pi.device)
      return fail(kInval, "gpu layer pointer %lld (%p) is not device memory", (long long)i, p);
    if (!range_inside(p, glo, ghi, pi))
      return fail(kInval,
                  "gpu block ids [%lld, %lld] address bytes outside the allocation of "
                  "layer pointer %lld (%zu bytes)",
                  (long long)g.min_gid, (long long)g.max_gid, (long long)i, pi.size);
  }
  return 0;
}

void prof_add_kernel(double ms, int64_t bytes) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof.kernel_launches += 1;
  g_prof.kernel_ms += ms;
  g_prof.kernel_bytes += bytes;
}

void prof_add_dma(double ms, int64_t copies, int64_t bytes) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof.dma_batches += 1;
  g_prof.dma_copies += copies;
  g_prof.dma_ms += ms;
  g_prof.dma_bytes += bytes;
}

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

// Tiles are tb blocks x tl layers.  Start from whole block rows (one block,
// every layer) and halve the layer window until there are about `factor`
// tiles per occupancy slot of the grid; when blocks are plentiful, group
// several per tile so one LDS id load serves more rows.  Rows per tile stay
// below 2^31.  Measured on MI355X (2 GiB gather at the Llama-3-8B shape):
// 32 rows in flight per wavefront with one workgroup per tile and 16 tiles
// per slot reaches the device's plain-copy rate (~5.9 TB/s).
void choose_tiles(int nb, int nl, int kv, int rpc, int grid_cap, int factor, CopyArgs* a) {
  const int64_t target = factor * static_cast<int64_t>(std::max(1, grid_cap));
  auto tiles = [&](int tb, int tl) {
    return static_cast<int64_t>((nb + tb - 1) / tb) * ((nl + tl - 1) / tl);
  };
  int tb = 1, tl = nl;
  while (tl > 1 && tiles(tb, tl) < target) tl = (tl + 1) / 2;
  while (tb < kMaxTileBlocks && tiles(tb * 2, tl) >= target) tb *= 2;
  while (tb > 1 && static_cast<int64_t>(tb) * tl * kv * rpc >= (int64_t(1) << 31)) tb /= 2;
  while (tl > 1 && static_cast<int64_t>(tb) * tl * kv * rpc >= (int64_t(1) << 31)) tl = (tl + 1) / 2;
  a->tile_blocks = tb;
  a->tile_layers = tl;
  a->tiles_b = (nb + tb - 1) / tb;
  a->num_tiles = static_cast<int32_t>(tiles(tb, tl));
}

// Fill the per-launch part of CopyArgs and launch over `nb` blocks starting at
// block `b0` of the (already packed) id list, for GPU layers [l0, l0 + nl).
// `cpu_base` is the CPU-side address of launch layer 0 of block index 0.
template <bool kH2D, bool kIota>
int launch_copy(const Geometry& g, char* ids_dev, char* cpu_base, int64_t cks, int64_t cls,
                int64_t cbs, int b0, int nb, int l0, int nl, int grid_cap,
                hipStream_t stream, ProfRecorder& prof) {
  CopyArgs a;
  memset(&a, 0, sizeof(a));
  a.ids = reinterpret_cast<const int64_t*>(ids_dev) + 2 * static_cast<int64_t>(b0);
  a.cpu_base = cpu_base;
  a.gpu_kv_stride = g.gks;
  a.gpu_block_stride = g.gbs;
  a.cpu_kv_stride = cks;
  a.cpu_layer_stride = cls;
  a.cpu_block_stride = cbs;
  a.chunk_vec = g.chunk / 16;
  a.rows_per_chunk = static_cast<int32_t>((a.chunk_vec + 63) / 64);
  a.num_blocks = nb;
  a.num_layers = nl;
  a.kv_dim = g.kv;
  a.ptrs_per_layer = g.ptrs_per_layer;
  for (int i = 0; i < nl * g.ptrs_per_layer; ++i)
    a.layer_ptr[i] = reinterpret_cast<uint64_t>(g.layer_ptrs[l0 * g.ptrs_per_layer + i]);
  choose_tiles(nb, nl, g.kv, a.rows_per_chunk, grid_cap,
               kIota ? (kH2D ? FKV_TILE_FACTOR_SCATTER : FKV_TILE_FACTOR_HBM) : FKV_TILE_FACTOR,
               &a);
  int grid = std::max(1, std::min(grid_cap, a.num_tiles));
  if (kIota && FKV_HBM_ONEPASS) grid = a.num_tiles;
  hipEvent_t ev = nullptr;
  if (prof.begin(stream, &ev)) return kInval;
  (void)hipGetLastError();  // a stale error from elsewhere must not be blamed on this launch
  hipLaunchKernelGGL((kv_chunk_copy_kernel<kH2D, kIota>), dim3(grid), dim3(kThreads), 0, stream, a);
  FKV_HIP(hipGetLastError());
  return prof.end(stream, ev, static_cast<int64_t>(nb) * nl * g.kv * g.chunk, 0, false);
}

void pack_ids_into(const Geometry& g, int64_t* h) {
  for (int i = 0; i < g.num_blocks; ++i) {
    h[2 * i] = g.gids[i];
    h[2 * i + 1] = g.cids[i];
  }
}

// Pack ids into the thread's pinned buffer as (gpu_id, cpu_id) pairs.
int pack_ids(const Geometry& g, char** ids_dev) {
  int64_t* h = nullptr;
  int rc = pinned_ids(static_cast<size_t>(g.num_blocks) * 16, &h, ids_dev);
  if (rc) return rc;
  pack_ids_into(g, h);
  return 0;
}

int stream_device(hipStream_t s, int* dev) {
  if (s == nullptr) {
    FKV_HIP(hipGetDevice(dev));
  } else {
    FKV_HIP(hipStreamGetDevice(s, dev));
  }
  if (*dev < 0 || *dev >= kMaxDevices) return fail(kInval, "device %d out of range", *dev);
  return 0;
}

// The HSA entry points the copy-engine path needs, resolved from the HSA
// runtime that the process's HIP runtime uses.  Binding by name could reach a
// second HSA runtime mapped into the process, which knows nothing of HIP's
// allocations.
struct HsaApi {
  decltype(&::hsa_iterate_agents) iterate_agents = nullptr;
  decltype(&::hsa_amd_pointer_info) pointer_info = nullptr;
  decltype(&::hsa_agent_get_info) agent_get_info = nullptr;
  decltype(&::hsa_status_string) status_string = nullptr;
  decltype(&::hsa_signal_create) signal_create = nullptr;
  decltype(&::hsa_signal_store_screlease) signal_store_screlease = nullptr;
  decltype(&::hsa_signal_wait_scacquire) signal_wait_scacquire = nullptr;
  decltype(&::hsa_amd_memory_copy_engine_status) copy_engine_status = nullptr;
  decltype(&::hsa_amd_memory_async_copy_on_engine) async_copy_on_engine = nullptr;
};
HsaApi g_hsa;
// Wait until every copy queued on a staging half has finished.  Each copy
// has its own signal: a counted signal shared by many copies would depend on
// every layer between here and the engines decrementing it by exactly one.
void sdma_wait(DeviceState& d, int half) {
  for (size_t i = 0; i < d.in_flight[half]; ++i)
    while (g_hsa.signal_wait_scacquire(d.sigs[half][i], HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX,
                                       HSA_WAIT_STATE_BLOCKED) >= 1) {
    }
  d.in_flight[half] = 0;
}

// When a transfer fails after enqueueing work, wait for that work before the
// call returns: a copy must not land in the caller's buffers, or read the
// reused id and staging buffers, after the error has been reported.
struct DrainOnError {
  hipStream_t stream;
  DeviceState* dev_state;
  bool armed = true;
  ~DrainOnError() {
    if (!armed) return;
    (void)hipStreamSynchronize(stream);
    if (dev_state && dev_state->sdma_init)
      for (int h = 0; h < 2; ++h) sdma_wait(*dev_state, h);
    (void)hipGetLastError();
  }
};

int transfer_zero_copy(const Geometry& g, hipStream_t stream, int dev, int transfer_cus,
                       bool h2d) {
  DeviceState& d = g_dev[dev];
  char* ids_dev = nullptr;
  int rc = pack_ids(g, &ids_dev);
  if (rc) return rc;
  DrainOnError drain{stream, nullptr};
  int cus = transfer_cus <= 0 ? std::min(kAutoZeroCopyCus, d.num_cus)
                              : std::min(transfer_cus, d.num_cus);
  const int grid_cap = cus * (h2d ? d.occ_zero_copy[1] : d.occ_zero_copy[0]);
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff +
                  static_cast<int64_t>(g.start_layer) * g.cls;
  ProfRecorder prof;
  const int per_launch = g.layers_per_launch();
  for (int l0 = 0; l0 < g.num_layers; l0 += per_launch) {
    const int nl = std::min(per_launch, g.num_layers - l0);
    char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
    rc = h2d ? launch_copy<true, false>(g, ids_dev, base, g.cks, g.cls, g.cbs, 0,
                                        g.num_blocks, l0, nl, grid_cap, stream, prof)
             : launch_copy<false, false>(g, ids_dev, base, g.cks, g.cls, g.cbs, 0,
                                         g.num_blocks, l0, nl, grid_cap, stream, prof);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

// One contiguous DMA between staging and the host cache.
struct Run {
  int64_t staging_off;
  char* host;
  int64_t bytes;
};

// Host runs for blocks [b0, b0+nb) of a piece whose staging layout is
// [block][layer][kv][chunk] over `nl` layers starting at `l0`.
void build_runs(const Geometry& g, int b0, int nb, int l0, int nl, std::vector<Run>& runs) {
  runs.clear();
  const int64_t row_chunks = static_cast<int64_t>(nl) * g.kv;
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) && (nl == 1 || g.cls == g.kv * g.chunk);
  char* host0 = g.cpu_ptr + g.startoff + static_cast<int64_t>(g.start_layer + l0) * g.cls;
  int64_t soff = 0;
  auto push = [&](char* h, int64_t bytes) {
    if (!runs.empty() && runs.back().host + runs.back().bytes == h &&
        runs.back().staging_off + runs.back().bytes == soff) {
      runs.back().bytes += bytes;
    } else {
      runs.push_back({soff, h, bytes});
    }
    soff += bytes;
  };
  for (int i = b0; i < b0 + nb; ++i) {
    char* hb = host0 + g.cids[i] * g.cbs;
    if (row_contig) {
      push(hb, row_chunks * g.chunk);
    } else {
      for (int l = 0; l < nl; ++l)
        for (int k = 0; k < g.kv; ++k) push(hb + l * g.cls + k * g.cks, g.chunk);
    }
  }
}

int sdma_engines_wanted() {
  const char* e = getenv("FLEXKV_SDMA_ENGINES");
  const int n = e ? atoi(e) : kDefaultSdmaEngines;
  return std::max(1, std::min(n, 32));
}

std::mutex g_hsa_mu;
bool g_hsa_loaded = false;

// The HSA runtime behind HIP is the mapped copy that knows `hip_ptr`, a
// device allocation HIP made: a process can map a second copy (a wheel's
// bundled runtime next to the system one a profiling tool preloaded), and
// which one HIP bound to depends on load order.
int load_hsa(const void* hip_ptr) {
  std::lock_guard<std::mutex> lk(g_hsa_mu);
  if (g_hsa_loaded) return 0;
  std::vector<std::string> paths;
  if (FILE* f = fopen("/proc/self/maps", "r")) {
    char line[4096];
    while (fgets(line, sizeof(line), f)) {
      const char* p = strchr(line, '/');
      if (!p || !strstr(p, "libhsa-runtime64.so")) continue;
      std::string path(p);
      while (!path.empty() && (path.back() == '\n' || path.back() == ' ')) path.pop_back();
      if (std::find(paths.begin(), paths.end(), path) == paths.end()) paths.push_back(path);
    }
    fclose(f);
  }
  void* lib = nullptr;
  for (const std::string& path : paths) {
    void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_NOLOAD);
    if (!h) continue;
    auto info = reinterpret_cast<decltype(&::hsa_amd_pointer_info)>(dlsym(h, "hsa_amd_pointer_info"));
    hsa_amd_pointer_info_t pi;
    memset(&pi, 0, sizeof(pi));
    pi.size = sizeof(pi);
    if (info && info(hip_ptr, &pi, nullptr, nullptr, nullptr) == HSA_STATUS_SUCCESS &&
        pi.type != HSA_EXT_POINTER_TYPE_UNKNOWN) {
      lib = h;
      break;
    }
    dlclose(h);
  }
  if (!lib) return fail(kInval, "no HSA runtime mapped into the process knows HIP's allocations");
  HsaApi a;
  int missing = 0;
  auto sym = [&](auto& fn, const char* name) {
    fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(lib, name));
    if (!fn) ++missing;
  };
  sym(a.iterate_agents, "hsa_iterate_agents");
  sym(a.pointer_info, "hsa_amd_pointer_info");
  sym(a.agent_get_info, "hsa_agent_get_info");
  sym(a.status_string, "hsa_status_string");
  sym(a.signal_create, "hsa_signal_create");
  sym(a.signal_store_screlease, "hsa_signal_store_screlease");
  sym(a.signal_wait_scacquire, "hsa_signal_wait_scacquire");
  sym(a.copy_engine_status, "hsa_amd_memory_copy_engine_status");
  sym(a.async_copy_on_engine, "hsa_amd_memory_async_copy_on_engine");
  if (missing) return fail(kInval, "the HSA runtime lacks %d entry points", missing);
  g_hsa = a;
  g_hsa_loaded = true;
  return 0;
}

hsa_status_t first_cpu_agent(hsa_agent_t a, void* out) {
  hsa_device_type_t t;
  if (g_hsa.agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) == HSA_STATUS_SUCCESS &&
      t == HSA_DEVICE_TYPE_CPU) {
    *static_cast<hsa_agent_t*>(out) = a;
    return HSA_STATUS_INFO_BREAK;
  }
  return HSA_STATUS_SUCCESS;
}

#define FKV_HSA(expr)                                                                   \
  do {                                                                                  \
    hsa_status_t st_ = (expr);                                                          \
    if (st_ != HSA_STATUS_SUCCESS) {                                                    \
      const char* m_ = nullptr;                                                         \
      (void)g_hsa.status_string(st_, &m_);                                                \
      return fail(static_cast<int>(hipErrorUnknown), "%s failed: %s", #expr, m_ ? m_ : "?"); \
    }                                                                                   \
  } while (0)

// HSA agents and SDMA engines for the copy-engine path on device `dev`: the
// GPU agent is the owner of `hip_ptr` (a device allocation HIP made on
// `dev`), the host side is the GPU's nearest CPU agent when the runtime
// reports one, else the first CPU agent.
int ensure_sdma(DeviceState& d, int dev, const void* hip_ptr) {
  if (d.sdma_init) return 0;
  if (int rc = load_hsa(hip_ptr)) return rc;
  hsa_amd_pointer_info_t pi;
  memset(&pi, 0, sizeof(pi));
  pi.size = sizeof(pi);
  FKV_HSA(g_hsa.pointer_info(hip_ptr, &pi, nullptr, nullptr, nullptr));
  hsa_device_type_t t;
  if (pi.agentOwner.handle == 0 ||
      g_hsa.agent_get_info(pi.agentOwner, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS ||
      t != HSA_DEVICE_TYPE_GPU)
    return fail(kInval, "no GPU agent owns the staging buffer of device %d", dev);
  struct {
    hsa_agent_t gpu, cpu;
  } q{pi.agentOwner, {0}};
  const hsa_status_t it = g_hsa.iterate_agents(first_cpu_agent, &q.cpu);
  if ((it != HSA_STATUS_SUCCESS && it != HSA_STATUS_INFO_BREAK) || q.cpu.handle == 0)
    return fail(kInval, "no CPU agent found for device %d", dev);
  hsa_agent_t nearest{};
  if (g_hsa.agent_get_info(q.gpu, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_NEAREST_CPU),
                           &nearest) == HSA_STATUS_SUCCESS && nearest.handle != 0)
    q.cpu = nearest;
  const int want = sdma_engines_wanted();
  for (int dir = 0; dir < 2; ++dir) {
    uint32_t mask = 0;
    FKV_HSA(dir == 0 ? g_hsa.copy_engine_status(q.cpu, q.gpu, &mask)
                     : g_hsa.copy_engine_status(q.gpu, q.cpu, &mask));
    d.engines[dir].clear();
    for (int b = 0; b < 32 && static_cast<int>(d.engines[dir].size()) < want; ++b)
      if (mask & (1u << b))
        d.engines[dir].push_back(static_cast<hsa_amd_sdma_engine_id_t>(1u << b));
    if (d.engines[dir].empty())
      return fail(kInval, "device %d reports no SDMA engine for %s copies", dev,
                  dir == 0 ? "device-to-host" : "host-to-device");
  }
  for (int h = 0; h < 2; ++h)
    FKV_HIP(hipEventCreateWithFlags(&d.ev_compute[h], hipEventDisableTiming));
  d.gpu_agent = q.gpu;
  d.cpu_agent = q.cpu;
  d.sdma_init = true;
  return 0;
}

int ensure_staging(DeviceState& d, size_t need_half) {
  size_t want = g_staging_request.load();
  if (want == 0) want = kDefaultStagingBytes;
  want = std::max(want, 2 * need_half);
  want = (want + 4095) & ~size_t(4095);
  if (d.staging && d.staging_bytes == want) return 0;
  if (d.staging) {
    FKV_HIP(hipFree(d.staging));
    d.staging = nullptr;
    d.staging_bytes = 0;
  }
  void* p = nullptr;
  FKV_HIP(hipMalloc(&p, want));
  d.staging = static_cast<char*>(p);
  d.staging_bytes = want;
  return 0;
}

// Queue the copies of `runs` between the host cache and staging half `half`
// on the device's SDMA engines, round robin, each with its own completion
// signal.
int issue_sdma(DeviceState& d, const std::vector<Run>& runs, char* staging, bool h2d, int half,
               hsa_agent_t host_agent) {
  const std::vector<hsa_amd_sdma_engine_id_t>& eng = d.engines[h2d ? 1 : 0];
  std::vector<hsa_signal_t>& sigs = d.sigs[half];
  while (sigs.size() < runs.size()) {
    hsa_signal_t sg;
    FKV_HSA(g_hsa.signal_create(1, 0, nullptr, &sg));
    sigs.push_back(sg);
  }
  for (size_t i = 0; i < runs.size(); ++i) {
    const Run& r = runs[i];
    char* dev_p = staging + r.staging_off;
    const hsa_amd_sdma_engine_id_t e = eng[i % eng.size()];
    g_hsa.signal_store_screlease(sigs[i], 1);
    const hsa_status_t st =
        h2d ? g_hsa.async_copy_on_engine(dev_p, d.gpu_agent, r.host, host_agent,
                                         static_cast<size_t>(r.bytes), 0, nullptr, sigs[i], e,
                                         false)
            : g_hsa.async_copy_on_engine(r.host, host_agent, dev_p, d.gpu_agent,
                                         static_cast<size_t>(r.bytes), 0, nullptr, sigs[i], e,
                                         false);
    if (st != HSA_STATUS_SUCCESS) {
      const char* m = nullptr;
      (void)g_hsa.status_string(st, &m);
      return fail(static_cast<int>(hipErrorUnknown), "SDMA copy of %lld bytes failed: %s",
                  static_cast<long long>(r.bytes), m ? m : "?");
    }
    d.in_flight[half] = i + 1;
  }
  return 0;
}

// Copy-engine transfer: the SDMA engines move whole-block runs between the
// host cache and double-buffered HBM staging; a gather (D2H) or scatter
// (H2D) kernel on the caller's stream moves them between staging and the
// per-layer cache.  The host thread orders the two, so no compute unit
// takes part in the PCIe copies.
//  D2H, per piece: wait for the half's previous copies -> gather kernel ->
//  wait for it -> queue the half's copies.
//  H2D: queue the copies of the first two pieces; per piece: wait for its
//  copies -> system-scope acquire -> scatter kernel; once that has read the
//  half, queue the copies of the piece two ahead into it.
int transfer_staged(const Geometry& g, hipStream_t stream, int dev, bool h2d) {
  DeviceState& d = g_dev[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  DeviceGuard guard;
  int rc = guard.set(dev);
  if (rc) return rc;
  char* ids_dev = nullptr;
  rc = pack_ids(g, &ids_dev);
  if (rc) return rc;

  // A piece is a run of whole blocks over a layer window; the window covers
  // all layers unless one block row would not fit a staging half.
  const size_t req = g_staging_request.load();
  const size_t half_default = (req ? req : kDefaultStagingBytes) / 2;
  int nl_piece = std::min(g.num_layers, g.layers_per_launch());
  while (nl_piece > 1 && static_cast<size_t>(nl_piece) * g.kv * g.chunk > half_default) nl_piece /= 2;
  const size_t row_bytes = static_cast<size_t>(nl_piece) * g.kv * g.chunk;
  rc = ensure_staging(d, row_bytes);
  if (rc) return rc;
  if ((rc = ensure_sdma(d, dev, d.staging))) return rc;
  const size_t half = d.staging_bytes / 2;
  const int blocks_per_piece = static_cast<int>(std::max<size_t>(1, half / row_bytes));
  const int grid_cap = d.num_cus * (h2d ? d.occ_staged[1] : d.occ_staged[0]);
  const hsa_agent_t host_agent = d.cpu_agent;   // device-resident caches never get here

  struct Piece {
    int l0, nl, b0, nb;
  };
  std::vector<Piece> pieces;
  for (int l0 = 0; l0 < g.num_layers; l0 += nl_piece)
    for (int b0 = 0; b0 < g.num_blocks; b0 += blocks_per_piece)
      pieces.push_back({l0, std::min(nl_piece, g.num_layers - l0), b0,
                        std::min(blocks_per_piece, g.num_blocks - b0)});
  const int np = static_cast<int>(pieces.size());

  // Host-side waits order everything below against the caller's stream, so
  // work already queued on it comes first.
  FKV_HIP(hipStreamSynchronize(stream));
  DrainOnError drain{stream, &d};
  ProfRecorder prof;
  std::vector<Run> runs;
  bool pending[2] = {false, false};
  int64_t dma_copies = 0, dma_bytes = 0;
  const auto t0 = std::chrono::steady_clock::now();
  auto queue_copies = [&](int pi) -> int {
    const Piece& p = pieces[pi];
    const int h = pi & 1;
    build_runs(g, p.b0, p.nb, p.l0, p.nl, runs);
    for (const Run& r : runs) dma_bytes += r.bytes;
    dma_copies += static_cast<int64_t>(runs.size());
    pending[h] = true;
    return issue_sdma(d, runs, d.staging + h * half, h2d, h, host_agent);
  };
  auto launch = [&](int pi) -> int {
    const Piece& p = pieces[pi];
    const int64_t cls = static_cast<int64_t>(g.kv) * g.chunk;   // staging layer stride
    const int64_t cbs = static_cast<int64_t>(p.nl) * cls;       // staging block stride
    char* stg = d.staging + (pi & 1) * half;
    const int64_t cks = g.kv == 1 ? 0 : g.chunk;
    return h2d ? launch_copy<true, true>(g, ids_dev, stg, cks, cls, cbs, p.b0, p.nb, p.l0, p.nl,
                                         grid_cap, stream, prof)
               : launch_copy<false, true>(g, ids_dev, stg, cks, cls, cbs, p.b0, p.nb, p.l0, p.nl,
                                          grid_cap, stream, prof);
  };
  if (!h2d) {
    for (int pi = 0; pi < np; ++pi) {
      const int h = pi & 1;
      if (pending[h]) {
        sdma_wait(d, h);
        pending[h] = false;
      }
      if ((rc = launch(pi))) return rc;
      FKV_HIP(hipEventRecord(d.ev_compute[h], stream));
      FKV_HIP(hipEventSynchronize(d.ev_compute[h]));
      if ((rc = queue_copies(pi))) return rc;
    }
  } else {
    for (int pi = 0; pi < std::min(np, 2); ++pi)
      if ((rc = queue_copies(pi))) return rc;
    for (int pi = 0; pi < np; ++pi) {
      const int h = pi & 1;
      sdma_wait(d, h);
      pending[h] = false;
      hipLaunchKernelGGL(acquire_system_kernel, dim3(d.num_cus), dim3(64), 0, stream);
      FKV_HIP(hipGetLastError());
      if ((rc = launch(pi))) return rc;
      if (pi + 2 < np) {
        FKV_HIP(hipEventRecord(d.ev_compute[h], stream));
        FKV_HIP(hipEventSynchronize(d.ev_compute[h]));
        if ((rc = queue_copies(pi + 2))) return rc;
      }
    }
  }
  for (int h = 0; h < 2; ++h)
    if (pending[h]) sdma_wait(d, h);
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  if (prof.on) {
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    prof_add_dma(ms, dma_copies, dma_bytes);
  }
  prof.flush();
  return 0;
}

// Gather (to_gpu = false) or scatter between the GPU cache and a contiguous
// buffer laid out [block][layer][K|V][chunk]; g.cpu_ptr is the buffer and
// g.cids is 0..n-1.  Uses every compute unit: the copy is HBM-bound.
int transfer_contiguous(const Geometry& g, hipStream_t stream, int dev, bool to_gpu) {
  DeviceState& d = g_dev[dev];
  char* ids_dev = nullptr;
  int rc = pack_ids(g, &ids_dev);
  if (rc) return rc;
  const int grid_cap = d.num_cus * (to_gpu ? d.occ_staged[1] : d.occ_staged[0]);
  DrainOnError drain{stream, nullptr};
  ProfRecorder prof;
  const int per_launch = g.layers_per_launch();
  for (int l0 = 0; l0 < g.num_layers; l0 += per_launch) {
    const int nl = std::min(per_launch, g.num_layers - l0);
    char* base = g.cpu_info.dev_ptr + static_cast<int64_t>(l0) * g.cls;
    rc = to_gpu ? launch_copy<true, true>(g, ids_dev, base, g.cks, g.cls, g.cbs, 0, g.num_blocks,
                                          l0, nl, grid_cap, stream, prof)
                : launch_copy<false, true>(g, ids_dev, base, g.cks, g.cls, g.cbs, 0, g.num_blocks,
                                           l0, nl, grid_cap, stream, prof);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

int contiguous_entry(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                     void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                     int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes, void* buffer,
                     size_t buffer_bytes, fkv_stream_t stream, int is_mla, bool to_gpu) {
  try {
    t_err.clear();
    if (num_blocks == 0 || num_layers == 0) return 0;
    if (num_blocks < 0 || num_layers < 0)
      return fail(kInval, "negative count: num_blocks=%d num_layers=%d", num_blocks, num_layers);
    std::vector<int64_t> iota(static_cast<size_t>(num_blocks));
    for (int i = 0; i < num_blocks; ++i) iota[i] = i;
    Geometry g;
    g.num_blocks = num_blocks;
    g.start_layer = 0;
    g.num_layers = num_layers;
    g.kv = is_mla ? 1 : 2;
    g.gids = gpu_block_ids;
    g.cids = iota.data();
    g.layer_ptrs = gpu_layer_ptrs;
    g.gks = gpu_kv_stride_bytes;
    g.gbs = gpu_block_stride_bytes;
    g.chunk = chunk_size_bytes;
    g.cks = g.kv == 1 ? 0 : chunk_size_bytes;
    g.cls = static_cast<int64_t>(g.kv) * chunk_size_bytes;
    g.cbs = static_cast<int64_t>(num_layers) * g.cls;
    g.startoff = 0;
    g.cpu_ptr = static_cast<char*>(buffer);
    const __int128 need = static_cast<__int128>(num_blocks) * g.cbs;
    if (need > static_cast<__int128>(buffer_bytes))
      return fail(kInval, "buffer holds %zu bytes, the blocks need %lld", buffer_bytes,
                  static_cast<long long>(need));
    int rc = validate(g, FKV_XFER_KERNEL);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    if ((rc = stream_device(s, &dev))) return rc;
    if ((rc = ensure_device_basics(dev))) return rc;
    return transfer_contiguous(g, s, dev, to_gpu);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

// The reference copy-engine loop, csrc/transfer.cu:97-121: one async copy per
// (layer, K|V, block) chunk, issued layer-major then K|V then block.
int transfer_ce_per_chunk(const Geometry& g, hipStream_t stream, bool h2d) {
  DrainOnError drain{stream, nullptr};
  ProfRecorder prof;
  hipEvent_t ev = nullptr;
  int rc = prof.begin(stream, &ev);
  if (rc) return rc;
  for (int l = 0; l < g.num_layers; ++l) {
    for (int k = 0; k < g.kv; ++k) {
      char* gk = g.gpu_base(l, k);
      for (int i = 0; i < g.num_blocks; ++i) {
        char* cpu = g.cpu_ptr + static_cast<int64_t>(l + g.start_layer) * g.cls + k * g.cks +
                    g.cids[i] * g.cbs + g.startoff;
        char* gpu = gk + g.gids[i] * g.gbs;
        if (h2d) {
          FKV_HIP(hipMemcpyAsync(gpu, cpu, g.chunk, hipMemcpyHostToDevice, stream));
        } else {
          FKV_HIP(hipMemcpyAsync(cpu, gpu, g.chunk, hipMemcpyDeviceToHost, stream));
        }
      }
    }
  }
  const int64_t copies = static_cast<int64_t>(g.num_layers) * g.kv * g.num_blocks;
  if ((rc = prof.end(stream, ev, copies * g.chunk, copies, true))) return rc;
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

// ---------------------------------------------------------------------------
// Asynchronous layer-grouped transfers.  A handle owns a pinned id buffer
// from a process-wide pool (returned at release) and one event per group.

struct PoolBuf {
  int64_t* host = nullptr;
  char* dev = nullptr;
  size_t cap = 0;
};
std::mutex g_pool_mu;
std::vector<PoolBuf> g_pool;   // free buffers

int pool_get(size_t bytes, PoolBuf* out) {
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    size_t best = g_pool.size();
    for (size_t i = 0; i < g_pool.size(); ++i)
      if (g_pool[i].cap >= bytes && (best == g_pool.size() || g_pool[i].cap < g_pool[best].cap))
        best = i;
    if (best != g_pool.size()) {
      *out = g_pool[best];
      g_pool.erase(g_pool.begin() + static_cast<long>(best));
      return 0;
    }
  }
  PoolBuf b;
  b.cap = std::max<size_t>(bytes, 64 << 10);
  void* p = nullptr;
  FKV_HIP(hipHostMalloc(&p, b.cap, hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent));
  void* dp = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return fail(static_cast<int>(e), "hipHostGetDevicePointer failed: %s", hipGetErrorString(e));
  }
  b.host = static_cast<int64_t*>(p);
  b.dev = static_cast<char*>(dp);
  *out = b;
  return 0;
}

void pool_put(const PoolBuf& b) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool.push_back(b);
}

}  // namespace

struct fkv_transfer_handle_s {
  int dev = 0;
  hipStream_t stream = nullptr;
  std::vector<hipEvent_t> done;   // one per layer group, in order
  PoolBuf ids;
  ProfRecorder prof;
  bool enqueued = false;          // every group was enqueued
};

namespace {

int layerwise_enqueue(const Geometry& g, hipStream_t stream, int dev, int transfer_cus, bool h2d,
                      int granularity, fkv_transfer_handle_s* h) {
  DeviceState& d = g_dev[dev];
  int rc = pool_get(static_cast<size_t>(g.num_blocks) * 16, &h->ids);
  if (rc) return rc;
  pack_ids_into(g, h->ids.host);
  const int automatic = h2d ? kAutoLayerwiseH2DCus : kAutoZeroCopyCus;
  const int cus = transfer_cus <= 0 ? std::min(automatic, d.num_cus)
                                    : std::min(transfer_cus, d.num_cus);
  const int grid_cap = cus * (h2d ? d.occ_zero_copy[1] : d.occ_zero_copy[0]);
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff + static_cast<int64_t>(g.start_layer) * g.cls;
  for (int g0 = 0; g0 < g.num_layers; g0 += granularity) {
    const int gend = std::min(g.num_layers, g0 + granularity);
    for (int l0 = g0; l0 < gend; l0 += g.layers_per_launch()) {
      const int nl = std::min(g.layers_per_launch(), gend - l0);
      char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
      rc = h2d ? launch_copy<true, false>(g, h->ids.dev, base, g.cks, g.cls, g.cbs, 0,
                                          g.num_blocks, l0, nl, grid_cap, stream, h->prof)
               : launch_copy<false, false>(g, h->ids.dev, base, g.cks, g.cls, g.cbs, 0,
                                           g.num_blocks, l0, nl, grid_cap, stream, h->prof);
      if (rc) return rc;
    }
    hipEvent_t ev = nullptr;
    FKV_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    h->done.push_back(ev);
    FKV_HIP(hipEventRecord(ev, stream));
  }
  h->enqueued = true;
  return 0;
}

// Wait for everything the handle enqueued, then free it.  Safe on a handle
// whose enqueue failed part-way.
int handle_destroy(fkv_transfer_handle_s* h) {
  int rc = 0;
  if (h->enqueued && !h->done.empty()) {
    hipError_t e = hipEventSynchronize(h->done.back());
    if (e != hipSuccess) rc = fail(static_cast<int>(e), "hipEventSynchronize: %s", hipGetErrorString(e));
  } else if (h->ids.host) {  // enqueue failed after taking ids: drain what was issued
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) rc = fail(static_cast<int>(e), "hipStreamSynchronize: %s", hipGetErrorString(e));
  }
  h->prof.flush();
  for (hipEvent_t ev : h->done) (void)hipEventDestroy(ev);
  if (h->ids.host) pool_put(h->ids);
  delete h;
  return rc;
}

Geometry make_geometry(int num_blocks, int start_layer_id, int num_layers,
                       const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                       int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                       const int64_t* cpu_block_ids, void* cpu_ptr, int64_t cpu_kv_stride_bytes,
                       int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
                       int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes, int is_mla) {
  Geometry g;
  g.num_blocks = num_blocks;
  g.start_layer = start_layer_id;
  g.num_layers = num_layers;
  g.kv = is_mla ? 1 : 2;
  g.gids = gpu_block_ids;
  g.cids = cpu_block_ids;
  g.layer_ptrs = gpu_layer_ptrs;
  g.gks = gpu_kv_stride_bytes;
  g.gbs = gpu_block_stride_bytes;
  g.cks = cpu_kv_stride_bytes;
  g.cls = cpu_layer_stride_bytes;
  g.cbs = cpu_block_stride_bytes;
  g.startoff = cpu_startoff_inside_chunks;
  g.chunk = chunk_size_bytes;
  g.cpu_ptr = static_cast<char*>(cpu_ptr);
  return g;
}

// Copy-engine mode hands a transfer to the SDMA engines only when the
// engines pay off: the op moves at least FLEXKV_CE_MIN_BYTES (default 8 MiB)
// and its contiguous host runs are at least 128 KiB.  Each engine copy costs
// about 6 us and the host-side ordering about 40 us per call (MI355X: a
// 1 MiB op of 64 KiB runs takes 77 us on the engines, 39 us in the zero-copy
// kernel); smaller or finer-grained transfers, and caches in device memory,
// go to the zero-copy kernel, with identical results.
constexpr int64_t kCeMinBytesDefault = int64_t(8) << 20;
constexpr int64_t kCeMinRunBytes = int64_t(128) << 10;

bool ce_pays_off(const Geometry& g) {
  // a "host" cache that is device memory has no PCIe copy to offload
  if (g.cpu_info.device) return false;
  const char* e = getenv("FLEXKV_CE_MIN_BYTES");
  const int64_t min_bytes = e ? std::max<int64_t>(0, atoll(e)) : kCeMinBytesDefault;
  const int64_t total = static_cast<int64_t>(g.num_blocks) * g.num_layers * g.kv * g.chunk;
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) &&
                          (g.num_layers == 1 || g.cls == g.kv * g.chunk);
  const int64_t run = row_contig ? static_cast<int64_t>(g.num_layers) * g.kv * g.chunk : g.chunk;
  return total >= min_bytes && (min_bytes == 0 || run >= kCeMinRunBytes);
}

// Validate, then run one synchronous transfer in the requested mode.
int transfer_entry(Geometry& g, hipStream_t s, int transfer_cus, bool h2d, int mode) {
  int rc = validate(g, mode);
  if (rc) return rc;
  int dev = 0;
  if ((rc = stream_device(s, &dev))) return rc;
  if ((rc = ensure_device_basics(dev))) return rc;
  switch (mode) {
    case FKV_XFER_KERNEL:
      return transfer_zero_copy(g, s, dev, transfer_cus, h2d);
    case FKV_XFER_CE:
      if (!ce_pays_off(g)) return transfer_zero_copy(g, s, dev, transfer_cus, h2d);
      return transfer_staged(g, s, dev, h2d);
    default:
      return transfer_ce_per_chunk(g, s, h2d);
  }
}
}  // namespace

extern "C" {

int fkv_transfer_kv_blocks(int num_blocks, int start_layer_id, int num_layers,
                           const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                           int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                           const int64_t* cpu_block_ids, void* cpu_ptr,
                           int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                           int64_t cpu_block_stride_bytes, int64_t cpu_startoff_inside_chunks,
                           int64_t chunk_size_bytes, fkv_stream_t stream, int transfer_cus,
                           int is_host_to_device, int use_ce_transfer, int is_mla) {
  try {
    t_err.clear();
    if (use_ce_transfer < FKV_XFER_KERNEL || use_ce_transfer > FKV_XFER_CE_PER_CHUNK)
      return fail(kInval, "use_ce_transfer must be 0 (kernel), 1 (CE) or 2 (CE per chunk), got %d",
                  use_ce_transfer);
    if (num_blocks == 0 || num_layers == 0) return 0;
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids,
                               gpu_layer_ptrs, gpu_kv_stride_bytes, gpu_block_stride_bytes,
                               cpu_block_ids, cpu_ptr, cpu_kv_stride_bytes,
                               cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    return transfer_entry(g, static_cast<hipStream_t>(stream), transfer_cus,
                          is_host_to_device != 0, use_ce_transfer);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_transfer_kv_blocks_kv_ptrs(int num_blocks, int start_layer_id, int num_layers,
                                   const int64_t* gpu_block_ids, void* const* gpu_kv_ptrs,
                                   int64_t gpu_block_stride_bytes, const int64_t* cpu_block_ids,
                                   void* cpu_ptr, int64_t cpu_kv_stride_bytes,
                                   int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
                                   int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes,
                                   fkv_stream_t stream, int transfer_cus, int is_host_to_device,
                                   int use_ce_transfer, int is_mla) {
  try {
    t_err.clear();
    if (use_ce_transfer < FKV_XFER_KERNEL || use_ce_transfer > FKV_XFER_CE_PER_CHUNK)
      return fail(kInval, "use_ce_transfer must be 0 (kernel), 1 (CE) or 2 (CE per chunk), got %d",
                  use_ce_transfer);
    if (num_blocks == 0 || num_layers == 0) return 0;
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids, gpu_kv_ptrs,
                               0, gpu_block_stride_bytes, cpu_block_ids, cpu_ptr,
                               cpu_kv_stride_bytes, cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    g.ptrs_per_layer = g.kv;
    return transfer_entry(g, static_cast<hipStream_t>(stream), transfer_cus,
                          is_host_to_device != 0, use_ce_transfer);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_gather_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                         void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                         int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes, void* buffer,
                         size_t buffer_bytes, fkv_stream_t stream, int is_mla) {
  return contiguous_entry(num_blocks, num_layers, gpu_block_ids, gpu_layer_ptrs,
                          gpu_kv_stride_bytes, gpu_block_stride_bytes, chunk_size_bytes, buffer,
                          buffer_bytes, stream, is_mla, false);
}

int fkv_scatter_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                          void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                          int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes,
                          const void* buffer, size_t buffer_bytes, fkv_stream_t stream,
                          int is_mla) {
  return contiguous_entry(num_blocks, num_layers, gpu_block_ids, gpu_layer_ptrs,
                          gpu_kv_stride_bytes, gpu_block_stride_bytes, chunk_size_bytes,
                          const_cast<void*>(buffer), buffer_bytes, stream, is_mla, true);
}

int fkv_transfer_kv_blocks_layerwise(
    int num_blocks, int start_layer_id, int num_layers, int layer_granularity,
    const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
    int64_t gpu_block_stride_bytes, const int64_t* cpu_block_ids, void* cpu_ptr,
    int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
    int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes, fkv_stream_t stream,
    int transfer_cus, int is_host_to_device, int is_mla, fkv_transfer_handle* out) {
  try {
    t_err.clear();
    if (!out) return fail(kInval, "out handle pointer is null");
    *out = nullptr;
    if (layer_granularity < 1) return fail(kInval, "layer_granularity must be >= 1");
    if (num_blocks < 0 || num_layers < 0)
      return fail(kInval, "negative count: num_blocks=%d num_layers=%d", num_blocks, num_layers);
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids,
                               gpu_layer_ptrs, gpu_kv_stride_bytes, gpu_block_stride_bytes,
                               cpu_block_ids, cpu_ptr, cpu_kv_stride_bytes,
                               cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* h = new fkv_transfer_handle_s();
    h->stream = s;
    int rc = 0;
    if (num_blocks > 0 && num_layers > 0) {
      if ((rc = validate(g, FKV_XFER_KERNEL)) || (rc = stream_device(s, &h->dev)) ||
          (rc = ensure_device_basics(h->dev)) ||
          (rc = layerwise_enqueue(g, s, h->dev, transfer_cus, is_host_to_device != 0,
                                  layer_granularity, h))) {
        const std::string msg = t_err;
        (void)handle_destroy(h);
        t_err = msg;
        return rc;
      }
    }
    *out = h;
    return 0;
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_handle_num_groups(fkv_transfer_handle h) {
  t_err.clear();
  if (!h) return fail(-1, "null handle");
  return static_cast<int>(h->done.size());
}

int fkv_handle_query(fkv_transfer_handle h, int group) {
  t_err.clear();
  if (!h || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(-1, "bad handle or group %d", group);
  hipError_t e = hipEventQuery(h->done[group]);
  if (e == hipSuccess) return 1;
  (void)hipGetLastError();
  if (e == hipErrorNotReady) return 0;
  return fail(-static_cast<int>(e), "hipEventQuery: %s", hipGetErrorString(e));
}

int fkv_handle_wait(fkv_transfer_handle h, int group) {
  t_err.clear();
  if (!h || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(kInval, "bad handle or group %d", group);
  FKV_HIP(hipEventSynchronize(h->done[group]));
  return 0;
}

int fkv_handle_stream_wait(fkv_transfer_handle h, int group, fkv_stream_t other) {
  t_err.clear();
  if (!h || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(kInval, "bad handle or group %d", group);
  FKV_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(other), h->done[group], 0));
  return 0;
}

int fkv_handle_release(fkv_transfer_handle h) {
  t_err.clear();
  if (!h) return 0;
  return handle_destroy(h);
}

int fkv_stream_create(int num_cus, fkv_stream_t* out) {
  t_err.clear();
  if (!out) return fail(kInval, "out stream pointer is null");
  *out = nullptr;
  int dev = 0;
  FKV_HIP(hipGetDevice(&dev));
  int ncu = 0;
  FKV_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  if (num_cus < 0 || num_cus > ncu)
    return fail(kInval, "num_cus must be in [0, %d], got %d", ncu, num_cus);
  const int use = num_cus == 0 ? ncu : num_cus;
  std::vector<uint32_t> mask(static_cast<size_t>((ncu + 31) / 32), 0u);
  for (int c = 0; c < use; ++c) mask[c / 32] |= 1u << (c % 32);
  hipStream_t st = nullptr;
  FKV_HIP(hipExtStreamCreateWithCUMask(&st, static_cast<uint32_t>(mask.size()), mask.data()));
  *out = st;
  return 0;
}

int fkv_stream_destroy(fkv_stream_t s) {
  t_err.clear();
  if (s) FKV_HIP(hipStreamDestroy(static_cast<hipStream_t>(s)));
  return 0;
}

const char* fkv_last_error(void) { return t_err.c_str(); }

int fkv_host_alloc(void** out_ptr, size_t bytes, unsigned flags) {
  t_err.clear();
  if (!out_ptr) return fail(kInval, "out_ptr is null");
  *out_ptr = nullptr;
  if (bytes == 0) return fail(kInval, "zero-byte host allocation");
  unsigned hf = hipHostMallocPortable | hipHostMallocMapped;
  if (flags == FKV_HOST_COHERENT) hf |= hipHostMallocCoherent;
  else if (flags == FKV_HOST_NONCOHERENT) hf |= hipHostMallocNonCoherent;
  else if (flags != FKV_HOST_DEFAULT) return fail(kInval, "unknown host alloc flags %u", flags);
  FKV_HIP(hipHostMalloc(out_ptr, bytes, hf));
  return 0;
}

int fkv_host_free(void* ptr) {
  t_err.clear();
  if (!ptr) return 0;
  FKV_HIP(hipHostFree(ptr));
  return 0;
}

int fkv_host_register(void* ptr, size_t bytes, unsigned flags) {
  t_err.clear();
  (void)flags;
  if (!ptr || bytes == 0) return fail(kInval, "null or empty range");
  PtrInfo pi;
  if (query_ptr(ptr, &pi) != 0 || !pi.host)
    return fail(kInval,
                "host range %p is not pinned; allocate the host cache pinned "
                "(fkv_host_alloc or pin_memory=True) instead of registering pageable memory",
                ptr);
  if (!range_inside(static_cast<char*>(ptr), 0, static_cast<__int128>(bytes), pi))
    return fail(kInval, "host range %p + %zu exceeds its pinned allocation (%zu bytes)", ptr,
                bytes, pi.size);
  return 0;
}

int fkv_host_unregister(void* ptr) {
  (void)ptr;
  t_err.clear();
  return 0;
}

int fkv_set_staging_bytes(size_t bytes) {
  t_err.clear();
  g_staging_request.store(bytes);
  return 0;
}

int fkv_release_staging(void) {
  t_err.clear();
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    DeviceState& d = g_dev[dev];
    std::lock_guard<std::mutex> lk(d.mu);
    if (d.staging) {
      DeviceGuard guard;
      int rc = guard.set(dev);
      if (rc) return rc;
      FKV_HIP(hipFree(d.staging));
      d.staging = nullptr;
      d.staging_bytes = 0;
    }
  }
  return 0;
}

int fkv_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof = fkv_profile{};
  g_prof_on.store(on != 0);
  return 0;
}

int fkv_profile_read(fkv_profile* out) {
  if (!out) return kInval;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  *out = g_prof;
  return 0;
}

const char* fkv_version(void) { return "flexkv_hip 0.1 gfx950"; }

}  // extern "C"
