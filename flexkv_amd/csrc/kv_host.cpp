// kv_host.cpp - host-only parts of the transfer library: error messages,
// pointer classification and bounds, argument validation, the pinned id
// buffers the kernels read, profiling counters, and the entry points that do
// no device work of their own (streams, host allocations, staging size,
// profiling, version).

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "kv_internal.h"

namespace fkv_detail {

std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}

std::vector<int64_t>& last_unsafe_host_blocks() {
  static thread_local std::vector<int64_t> ids;
  return ids;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

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

bool range_inside(const char* p, __int128 lo, __int128 hi, const PtrInfo& info) {
  const __int128 start = static_cast<__int128>(reinterpret_cast<uintptr_t>(p)) + lo;
  const __int128 end = static_cast<__int128>(reinterpret_cast<uintptr_t>(p)) + hi;
  const __int128 a0 = static_cast<__int128>(reinterpret_cast<uintptr_t>(info.base));
  const __int128 a1 = a0 + static_cast<__int128>(info.size);
  return lo <= hi && start >= a0 && end <= a1;
}

DeviceState g_dev[kMaxDevices];
std::atomic<size_t> g_staging_request{0};

// Profiling
std::atomic<bool> g_prof_on{false};

namespace {
std::mutex g_prof_mu;
fkv_profile g_prof{};

// The pool of pinned id buffers (ids_acquire / ids_release).
std::mutex g_ids_mu;
std::vector<IdBuf> g_ids_free;

// The per-device pools of device id buffers (dev_ids_acquire / _release).
std::mutex g_dev_ids_mu;
std::vector<IdBuf> g_dev_ids_free[kMaxDevices];

// Streams made by fkv_stream_create and not destroyed yet; fkv_finalize
// destroys them.
std::mutex g_streams_mu;
std::vector<hipStream_t> g_streams;
}  // namespace

int ids_acquire(size_t bytes, IdBuf* out) {
  {
    std::lock_guard<std::mutex> lk(g_ids_mu);
    size_t best = g_ids_free.size();
    for (size_t i = 0; i < g_ids_free.size(); ++i)
      if (g_ids_free[i].cap >= bytes &&
          (best == g_ids_free.size() || g_ids_free[i].cap < g_ids_free[best].cap))
        best = i;
    if (best != g_ids_free.size()) {
      *out = g_ids_free[best];
      g_ids_free.erase(g_ids_free.begin() + static_cast<long>(best));
      return 0;
    }
  }
  // Capacities are powers of two (at least 64 KiB), so rising request sizes
  // leave at most one buffer per size class in the pool, not one per size.
  IdBuf b;
  b.cap = size_t(64) << 10;
  while (b.cap < bytes) b.cap <<= 1;
  void* p = nullptr;
  FKV_HIP(hipHostMalloc(&p, b.cap, hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent));
  void* dp = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return fail(static_cast<int>(e), "hipHostGetDevicePointer failed: %s", hipGetErrorString(e));
  }
  b.host = static_cast<int64_t*>(p);
  b.dev = static_cast<char*>(dp);
  *out = b;
  return 0;
}

void ids_release(const IdBuf& b) {
  std::lock_guard<std::mutex> lk(g_ids_mu);
  g_ids_free.push_back(b);
}

int ids_pool_free() {
  std::vector<IdBuf> bufs;
  {
    std::lock_guard<std::mutex> lk(g_ids_mu);
    bufs.swap(g_ids_free);
  }
  int rc = 0;
  for (const IdBuf& b : bufs) {
    const hipError_t e = hipHostFree(b.host);
    if (e != hipSuccess && rc == 0)
      rc = fail(static_cast<int>(e), "hipHostFree of an id buffer: %s", hipGetErrorString(e));
  }
  return rc;
}

int dev_ids_acquire(int dev, size_t bytes, IdBuf* out) {
  {
    std::lock_guard<std::mutex> lk(g_dev_ids_mu);
    std::vector<IdBuf>& pool = g_dev_ids_free[dev];
    size_t best = pool.size();
    for (size_t i = 0; i < pool.size(); ++i)
      if (pool[i].cap >= bytes && (best == pool.size() || pool[i].cap < pool[best].cap)) best = i;
    if (best != pool.size()) {
      *out = pool[best];
      pool.erase(pool.begin() + static_cast<long>(best));
      return 0;
    }
  }
  IdBuf b;
  b.cap = size_t(64) << 10;
  while (b.cap < bytes) b.cap <<= 1;
  DeviceGuard guard;
  int rc = guard.set(dev);
  if (rc) return rc;
  void* p = nullptr;
  FKV_HIP(hipMalloc(&p, b.cap));
  b.dev = static_cast<char*>(p);
  *out = b;
  return 0;
}

void dev_ids_release(int dev, const IdBuf& b) {
  std::lock_guard<std::mutex> lk(g_dev_ids_mu);
  g_dev_ids_free[dev].push_back(b);
}

int dev_ids_pool_free() {
  int rc = 0;
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    std::vector<IdBuf> bufs;
    {
      std::lock_guard<std::mutex> lk(g_dev_ids_mu);
      bufs.swap(g_dev_ids_free[dev]);
    }
    if (bufs.empty()) continue;
    DeviceGuard guard;
    const int r = guard.set(dev);
    if (r) {
      if (!rc) rc = r;
      continue;
    }
    for (const IdBuf& b : bufs) {
      const hipError_t e = hipFree(b.dev);
      if (e != hipSuccess && rc == 0)
        rc = fail(static_cast<int>(e), "hipFree of a device id buffer: %s", hipGetErrorString(e));
    }
  }
  return rc;
}

int streams_destroy_all() {
  std::vector<hipStream_t> streams;
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    streams.swap(g_streams);
  }
  int rc = 0;
  for (hipStream_t s : streams) {
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipStreamDestroy(s);
    if (e != hipSuccess && rc == 0)
      rc = fail(static_cast<int>(e), "destroying a library stream: %s", hipGetErrorString(e));
  }
  return rc;
}

bool geometry_vec16(const Geometry& g) {
  const int64_t vals[] = {g.chunk, g.gks, g.gbs, g.cks, g.cls, g.cbs, g.startoff};
  for (int64_t v : vals)
    if (v % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(g.cpu_ptr) % 16 != 0) return false;
  if (g.layer_ptrs && g.num_layers > 0) {
    const int64_t nptr = static_cast<int64_t>(g.num_layers) * g.ptrs_per_layer;
    for (int64_t i = 0; i < nptr; ++i)
      if (reinterpret_cast<uintptr_t>(g.layer_ptrs[i]) % 16 != 0) return false;
  }
  return true;
}

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

void prof_add_dma(double ms, int64_t copies, int64_t bytes, int64_t held_copies) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof.dma_batches += 1;
  g_prof.dma_copies += copies;
  g_prof.dma_ms += ms;
  g_prof.dma_bytes += bytes;
  g_prof.dma_held_copies += held_copies;
}

void pack_ids_into(const Geometry& g, int64_t* h) {
  for (int i = 0; i < g.num_blocks; ++i) {
    h[2 * i] = g.gids[i];
    h[2 * i + 1] = g.cids[i];
  }
}

int pack_ids(const Geometry& g, IdLease& lease) {
  int rc = ids_acquire(static_cast<size_t>(g.num_blocks) * 16, &lease.buf);
  if (rc) return rc;
  pack_ids_into(g, lease.buf.host);
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

}  // namespace fkv_detail

using namespace fkv_detail;

extern "C" {

int fkv_stream_create(int num_cus, fkv_stream_t* out) {
  last_error().clear();
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
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    g_streams.push_back(st);
  }
  *out = st;
  return 0;
}

int fkv_stream_destroy(fkv_stream_t s) {
  last_error().clear();
  if (!s) return 0;
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    auto it = std::find(g_streams.begin(), g_streams.end(), static_cast<hipStream_t>(s));
    if (it == g_streams.end())
      return fail(kInval, "stream %p was not made by fkv_stream_create or is already destroyed", s);
    g_streams.erase(it);
  }
  FKV_HIP(hipStreamDestroy(static_cast<hipStream_t>(s)));
  return 0;
}

const char* fkv_last_error(void) { return last_error().c_str(); }

int fkv_last_unsafe_host_blocks(int64_t* out, int cap) {
  const std::vector<int64_t>& ids = last_unsafe_host_blocks();
  const int n = static_cast<int>(ids.size());
  if (out && cap > 0) std::memcpy(out, ids.data(), sizeof(int64_t) * std::min(n, cap));
  return n;
}

int fkv_host_alloc(void** out_ptr, size_t bytes, unsigned flags) {
  last_error().clear();
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
  last_error().clear();
  if (!ptr) return 0;
  FKV_HIP(hipHostFree(ptr));
  return 0;
}

int fkv_host_register(void* ptr, size_t bytes, unsigned flags) {
  last_error().clear();
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
  last_error().clear();
  return 0;
}

int fkv_set_staging_bytes(size_t bytes) {
  last_error().clear();
  g_staging_request.store(bytes);
  return 0;
}

int fkv_release_staging(void) {
  last_error().clear();
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    for (CopyLane& ln : g_dev[dev].lane) {
      std::lock_guard<std::mutex> lk(ln.mu);
      // a stalled lane's engine may still write its staging buffer
      if (ln.staging && !ln.stalled) {
        DeviceGuard guard;
        int rc = guard.set(dev);
        if (rc) return rc;
        FKV_HIP(hipFree(ln.staging));
        ln.staging = nullptr;
        ln.staging_bytes = 0;
      }
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
