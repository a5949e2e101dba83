// kv_sdma.cpp - the copy engines of the copy-engine transfer path: the HSA
// entry points resolved from the runtime HIP uses, the GPU and host agents and
// SDMA engines of a device, its staging buffer, and the queueing of and
// waiting for whole-block copies between staging and the host cache.

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "kv_internal.h"

namespace fkv_detail {

namespace {

// SDMA engines each direction spreads its copies over.  Measured on MI355X
// (16 engines) with 2 MiB copies: four move 56-57 GB/s either way, and
// device-to-host drops to 47 GB/s on eight.  While both directions run they
// take the duplex split instead (kDefaultDuplexD2HEngines).
//
// Engines 0-3 are the fast ones across the host link.  One 1 GiB copy on
// one engine (MI355X, HSA copies pinned to the engine): engines 0-3 move
// 56.9 GB/s device-to-host and 57.4 host-to-device, engines 4-7 12.8 and
// 51.0.  Host-to-device copies on four engines: 640 KiB copies 57.0 GB/s on
// 0-3, 47.3 on 4-7; 2 MiB copies 56.8 / 56.5.  Copies on engines 4-7 also
// slow a scatter kernel beside them more (Llama-3-8B, 512 MiB scatter
// pieces: 0.605 of HBM peak beside engines 4-7, 0.625 beside 0-3).  So both
// directions' one-way sets are engines 0-3.
constexpr int kDefaultSdmaEngines[2] = {4, 4};   // [D2H, H2D]
// Engines 0-7.  Host-to-device copies on engines 8-15 slow compute kernels
// running beside them about twice over, at any copy size: 160 bf16 GEMMs
// [8192x4096]x[4096x4096] took 1.85x / 2.0x their time beside a 56.6 GB/s
// H2D on engines 6-11 / 8-15, against 1.07x on engines 4-7 (MI355X; D2H on
// engines 0-7: 1.09-1.12x).
constexpr uint32_t kComputeFriendlyEngines = 0xFFu;
// The wide engine set (FLEXKV_SDMA_ENGINES_WIDE): host-to-device copies bound
// by the engines' per-copy cost spread over it, those of the copy-engine
// layer-wise pipeline (one block's layer window, 64-256 KiB at Llama-3-8B)
// and synchronous ones shorter than kWideCopyBytes on average; engines 0-3
// first, then 4-7 (256 KiB copies: 56.1 GB/s on engines 0-5, 51.7 on 0-3,
// 50.7 on 4-7 with 0-1).
constexpr int kDefaultWideEngines = 8;
// Synchronous host-to-device transfers whose copies are short spread over the
// first kSyncWideEngines of the wide set instead (FLEXKV_SDMA_ENGINES_WIDE_SYNC).
// Their scatter kernels run while the next piece's copies are in flight, and
// the engines' traffic slows them: measured on MI355X with 640 KiB copies
// over 8 / 6 / 4 engines (4-7 first): scatter pieces 4.26 / 4.65 / 4.90 TB/s.
// The engines beyond the first four hold back while a scatter runs
// (SdmaHold).  The layer-wise pipeline keeps all 8: its one-window copies
// need them (50.6 against 45.6 GB/s on 6).
constexpr int kSyncWideEngines = 6;
// The duplex split (FLEXKV_SDMA_DUPLEX_D2H; 0 turns it off): while a
// transfer of the other direction is in flight, device-to-host copies take
// this many of engines 0-7 and host-to-device copies the rest.  Measured on
// MI355X, one 2 GiB D2H and one 2 GiB H2D at once (Llama-3-8B shape, both
// directions' bytes over the wall time): 69.5 GB/s on the one-way sets
// (D2H 0-3, H2D 4-7), where the host-to-device copies keep the link and
// device-to-host falls to about 22 GB/s while both run; 81.9 / 81.4 / 81.2
// GB/s on splits 5+3 / 5+2 / 6+2; 67.4 on 4+2; 56.2 on 7+1.  One way,
// device-to-host is fastest on four engines (56.5 GB/s, 52.5 on six).
constexpr int kDefaultDuplexD2HEngines = 5;
constexpr int64_t kDefaultMaxCopyBytes = int64_t(4) << 20;

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
  decltype(&::hsa_signal_destroy) signal_destroy = nullptr;
  decltype(&::hsa_system_get_info) system_get_info = nullptr;
  decltype(&::hsa_amd_signal_create) amd_signal_create = nullptr;
  decltype(&::hsa_signal_load_scacquire) signal_load_scacquire = nullptr;
  decltype(&::hsa_signal_store_screlease) signal_store_screlease = nullptr;
  decltype(&::hsa_signal_wait_scacquire) signal_wait_scacquire = nullptr;
  decltype(&::hsa_amd_memory_copy_engine_status) copy_engine_status = nullptr;
  decltype(&::hsa_amd_memory_async_copy_on_engine) async_copy_on_engine = nullptr;
  decltype(&::hsa_amd_memory_async_copy_rect) async_copy_rect = nullptr;   // optional
};
HsaApi g_hsa;

// Engines per direction; FLEXKV_SDMA_ENGINES=0 turns the engines off.
// Engines of one direction (0: device-to-host, 1: host-to-device):
// FLEXKV_SDMA_ENGINES sets both, FLEXKV_SDMA_ENGINES_D2H / _H2D one.
int sdma_engines_wanted(int dir) {
  const char* both = getenv("FLEXKV_SDMA_ENGINES");
  const char* one = getenv(dir == 0 ? "FLEXKV_SDMA_ENGINES_D2H" : "FLEXKV_SDMA_ENGINES_H2D");
  int n = kDefaultSdmaEngines[dir];
  if (both) n = atoi(both);
  if (one) n = atoi(one);
  return std::max(0, std::min(n, 32));
}

std::mutex g_hsa_mu;
bool g_hsa_loaded = false;
// HSA timestamp ticks per millisecond (the unit of a wait's timeout hint);
// 1 GHz until the runtime reports its frequency.
uint64_t g_ticks_per_ms = 1000000;

// FLEXKV_SDMA_TIMEOUT_MS bounds each host wait on a staging half.
int64_t sdma_timeout_ms() {
  const char* e = getenv("FLEXKV_SDMA_TIMEOUT_MS");
  const int64_t v = e ? atoll(e) : kDefaultSdmaTimeoutMs;
  return v > 0 ? v : kDefaultSdmaTimeoutMs;
}

// The signal operations wait_copies needs, on the runtime's own calls.
struct HsaSignalOps {
  hsa_signal_value_t wait(hsa_signal_t s, uint64_t hint, bool spin) {
    return g_hsa.signal_wait_scacquire(s, HSA_SIGNAL_CONDITION_LT, 1, hint,
                                       spin ? HSA_WAIT_STATE_ACTIVE : HSA_WAIT_STATE_BLOCKED);
  }
  hsa_signal_value_t load(hsa_signal_t s) { return g_hsa.signal_load_scacquire(s); }
  uint64_t ticks_per_ms() const { return g_ticks_per_ms; }
};

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
  sym(a.signal_destroy, "hsa_signal_destroy");
  sym(a.system_get_info, "hsa_system_get_info");
  sym(a.amd_signal_create, "hsa_amd_signal_create");
  sym(a.signal_load_scacquire, "hsa_signal_load_scacquire");
  sym(a.signal_store_screlease, "hsa_signal_store_screlease");
  sym(a.signal_wait_scacquire, "hsa_signal_wait_scacquire");
  sym(a.copy_engine_status, "hsa_amd_memory_copy_engine_status");
  sym(a.async_copy_on_engine, "hsa_amd_memory_async_copy_on_engine");
  if (missing) return fail(kInval, "the HSA runtime lacks %d entry points", missing);
  a.async_copy_rect = reinterpret_cast<decltype(a.async_copy_rect)>(
      dlsym(lib, "hsa_amd_memory_async_copy_rect"));
  uint64_t freq = 0;
  if (a.system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &freq) == HSA_STATUS_SUCCESS &&
      freq >= 1000)
    g_ticks_per_ms = freq / 1000;
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

}  // namespace

int sdma_wait(DeviceState& dev, CopyLane& d, int half, bool spin) {
  if (d.queued[half].empty()) return 0;
  // The polled signals are created for GPU consumers, so the host only ever
  // loads their values (any agent may) and never waits on them.
  HsaSignalOps ops;
  const int64_t limit_ms = sdma_timeout_ms();
  const WaitOutcome w = wait_half(ops, d.wake[half], d.queued[half], spin,
                                  std::chrono::steady_clock::now() +
                                      std::chrono::milliseconds(limit_ms),
                                  d.rows, half);
  if (!w.done) {
    // Give up on this half: its copies may still complete (or never), so
    // their signals and the staging buffer are never reused or freed, and
    // the host blocks they write are now in d.rows' unsafe list.
    for (hsa_signal_t s : d.queued[half]) d.abandoned.push_back(s);
    for (int h = 0; h < 2; ++h) {
      auto drop = [&](std::vector<hsa_signal_t>& pool) {
        pool.erase(std::remove_if(pool.begin(), pool.end(),
                                  [&](hsa_signal_t s) {
                                    for (hsa_signal_t a : d.abandoned)
                                      if (a.handle == s.handle) return true;
                                    return false;
                                  }),
                   pool.end());
      };
      drop(d.polled_pool[h]);
      drop(d.irq_pool[h]);
    }
    d.queued[half].clear();
    d.wake[half].clear();
    d.stalled = true;
    dev.sdma_failed.store(true);
    return fail(static_cast<int>(hipErrorLaunchTimeOut),
                "copy-engine copies of staging half %d did not finish within %lld ms (a "
                "completion signal still reads %lld); copy-engine transfers on this device "
                "use the zero-copy kernel from now on (FLEXKV_SDMA_TIMEOUT_MS sets the limit)",
                half, static_cast<long long>(limit_ms), static_cast<long long>(w.value));
  }
  d.queued[half].clear();
  d.wake[half].clear();
  return 0;
}

int lane_release(DeviceState& dev, CopyLane& d) {
  int rc = 0;
  for (int h = 0; h < 2; ++h) {
    const int r = sdma_wait(dev, d, h, false);
    if (r && !rc) rc = r;
  }
  if (d.stalled) return rc;   // an engine may still use the staging buffer and signals
  if (g_hsa_loaded) {
    for (int h = 0; h < 2; ++h) {
      for (hsa_signal_t s : d.polled_pool[h]) (void)g_hsa.signal_destroy(s);
      for (hsa_signal_t s : d.irq_pool[h]) (void)g_hsa.signal_destroy(s);
      d.polled_pool[h].clear();
      d.irq_pool[h].clear();
    }
  }
  for (int h = 0; h < 2; ++h) {
    if (d.ev_compute[h]) {
      const hipError_t e = hipEventDestroy(d.ev_compute[h]);
      if (e != hipSuccess && !rc)
        rc = fail(static_cast<int>(e), "hipEventDestroy: %s", hipGetErrorString(e));
      d.ev_compute[h] = nullptr;
    }
  }
  if (d.staging) {
    const hipError_t e = hipFree(d.staging);
    if (e != hipSuccess && !rc)
      rc = fail(static_cast<int>(e), "hipFree of a staging buffer: %s", hipGetErrorString(e));
    d.staging = nullptr;
    d.staging_bytes = 0;
  }
  std::lock_guard<std::mutex> lk(d.stream_mu);
  if (d.pipeline_stream) {
    hipError_t e = hipStreamSynchronize(d.pipeline_stream);
    if (e == hipSuccess) e = hipStreamDestroy(d.pipeline_stream);
    if (e != hipSuccess && !rc)
      rc = fail(static_cast<int>(e), "destroying the layer-wise pipeline stream: %s",
                hipGetErrorString(e));
    d.pipeline_stream = nullptr;
  }
  return rc;
}

namespace {
// Largest single engine copy (bytes; FLEXKV_SDMA_MAX_COPY_BYTES).  Longer
// contiguous host runs are cut so their pieces spread over the direction's
// engines: one engine alone moves a 512 MiB host-to-device run at 50.7 GB/s
// against 56-57 GB/s for copies of a few MiB round robin over four (MI355X).
int64_t max_copy_bytes() {
  const char* e = getenv("FLEXKV_SDMA_MAX_COPY_BYTES");
  const int64_t v = e ? atoll(e) : kDefaultMaxCopyBytes;
  return v >= 4096 ? v : kDefaultMaxCopyBytes;
}
}  // namespace

bool layer_major_pays_off(const Geometry& g, int64_t min_run_bytes) {
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) &&
                          (g.num_layers == 1 || g.cls == g.kv * g.chunk);
  if (row_contig || g.cbs != g.chunk || g.num_blocks < 2) return false;
  int64_t runs = 1;
  for (int i = 1; i < g.num_blocks; ++i) runs += g.cids[i] != g.cids[i - 1] + 1;
  return static_cast<int64_t>(g.num_blocks) * g.chunk >= runs * min_run_bytes;
}

void build_runs(const Geometry& g, int b0, int nb, int l0, int nl, bool rect, bool layer_major,
                std::vector<Run>& runs) {
  runs.clear();
  const int64_t cap = max_copy_bytes();
  const int64_t row_chunks = static_cast<int64_t>(nl) * g.kv;
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) && (nl == 1 || g.cls == g.kv * g.chunk);
  const int64_t pitch = rect ? host_slice_pitch(g, nl) : 0;
  char* host0 = g.cpu_ptr + g.startoff + static_cast<int64_t>(g.start_layer + l0) * g.cls;
  if (layer_major) {
    int64_t soff = 0;
    for (int l = 0; l < nl; ++l)
      for (int k = 0; k < g.kv; ++k)
        for (int i = b0; i < b0 + nb; ++i, soff += g.chunk) {
          char* h = host0 + l * g.cls + k * g.cks + g.cids[i] * g.cbs;
          if (i > b0 && runs.back().host + runs.back().bytes == h &&
              runs.back().bytes + g.chunk <= cap) {
            runs.back().bytes += g.chunk;   // staging is contiguous along i
          } else {
            runs.push_back({soff, h, g.chunk});
          }
        }
    return;
  }
  if (pitch > 0) {
    for (int i = b0; i < b0 + nb; ++i) {
      Run r{static_cast<int64_t>(i - b0) * row_chunks * g.chunk, host0 + g.cids[i] * g.cbs,
            g.chunk};
      r.slices = static_cast<int32_t>(row_chunks);
      r.host_pitch = pitch;
      runs.push_back(r);
    }
    return;
  }
  int64_t soff = 0;
  auto push = [&](char* h, int64_t bytes) {
    if (!runs.empty() && runs.back().host + runs.back().bytes == h &&
        runs.back().staging_off + runs.back().bytes == soff &&
        runs.back().bytes + bytes <= cap) {
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

int ensure_sdma(DeviceState& d, int dev, const void* hip_ptr) {
  std::lock_guard<std::mutex> lk(d.sdma_mu);
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
  // Each direction takes `want` engines, from engines 0-7 first, so with the
  // default four both directions' one-way sets are engines 0-3, the fast
  // ones (kDefaultSdmaEngines).  While both directions have transfers in
  // flight they take the duplex split.
  if (sdma_engines_wanted(0) == 0 || sdma_engines_wanted(1) == 0)
    return fail(kInval, "copy engines turned off (FLEXKV_SDMA_ENGINES=0)");
  for (int dir = 0; dir < 2; ++dir) {
    const int want = sdma_engines_wanted(dir);
    uint32_t mask = 0;
    FKV_HSA(dir == 0 ? g_hsa.copy_engine_status(q.cpu, q.gpu, &mask)
                     : g_hsa.copy_engine_status(q.gpu, q.cpu, &mask));
    d.engines[dir].clear();
    const uint32_t tiers[2] = {mask & kComputeFriendlyEngines, mask & ~kComputeFriendlyEngines};
    for (uint32_t tier : tiers)
      for (int b = 0; b < 32 && static_cast<int>(d.engines[dir].size()) < want; ++b)
        if (tier & (1u << b)) d.engines[dir].push_back(static_cast<hsa_amd_sdma_engine_id_t>(1u << b));
    if (d.engines[dir].empty())
      return fail(kInval, "device %d reports no SDMA engine for %s copies", dev,
                  dir == 0 ? "device-to-host" : "host-to-device");
  }
  {
    // the wide set, in order of preference: engines 0-7, then (only when
    // more are asked for) the others
    const char* e = getenv("FLEXKV_SDMA_ENGINES_WIDE");
    if (!e) e = getenv("FLEXKV_SDMA_ENGINES_LAYERWISE");   // the earlier name
    const int wide = std::max(1, std::min(e ? atoi(e) : kDefaultWideEngines, 32));
    uint32_t mask = 0;
    FKV_HSA(g_hsa.copy_engine_status(q.gpu, q.cpu, &mask));
    d.engines_wide.clear();
    const uint32_t tiers[2] = {mask & kComputeFriendlyEngines, mask & ~kComputeFriendlyEngines};
    for (uint32_t tier : tiers)
      for (int b = 0; b < 32 && static_cast<int>(d.engines_wide.size()) < wide; ++b)
        if (tier & (1u << b))
          d.engines_wide.push_back(static_cast<hsa_amd_sdma_engine_id_t>(1u << b));
    if (d.engines_wide.empty()) d.engines_wide = d.engines[1];
    const char* es = getenv("FLEXKV_SDMA_ENGINES_WIDE_SYNC");
    const size_t sync = static_cast<size_t>(std::max(1, es ? atoi(es) : kSyncWideEngines));
    d.engines_wide_sync.assign(d.engines_wide.begin(),
                               d.engines_wide.begin() +
                                   static_cast<std::ptrdiff_t>(std::min(sync, d.engines_wide.size())));
  }
  {
    // the duplex split of engines 0-7: device-to-host takes the first
    // FLEXKV_SDMA_DUPLEX_D2H engines both directions report, host-to-device
    // the others
    const char* e = getenv("FLEXKV_SDMA_DUPLEX_D2H");
    const int nd = std::max(0, std::min(e ? atoi(e) : kDefaultDuplexD2HEngines, 8));
    uint32_t m0 = 0, m1 = 0;
    FKV_HSA(g_hsa.copy_engine_status(q.cpu, q.gpu, &m0));
    FKV_HSA(g_hsa.copy_engine_status(q.gpu, q.cpu, &m1));
    const uint32_t both = m0 & m1 & kComputeFriendlyEngines;
    d.engines_duplex[0].clear();
    d.engines_duplex[1].clear();
    for (int b = 0; b < 32; ++b)
      if (both & (1u << b)) {
        const int dir = static_cast<int>(d.engines_duplex[0].size()) < nd ? 0 : 1;
        d.engines_duplex[dir].push_back(static_cast<hsa_amd_sdma_engine_id_t>(1u << b));
      }
    if (nd == 0 || d.engines_duplex[0].empty() || d.engines_duplex[1].empty()) {
      d.engines_duplex[0].clear();
      d.engines_duplex[1].clear();
    }
  }
  d.gpu_agent = q.gpu;
  d.cpu_agent = q.cpu;
  d.sdma_init = true;
  return 0;
}

int ensure_staging(CopyLane& d, size_t need_half) {
  if (d.stalled) return fail(kInval, "the copy engines of this lane stalled earlier");
  for (int h = 0; h < 2; ++h)
    if (!d.ev_compute[h]) FKV_HIP(hipEventCreateWithFlags(&d.ev_compute[h], hipEventDisableTiming));
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

int issue_sdma(DeviceState& d, CopyLane& lane, const std::vector<Run>& runs, char* staging,
               bool h2d, int half, hsa_agent_t host_agent, int wide, SdmaHold* hold,
               bool held_part) {
  // While the other direction has a copy-engine transfer in flight, the
  // directions split engines 0-7 (the duplex sets); otherwise each takes its
  // one-way set, or host-to-device the wide set where asked.
  const int dir = h2d ? 1 : 0;
  const bool duplex = !d.engines_duplex[dir].empty() &&
                      d.busy[1 - dir].load(std::memory_order_relaxed) > 0;
  const std::vector<hsa_amd_sdma_engine_id_t>& set =
      duplex ? d.engines_duplex[dir]
             : (wide == kEnginesWide && h2d && !d.engines_wide.empty()) ? d.engines_wide
             : (wide == kEnginesWideSync && h2d && !d.engines_wide_sync.empty())
                 ? d.engines_wide_sync
                 : d.engines[dir];
  // The engines of this call: the whole set; its first kHoldKeepEngines when
  // the held engines' share is deferred; the rest for a deferred share.
  size_t e0 = 0, e1 = set.size();
  size_t n = runs.size();
  const bool linear = n > 0 && runs[0].slices == 0;
  if (hold) hold->deferred.clear();
  if (held_part) {
    if (set.size() > kHoldKeepEngines) e0 = kHoldKeepEngines;
  } else if (hold && hold->held_fraction > 0 && linear && set.size() > kHoldKeepEngines) {
    // Held engines start held_fraction f of the half's time late.  Kept
    // engines run faster while they are alone on the link: each moves about
    // rho = (set / kept) * 0.93 times a held engine's rate then (MI355X,
    // 640 KiB host-to-device copies: 52.7 GB/s on four engines, 56.6 on six).
    // For all to end together a held engine takes 1 / (1 + rho f / (1 - f))
    // of a kept engine's copies.
    const double f = std::min(0.5, hold->held_fraction);
    const double kept = static_cast<double>(kHoldKeepEngines);
    const double held = static_cast<double>(set.size() - kHoldKeepEngines);
    const double rho = static_cast<double>(set.size()) / kept * 0.93;
    const double b = 1.0 / (1.0 + rho * f / (1.0 - f));
    size_t nd = static_cast<size_t>(static_cast<double>(n) * held * b / (kept + held * b) + 0.5);
    nd = std::min(nd, n > kHoldKeepEngines ? n - kHoldKeepEngines : size_t(0));
    if (nd > 0) {
      hold->deferred.assign(runs.end() - static_cast<std::ptrdiff_t>(nd), runs.end());
      n -= nd;
      e1 = kHoldKeepEngines;
    }
  }
  const size_t ne = e1 - e0;
  // The engine of each copy (rect copies: the runtime's one engine, key ne)
  // and whether it is that engine's last copy of this call.
  std::vector<uint8_t> last(n, 0);
  uint64_t seen = 0;   // bit per engine key (at most 33)
  size_t tails = 0;
  for (size_t i = n; i-- > 0;) {
    const size_t key = runs[i].slices > 0 ? ne : i % ne;
    if (!(seen >> key & 1)) {
      seen |= uint64_t(1) << key;
      last[i] = 1;
      ++tails;
    }
  }
  // A deferred share follows the copies already queued on the half, with
  // signals of its own from the pools.
  if (!held_part) {
    lane.queued[half].clear();
    lane.wake[half].clear();
    lane.used_polled[half] = 0;
    lane.used_irq[half] = 0;
  }
  std::vector<hsa_signal_t>& polled = lane.polled_pool[half];
  std::vector<hsa_signal_t>& irq = lane.irq_pool[half];
  size_t np = lane.used_polled[half], ni = lane.used_irq[half];
  while (polled.size() < np + (n - tails)) {
    hsa_signal_t sg;
    FKV_HSA(g_hsa.amd_signal_create(1, 0, nullptr, HSA_AMD_SIGNAL_AMD_GPU_ONLY, &sg));
    polled.push_back(sg);
  }
  while (irq.size() < ni + tails) {
    hsa_signal_t sg;
    FKV_HSA(g_hsa.signal_create(1, 0, nullptr, &sg));
    irq.push_back(sg);
  }
  for (size_t i = 0; i < n; ++i) {
    const Run& r = runs[i];
    char* dev_p = staging + r.staging_off;
    const hsa_signal_t sig = last[i] ? irq[ni++] : polled[np++];
    g_hsa.signal_store_screlease(sig, 1);
    hsa_status_t st;
    if (r.slices > 0) {
      // the runtime puts rect copies on the device's own engine for the direction
      hsa_pitched_ptr_t hp{r.host, static_cast<size_t>(r.bytes), static_cast<size_t>(r.host_pitch)};
      hsa_pitched_ptr_t sp{dev_p, static_cast<size_t>(r.bytes), static_cast<size_t>(r.bytes)};
      const hsa_dim3_t zero{0, 0, 0};
      const hsa_dim3_t range{static_cast<uint32_t>(r.bytes), 1, static_cast<uint32_t>(r.slices)};
      st = h2d ? g_hsa.async_copy_rect(&sp, &zero, &hp, &zero, &range, d.gpu_agent,
                                       hsaHostToDevice, 0, nullptr, sig)
               : g_hsa.async_copy_rect(&hp, &zero, &sp, &zero, &range, d.gpu_agent,
                                       hsaDeviceToHost, 0, nullptr, sig);
    } else {
      const hsa_amd_sdma_engine_id_t e = set[e0 + i % ne];
      st = h2d ? g_hsa.async_copy_on_engine(dev_p, d.gpu_agent, r.host, host_agent,
                                            static_cast<size_t>(r.bytes), 0, nullptr, sig, e,
                                            false)
               : g_hsa.async_copy_on_engine(r.host, host_agent, dev_p, d.gpu_agent,
                                            static_cast<size_t>(r.bytes), 0, nullptr, sig, e,
                                            false);
    }
    if (st != HSA_STATUS_SUCCESS) {
      const char* m = nullptr;
      (void)g_hsa.status_string(st, &m);
      lane.used_polled[half] = np;
      lane.used_irq[half] = ni;
      return fail(static_cast<int>(hipErrorUnknown), "SDMA %s of %lld bytes x %d failed: %s",
                  r.slices > 0 ? "rect copy" : "copy", static_cast<long long>(r.bytes),
                  std::max(1, static_cast<int>(r.slices)), m ? m : "?");
    }
    lane.queued[half].push_back(sig);
    if (last[i]) lane.wake[half].push_back(sig);
  }
  lane.used_polled[half] = np;
  lane.used_irq[half] = ni;
  return 0;
}

int sdma_prepare_lane(DeviceState& d, CopyLane& lane, bool h2d, size_t copies_per_half,
                      char* host, size_t host_bytes) {
  for (int h = 0; h < 2; ++h) {
    while (lane.polled_pool[h].size() < copies_per_half) {
      hsa_signal_t sg;
      FKV_HSA(g_hsa.amd_signal_create(1, 0, nullptr, HSA_AMD_SIGNAL_AMD_GPU_ONLY, &sg));
      lane.polled_pool[h].push_back(sg);
    }
  }
  // every engine the direction may take: its one-way set, its side of the
  // duplex split and, host-to-device, the wide set
  const int dir = h2d ? 1 : 0;
  std::vector<hsa_amd_sdma_engine_id_t> eng = d.engines[dir];
  auto add = [&](const std::vector<hsa_amd_sdma_engine_id_t>& v) {
    for (hsa_amd_sdma_engine_id_t e : v)
      if (std::find(eng.begin(), eng.end(), e) == eng.end()) eng.push_back(e);
  };
  add(d.engines_duplex[dir]);
  if (h2d) add(d.engines_wide);
  const size_t bytes = 4096;
  if (eng.size() * bytes > host_bytes || eng.size() * bytes > lane.staging_bytes)
    return fail(kInval, "internal: %zu warm-up copies do not fit their buffers", eng.size());
  std::vector<hsa_signal_t>& irq = lane.irq_pool[0];
  while (irq.size() < eng.size()) {
    hsa_signal_t sg;
    FKV_HSA(g_hsa.signal_create(1, 0, nullptr, &sg));
    irq.push_back(sg);
  }
  lane.queued[0].clear();
  lane.wake[0].clear();
  for (size_t i = 0; i < eng.size(); ++i) {
    const hsa_signal_t sig = irq[i];
    g_hsa.signal_store_screlease(sig, 1);
    char* dev_p = lane.staging + i * bytes;
    char* host_p = host + i * bytes;
    const hsa_status_t st =
        h2d ? g_hsa.async_copy_on_engine(dev_p, d.gpu_agent, host_p, d.cpu_agent, bytes, 0,
                                         nullptr, sig, eng[i], false)
            : g_hsa.async_copy_on_engine(host_p, d.cpu_agent, dev_p, d.gpu_agent, bytes, 0,
                                         nullptr, sig, eng[i], false);
    if (st != HSA_STATUS_SUCCESS) {
      const char* m = nullptr;
      (void)g_hsa.status_string(st, &m);
      // copies queued so far are waited for below, so nothing is left in flight
      const int w = sdma_wait(d, lane, 0, false);
      (void)w;
      return fail(static_cast<int>(hipErrorUnknown), "warm-up copy on an SDMA engine failed: %s",
                  m ? m : "?");
    }
    lane.queued[0].push_back(sig);
    lane.wake[0].push_back(sig);
  }
  return sdma_wait(d, lane, 0, false);
}

bool sdma_rect_available() { return g_hsa.async_copy_rect != nullptr; }

}  // namespace fkv_detail

using namespace fkv_detail;

extern "C" int fkv_abandoned_copies_pending(int device) {
  last_error().clear();
  int dev = device;
  if (dev < 0 && hipGetDevice(&dev) != hipSuccess) return fail(-1, "no current device");
  if (dev >= kMaxDevices) return fail(-1, "device %d out of range", dev);
  int pending = 0;
  for (CopyLane& ln : g_dev[dev].lane) {
    std::lock_guard<std::mutex> lk(ln.mu);
    if (ln.abandoned.empty() || !g_hsa_loaded) continue;
    for (hsa_signal_t s : ln.abandoned)
      if (g_hsa.signal_load_scacquire(s) >= 1) ++pending;
  }
  return pending;
}
