// Tensor-parallel transfer groups: the ranks of one data-parallel group move
// their own head slices of the same blocks at once, each into (or out of)
// its own byte range of the shared host chunk.  Replaces
// flexkv::TPTransferThreadGroup (csrc/tp_transfer_thread_group.cpp:23-109).
//
// Each rank has one host thread and one stream on its device, made when the
// group is created and kept for the group's life; a transfer hands the job to
// every rank thread, each makes its own synchronous fkv_transfer_kv_blocks
// call, and the transfer returns when all of them have (the reference starts
// and joins a thread per rank on every transfer).  Ranks may share a device:
// their calls then run side by side on separate streams.
#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "flexkv_hip.h"
#include "kv_internal.h"

using namespace fkv_detail;

namespace {

constexpr int kMaxRanks = 64;

struct TpJob {
  int num_blocks = 0;
  const int64_t* gpu_ids = nullptr;
  const int64_t* cpu_ids = nullptr;
  int64_t gpu_kv_stride = 0, gpu_block_stride = 0, gpu_chunk = 0;
  int64_t cpu_kv_stride = 0, cpu_layer_stride = 0, cpu_block_stride = 0;
  int transfer_cus = -1, h2d = 0, use_ce = 0, layer_id = 0, layer_granularity = 0, is_mla = 0;
};

}  // namespace

struct fkv_tp_group_s {
  int num_ranks = 0;
  int num_layers = 0;
  std::vector<int> devices;
  std::vector<void*> layer_ptrs;   // [rank][layer]
  void* cpu_ptr = nullptr;
  std::vector<hipStream_t> streams;
  std::vector<std::thread> threads;
  std::mutex call_mu;   // one transfer of the group at a time
  std::mutex mu;        // guards everything below
  std::condition_variable go, done;
  uint64_t generation = 0;
  int pending = 0;
  bool stop = false;
  TpJob job;
  std::vector<int> rc;
  std::vector<std::string> msg;
  std::vector<std::vector<int64_t>> unsafe;
};

namespace {

std::mutex g_groups_mu;
std::vector<fkv_tp_group_s*> g_groups;   // live groups, for fkv_finalize

// One rank's share of a transfer: its layer window of its own pointer table,
// its own offset inside each host chunk.  Under MLA every rank holds the same
// latent, so device-to-host is moved by rank 0 alone (the reference has every
// rank write the same bytes to offset 0, csrc/tp_transfer_thread_group.cpp:79-80)
// and host-to-device by every rank.
int rank_transfer(fkv_tp_group_s* g, int r, const TpJob& j) {
  if (j.is_mla && !j.h2d && r != 0) return 0;
  // rank r's table starts at r * num_layers (the reference offsets it by
  // r * layer_granularity, csrc/tp_transfer_thread_group.cpp:70,76-77, which
  // addresses another rank's layers when the window is not all layers)
  void* const* ptrs = g->layer_ptrs.data() + static_cast<size_t>(r) * g->num_layers + j.layer_id;
  const int64_t startoff = j.is_mla ? 0 : static_cast<int64_t>(r) * j.gpu_chunk;
  return fkv_transfer_kv_blocks(j.num_blocks, j.layer_id, j.layer_granularity, j.gpu_ids, ptrs,
                                j.gpu_kv_stride, j.gpu_block_stride, j.cpu_ids, g->cpu_ptr,
                                j.cpu_kv_stride, j.cpu_layer_stride, j.cpu_block_stride,
                                startoff, j.gpu_chunk, g->streams[r], j.transfer_cus, j.h2d,
                                j.use_ce, j.is_mla);
}

void rank_loop(fkv_tp_group_s* g, int r) {
  const hipError_t se = hipSetDevice(g->devices[r]);
  uint64_t seen = 0;
  for (;;) {
    TpJob job;
    {
      std::unique_lock<std::mutex> lk(g->mu);
      g->go.wait(lk, [&] { return g->stop || g->generation != seen; });
      if (g->stop) return;
      seen = g->generation;
      job = g->job;
    }
    int rc = 0;
    std::string msg;
    std::vector<int64_t> unsafe;
    if (se != hipSuccess) {
      rc = static_cast<int>(se);
      msg = std::string("hipSetDevice failed: ") + hipGetErrorString(se);
    } else {
      try {
        rc = rank_transfer(g, r, job);
        if (rc) {
          msg = last_error();
          unsafe = last_unsafe_host_blocks();
        }
      } catch (const std::exception& e) {   // nothing may end the rank thread
        rc = static_cast<int>(hipErrorUnknown);
        msg = std::string("exception: ") + e.what();
      }
    }
    std::lock_guard<std::mutex> lk(g->mu);
    g->rc[r] = rc;
    g->msg[r] = std::move(msg);
    g->unsafe[r] = std::move(unsafe);
    if (--g->pending == 0) g->done.notify_all();
  }
}

// Stops and joins the rank threads, destroys the streams (each synchronised
// first) and frees the group.  No transfer of the group may be running.
int group_destroy(fkv_tp_group_s* g) {
  {
    std::lock_guard<std::mutex> lk(g->mu);
    g->stop = true;
  }
  g->go.notify_all();
  for (std::thread& t : g->threads)
    if (t.joinable()) t.join();
  int rc = 0;
  for (size_t r = 0; r < g->streams.size(); ++r) {
    if (!g->streams[r]) continue;
    DeviceGuard guard;
    int e = guard.set(g->devices[r]);
    if (!e) {
      hipError_t s = hipStreamSynchronize(g->streams[r]);
      if (s == hipSuccess) s = hipStreamDestroy(g->streams[r]);
      if (s != hipSuccess)
        e = fail(static_cast<int>(s), "destroying the stream of TP rank %zu: %s", r,
                 hipGetErrorString(s));
    }
    if (e && !rc) rc = e;
  }
  delete g;
  return rc;
}

}  // namespace

namespace fkv_detail {
// fkv_finalize: groups the caller never destroyed
int tp_groups_destroy_all() {
  std::vector<fkv_tp_group_s*> groups;
  {
    std::lock_guard<std::mutex> lk(g_groups_mu);
    groups.swap(g_groups);
  }
  int rc = 0;
  for (fkv_tp_group_s* g : groups) {
    { std::lock_guard<std::mutex> call(g->call_mu); }   // a running transfer ends first
    const int r = group_destroy(g);
    if (r && !rc) rc = r;
  }
  return rc;
}
}  // namespace fkv_detail

extern "C" {

int fkv_tp_group_create(int num_ranks, const int* devices, void* const* gpu_layer_ptrs,
                        int num_layers, void* cpu_ptr, fkv_tp_group_t* out) try {
  last_error().clear();
  if (!out) return fail(kInval, "fkv_tp_group_create: null output handle");
  *out = nullptr;
  if (num_ranks < 1 || num_ranks > kMaxRanks)
    return fail(kInval, "a TP group has 1 to %d ranks, not %d", kMaxRanks, num_ranks);
  if (!devices || !gpu_layer_ptrs || !cpu_ptr || num_layers < 1)
    return fail(kInval, "fkv_tp_group_create: null devices, layer pointers or host cache, or "
                "no layers");
  int count = 0;
  FKV_HIP(hipGetDeviceCount(&count));
  for (int r = 0; r < num_ranks; ++r) {
    if (devices[r] < 0 || devices[r] >= count || devices[r] >= kMaxDevices)
      return fail(kInval, "TP rank %d: device %d does not exist (%d devices)", r, devices[r],
                  count);
    for (int l = 0; l < num_layers; ++l)
      if (!gpu_layer_ptrs[static_cast<size_t>(r) * num_layers + l])
        return fail(kInval, "TP rank %d: layer pointer %d is null", r, l);
  }
  auto* g = new fkv_tp_group_s();
  g->num_ranks = num_ranks;
  g->num_layers = num_layers;
  g->devices.assign(devices, devices + num_ranks);
  g->layer_ptrs.assign(gpu_layer_ptrs, gpu_layer_ptrs + static_cast<size_t>(num_ranks) * num_layers);
  g->cpu_ptr = cpu_ptr;
  g->streams.assign(num_ranks, nullptr);
  g->rc.assign(num_ranks, 0);
  g->msg.assign(num_ranks, std::string());
  g->unsafe.assign(num_ranks, std::vector<int64_t>());
  for (int r = 0; r < num_ranks; ++r) {
    DeviceGuard guard;
    int e = guard.set(devices[r]);
    if (!e) {
      const hipError_t s = hipStreamCreateWithFlags(&g->streams[r], hipStreamNonBlocking);
      if (s != hipSuccess)
        e = fail(static_cast<int>(s), "TP rank %d: hipStreamCreateWithFlags failed: %s", r,
                 hipGetErrorString(s));
    }
    if (e) {
      const std::string m = last_error();
      (void)group_destroy(g);
      last_error() = m;
      return e;
    }
  }
  try {
    for (int r = 0; r < num_ranks; ++r) g->threads.emplace_back(rank_loop, g, r);
  } catch (const std::exception& ex) {
    (void)group_destroy(g);
    return fail(static_cast<int>(hipErrorUnknown), "starting TP rank threads: %s", ex.what());
  }
  {
    std::lock_guard<std::mutex> lk(g_groups_mu);
    g_groups.push_back(g);
  }
  *out = g;
  return 0;
} catch (const std::exception& e) {
  return fail(static_cast<int>(hipErrorUnknown), "fkv_tp_group_create: %s", e.what());
}

int fkv_tp_group_transfer(fkv_tp_group_t g, int num_blocks, const int64_t* gpu_block_ids,
                          int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                          int64_t gpu_chunk_size_bytes, const int64_t* cpu_block_ids,
                          int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                          int64_t cpu_block_stride_bytes, int transfer_cus,
                          int is_host_to_device, int use_ce_transfer, int layer_id,
                          int layer_granularity, int is_mla) try {
  last_error().clear();
  last_unsafe_host_blocks().clear();
  if (!g) return fail(kInval, "null TP group");
  if (num_blocks < 0) return fail(kInval, "num_blocks %d < 0", num_blocks);
  if (layer_id < 0 || layer_granularity < 1 || layer_id + layer_granularity > g->num_layers)
    return fail(kInval, "layer window [%d, %d) is outside the group's %d layers", layer_id,
                layer_id + layer_granularity, g->num_layers);
  if (num_blocks == 0) return 0;
  if (!gpu_block_ids || !cpu_block_ids) return fail(kInval, "null block ids");
  std::lock_guard<std::mutex> call(g->call_mu);
  {
    std::lock_guard<std::mutex> lk(g->mu);
    TpJob& j = g->job;
    j.num_blocks = num_blocks;
    j.gpu_ids = gpu_block_ids;
    j.cpu_ids = cpu_block_ids;
    j.gpu_kv_stride = gpu_kv_stride_bytes;
    j.gpu_block_stride = gpu_block_stride_bytes;
    j.gpu_chunk = gpu_chunk_size_bytes;
    j.cpu_kv_stride = cpu_kv_stride_bytes;
    j.cpu_layer_stride = cpu_layer_stride_bytes;
    j.cpu_block_stride = cpu_block_stride_bytes;
    j.transfer_cus = transfer_cus;
    j.h2d = is_host_to_device;
    j.use_ce = use_ce_transfer;
    j.layer_id = layer_id;
    j.layer_granularity = layer_granularity;
    j.is_mla = is_mla;
    g->pending = g->num_ranks;
    ++g->generation;
  }
  g->go.notify_all();
  std::unique_lock<std::mutex> lk(g->mu);
  g->done.wait(lk, [&] { return g->pending == 0; });
  int rc = 0;
  std::string msg;
  for (int r = 0; r < g->num_ranks; ++r) {
    if (!g->rc[r]) continue;
    if (!rc) {
      rc = g->rc[r];
      char head[64];
      snprintf(head, sizeof(head), "TP rank %d (device %d): ", r, g->devices[r]);
      msg = head + g->msg[r];
    }
    std::vector<int64_t>& u = last_unsafe_host_blocks();
    u.insert(u.end(), g->unsafe[r].begin(), g->unsafe[r].end());
  }
  if (rc) last_error() = msg;
  return rc;
} catch (const std::exception& e) {
  return fail(static_cast<int>(hipErrorUnknown), "fkv_tp_group_transfer: %s", e.what());
}

int fkv_tp_group_destroy(fkv_tp_group_t g) try {
  last_error().clear();
  if (!g) return 0;
  {
    std::lock_guard<std::mutex> lk(g_groups_mu);
    bool found = false;
    for (size_t i = 0; i < g_groups.size(); ++i)
      if (g_groups[i] == g) {
        g_groups.erase(g_groups.begin() + static_cast<std::ptrdiff_t>(i));
        found = true;
        break;
      }
    if (!found) return fail(kInval, "not a live TP group");
  }
  { std::lock_guard<std::mutex> call(g->call_mu); }   // a running transfer ends first
  return group_destroy(g);
} catch (const std::exception& e) {
  return fail(static_cast<int>(hipErrorUnknown), "fkv_tp_group_destroy: %s", e.what());
}

}  // extern "C"
