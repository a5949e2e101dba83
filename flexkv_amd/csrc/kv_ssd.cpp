// kv_ssd.cpp - host cache <-> SSD files for KV blocks (host code only).
//
// File layout and block mapping follow the reference SSD tier
// (csrc/transfer_ssd.cpp:17-285, flexkv/storage/allocator.py:132-193,
// flexkv/transfer/worker.py:482-602):
//   * SSD block b lives on device d = (b / rr) % D at device block
//     ((b / rr) / D) * rr + b % rr  (rr = round-robin width);
//   * a device block x lives in file x % F of that device, at in-file block
//     x / F;
//   * chunk (layer l, K|V k) of a block is at
//       file:  x_in_file * block_stride + l * ssd_layer_stride + k * ssd_kv_stride
//       host:  cpu_id    * block_stride + l * cpu_layer_stride + k * cpu_kv_stride
//     and is chunk_size bytes;
//   * each device's blocks are split into contiguous ranges over
//     num_threads_per_device threads.
// Reads use O_DIRECT descriptors when chunk_size is a multiple of 4096
// (transfer_ssd.cpp:201), like the reference.  Unlike the reference's one
// request per chunk, chunks adjacent in both the file and the host cache are
// merged into one request: a block's layer window in block-wise layouts, and
// runs of consecutive blocks in either layout.

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "flexkv_hip.h"
#include "fkv_error.h"

namespace {

int ssd_fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  fkv_detail::last_error() = buf;
  return 1;
}

// Full-length pread/pwrite, retrying short transfers and EINTR.  Returns 0,
// the errno of the failed call, or -1 when a read hits the end of the file.
int io_all(int fd, char* buf, int64_t bytes, int64_t off, bool is_read) {
  while (bytes > 0) {
    const ssize_t r = is_read ? pread(fd, buf, static_cast<size_t>(bytes), off)
                              : pwrite(fd, buf, static_cast<size_t>(bytes), off);
    if (r < 0) {
      if (errno == EINTR) continue;
      return errno ? errno : EIO;
    }
    if (r == 0) return -1;
    buf += r;
    off += r;
    bytes -= r;
  }
  return 0;
}

}  // namespace

struct fkv_ssd_s {
  int num_devices = 0;
  int files_per_device = 0;
  std::vector<std::vector<int>> fd_buffered;  // [device][file]
  std::vector<std::vector<int>> fd_direct;    // [device][file], -1 if unavailable
};

extern "C" {

int fkv_ssd_open(const char* const* paths, int num_devices, int files_per_device,
                 fkv_ssd_t* out) try {
  fkv_detail::last_error().clear();
  if (!out || !paths || num_devices <= 0 || files_per_device <= 0)
    return ssd_fail("bad arguments to fkv_ssd_open");
  *out = nullptr;
  auto* h = new fkv_ssd_s();
  h->num_devices = num_devices;
  h->files_per_device = files_per_device;
  h->fd_buffered.assign(num_devices, std::vector<int>(files_per_device, -1));
  h->fd_direct.assign(num_devices, std::vector<int>(files_per_device, -1));
  for (int d = 0; d < num_devices; ++d) {
    for (int f = 0; f < files_per_device; ++f) {
      const char* p = paths[d * files_per_device + f];
      const int fd = open(p, O_RDWR);
      if (fd < 0) {
        const int e = errno;
        fkv_ssd_close(h);
        return ssd_fail("open(%s) failed: %s", p, strerror(e));
      }
      posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
      h->fd_buffered[d][f] = fd;
      h->fd_direct[d][f] = open(p, O_RDWR | O_DIRECT);  // may fail (e.g. tmpfs): fall back
    }
  }
  *out = h;
  return 0;
} catch (const std::exception& e) {
  return ssd_fail("fkv_ssd_open: %s", e.what());
}

int fkv_ssd_close(fkv_ssd_t h) {
  if (!h) return 0;
  for (auto* v : {&h->fd_buffered, &h->fd_direct})
    for (auto& row : *v)
      for (int fd : row)
        if (fd >= 0) close(fd);
  delete h;
  return 0;
}

int fkv_transfer_kv_blocks_ssd(fkv_ssd_t h, int start_layer, int num_layers, void* cpu_ptr,
                               const int64_t* ssd_block_ids, const int64_t* cpu_block_ids,
                               int num_blocks, int64_t cpu_layer_stride_bytes,
                               int64_t cpu_kv_stride_bytes, int64_t ssd_layer_stride_bytes,
                               int64_t ssd_kv_stride_bytes, int64_t chunk_size_bytes,
                               int64_t block_stride_bytes, int is_read, int round_robin,
                               int num_threads_per_device, int is_mla) try {
  fkv_detail::last_error().clear();
  if (!h) return ssd_fail("null SSD context");
  if (num_blocks <= 0 || num_layers <= 0) return 0;
  if (!cpu_ptr || !ssd_block_ids || !cpu_block_ids || chunk_size_bytes <= 0 || round_robin <= 0 ||
      start_layer < 0 || num_threads_per_device <= 0)
    return ssd_fail("bad arguments to fkv_transfer_kv_blocks_ssd");
  const int D = h->num_devices, F = h->files_per_device, kv = is_mla ? 1 : 2;
  // partition by device, keeping the id-list order within a device
  std::vector<std::vector<int64_t>> dev_ssd(D), dev_cpu(D);
  for (int i = 0; i < num_blocks; ++i) {
    const int64_t b = ssd_block_ids[i], c = cpu_block_ids[i];
    if (b < 0 || c < 0) return ssd_fail("negative block id at position %d", i);
    const int64_t q = b / round_robin;
    const int d = static_cast<int>(q % D);
    dev_ssd[d].push_back((q / D) * round_robin + b % round_robin);
    dev_cpu[d].push_back(c);
  }
  const bool direct = is_read && chunk_size_bytes % 4096 == 0;
  // Chunks are visited in the order that makes neighbours adjacent in both
  // the file and the host cache: block by block when a block's layer window
  // is contiguous on both sides (block-wise layouts, MLA), else layer by
  // layer and K|V by K|V over the blocks (layer-wise layouts).  Adjacent
  // chunks of one file merge into one request.
  const bool block_major = (kv == 1 || (cpu_kv_stride_bytes == chunk_size_bytes &&
                                        ssd_kv_stride_bytes == chunk_size_bytes)) &&
                           (num_layers == 1 || (cpu_layer_stride_bytes == kv * chunk_size_bytes &&
                                                ssd_layer_stride_bytes == kv * chunk_size_bytes));
  std::atomic<int> failed{0};
  std::string first_err;
  std::atomic<bool> have_err{false};
  auto record = [&](const char* what, int d, int64_t blk, int err) {
    failed = 1;
    bool expect = false;
    if (have_err.compare_exchange_strong(expect, true)) {
      char buf[256];
      snprintf(buf, sizeof(buf), "%s failed on device %d block %lld: %s", what, d,
               static_cast<long long>(blk), err > 0 ? strerror(err) : "unexpected end of file");
      first_err = buf;
    }
  };
  auto work = [&](int d, size_t lo, size_t hi) {
    char* base = static_cast<char*>(cpu_ptr);
    // the request being built: `bytes` at host `buf`, file `file` offset `off`
    struct Pending {
      int file = -1;
      char* buf = nullptr;
      int64_t off = 0, bytes = 0, first_block = 0;
    } p;
    auto flush = [&]() {
      if (p.bytes == 0 || failed) return;
      const int fd = h->fd_buffered[d][p.file];
      const int dfd = direct ? h->fd_direct[d][p.file] : -1;
      int err = -2;
      // O_DIRECT needs an aligned buffer, size and offset; else the page cache
      if (dfd >= 0 && reinterpret_cast<uintptr_t>(p.buf) % 4096 == 0 && p.bytes % 4096 == 0 &&
          p.off % 4096 == 0)
        err = io_all(dfd, p.buf, p.bytes, p.off, true);
      if (err != 0) err = io_all(fd, p.buf, p.bytes, p.off, is_read != 0);
      if (err) record(is_read ? "read" : "write", d, p.first_block, err);
      p.bytes = 0;
    };
    auto add = [&](int64_t x, char* buf, int64_t off, int64_t bytes) {
      const int f = static_cast<int>(x % F);
      if (p.bytes > 0 && f == p.file && buf == p.buf + p.bytes && off == p.off + p.bytes) {
        p.bytes += bytes;
        return;
      }
      flush();
      p.file = f;
      p.buf = buf;
      p.off = off;
      p.bytes = bytes;
      p.first_block = x;
    };
    auto host_chunk = [&](size_t j, int l, int k) {
      return base + dev_cpu[d][j] * block_stride_bytes +
             static_cast<int64_t>(l) * cpu_layer_stride_bytes + k * cpu_kv_stride_bytes;
    };
    auto file_chunk = [&](size_t j, int l, int k) {
      return (dev_ssd[d][j] / F) * block_stride_bytes +
             static_cast<int64_t>(l) * ssd_layer_stride_bytes + k * ssd_kv_stride_bytes;
    };
    if (block_major) {
      const int64_t row = static_cast<int64_t>(num_layers) * kv * chunk_size_bytes;
      for (size_t j = lo; j < hi && !failed; ++j)
        add(dev_ssd[d][j], host_chunk(j, start_layer, 0), file_chunk(j, start_layer, 0), row);
    } else {
      for (int l = start_layer; l < start_layer + num_layers && !failed; ++l)
        for (int k = 0; k < kv && !failed; ++k)
          for (size_t j = lo; j < hi && !failed; ++j)
            add(dev_ssd[d][j], host_chunk(j, l, k), file_chunk(j, l, k), chunk_size_bytes);
    }
    flush();
  };
  std::vector<std::thread> threads;
  threads.reserve(static_cast<size_t>(D) * num_threads_per_device);
  for (int d = 0; d < D && !failed; ++d) {
    const size_t n = dev_ssd[d].size();
    if (n == 0) continue;
    const size_t per = (n + num_threads_per_device - 1) / num_threads_per_device;
    for (size_t lo = 0; lo < n && !failed; lo += per) {
      try {
        threads.emplace_back(work, d, lo, std::min(n, lo + per));
      } catch (const std::exception&) {
        work(d, lo, std::min(n, lo + per));  // no thread available: do this range here
      }
    }
  }
  for (auto& t : threads) t.join();
  if (failed) return ssd_fail("%s", first_err.c_str());
  return 0;
} catch (const std::exception& e) {
  return ssd_fail("fkv_transfer_kv_blocks_ssd: %s", e.what());
}

}  // extern "C"
