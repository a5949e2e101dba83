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
//     and is chunk_size bytes.
// Reads use O_DIRECT descriptors when chunk_size is a multiple of 4096
// (transfer_ssd.cpp:201), like the reference.  The kernel cannot do direct
// I/O into host memory that HIP pinned (hipHostMalloc memory is not
// page-pinnable by get_user_pages: O_DIRECT reads into it fail with EFAULT),
// so direct reads land in page-aligned bounce buffers of ordinary
// memory and are copied into the host cache from there.  Unlike the reference's one
// request per chunk, chunks adjacent in both the file and the host cache are
// merged into one request (up to FLEXKV_SSD_MAX_REQUEST_BYTES, default
// 1 GiB): a block's layer window in block-wise layouts, and runs of
// consecutive blocks in either layout.
//
// Two engines run the requests, as in the reference:
//   * threads (iouring_entries = 0): each device's blocks are split into
//     contiguous ranges over num_threads_per_device threads, each issuing
//     blocking pread/pwrite (transfer_ssd.cpp:241-264);
//   * io_uring (iouring_entries > 0 and the kernel allows a ring): the
//     calling thread queues every request of every device on one ring of that
//     depth and waits for all completions (transfer_ssd.cpp:34-117, 229-272;
//     IOUring at transfer_ssd.h:9-170).  The ring is driven through the raw
//     io_uring_setup / io_uring_enter system calls.  When the ring cannot be
//     created the handle falls back to the threads engine, as the reference
//     does when io_uring_queue_init fails.

#include <fcntl.h>
#include <linux/io_uring.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/syscall.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
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

// One submission ring, set up and driven with the io_uring system calls.
// Not thread-safe: the owning handle serialises its users.
class Uring {
 public:
  ~Uring() { reset(); }

  // 0, or the errno of the failed setup call.
  int init(unsigned entries, unsigned flags) {
    io_uring_params p;
    memset(&p, 0, sizeof(p));
    p.flags = flags;
    const long fd = syscall(__NR_io_uring_setup, entries, &p);
    if (fd < 0) return errno ? errno : EINVAL;
    fd_ = static_cast<int>(fd);
    flags_ = flags;
    sq_len_ = p.sq_off.array + p.sq_entries * sizeof(unsigned);
    cq_len_ = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
    const bool single = (p.features & IORING_FEAT_SINGLE_MMAP) != 0;
    if (single) sq_len_ = cq_len_ = std::max(sq_len_, cq_len_);
    sq_ptr_ = mmap(nullptr, sq_len_, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd_,
                   IORING_OFF_SQ_RING);
    if (sq_ptr_ == MAP_FAILED) return fail_init();
    if (single) {
      cq_ptr_ = sq_ptr_;
    } else {
      cq_ptr_ = mmap(nullptr, cq_len_, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd_,
                     IORING_OFF_CQ_RING);
      if (cq_ptr_ == MAP_FAILED) {
        cq_ptr_ = nullptr;
        return fail_init();
      }
    }
    sqes_len_ = p.sq_entries * sizeof(io_uring_sqe);
    void* sq = mmap(nullptr, sqes_len_, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd_,
                    IORING_OFF_SQES);
    if (sq == MAP_FAILED) return fail_init();
    sqes_ = static_cast<io_uring_sqe*>(sq);
    char* s = static_cast<char*>(sq_ptr_);
    char* c = static_cast<char*>(cq_ptr_);
    sq_head_ = reinterpret_cast<unsigned*>(s + p.sq_off.head);
    sq_tail_ = reinterpret_cast<unsigned*>(s + p.sq_off.tail);
    sq_mask_ = *reinterpret_cast<unsigned*>(s + p.sq_off.ring_mask);
    sq_flags_ = reinterpret_cast<unsigned*>(s + p.sq_off.flags);
    sq_array_ = reinterpret_cast<unsigned*>(s + p.sq_off.array);
    cq_head_ = reinterpret_cast<unsigned*>(c + p.cq_off.head);
    cq_tail_ = reinterpret_cast<unsigned*>(c + p.cq_off.tail);
    cq_mask_ = *reinterpret_cast<unsigned*>(c + p.cq_off.ring_mask);
    cqes_ = reinterpret_cast<io_uring_cqe*>(c + p.cq_off.cqes);
    depth_ = p.sq_entries;
    tail_ = *sq_tail_;
    return 0;
  }

  bool enabled() const { return fd_ >= 0; }
  bool sqpoll() const { return (flags_ & IORING_SETUP_SQPOLL) != 0; }
  unsigned depth() const { return depth_; }

  // A zeroed submission entry, or nullptr when the submission ring is full.
  io_uring_sqe* next_sqe() {
    const unsigned head = __atomic_load_n(sq_head_, __ATOMIC_ACQUIRE);
    if (tail_ - head >= depth_) return nullptr;
    io_uring_sqe* e = &sqes_[tail_ & sq_mask_];
    memset(e, 0, sizeof(*e));
    return e;
  }
  // Publish the entry next_sqe() returned.
  void push() {
    sq_array_[tail_ & sq_mask_] = tail_ & sq_mask_;
    ++tail_;
    __atomic_store_n(sq_tail_, tail_, __ATOMIC_RELEASE);
    ++unsubmitted_;
  }

  // Hand published entries to the kernel and, with wait_nr > 0, block until
  // at least that many completions are available.  0 or an errno.
  int enter(unsigned wait_nr) {
    for (;;) {
      unsigned fl = wait_nr ? IORING_ENTER_GETEVENTS : 0;
      unsigned submit = unsubmitted_;
      if (flags_ & IORING_SETUP_SQPOLL) {
        // the kernel's poll thread consumes the ring; only wake it
        submit = 0;
        unsubmitted_ = 0;
        if (__atomic_load_n(sq_flags_, __ATOMIC_ACQUIRE) & IORING_SQ_NEED_WAKEUP)
          fl |= IORING_ENTER_SQ_WAKEUP;
        if (fl == 0) return 0;
      } else if (submit == 0 && wait_nr == 0) {
        return 0;
      }
      const long r = syscall(__NR_io_uring_enter, fd_, submit, wait_nr, fl, nullptr, 0);
      if (r < 0) {
        if (errno == EINTR) continue;
        return errno ? errno : EIO;
      }
      unsubmitted_ -= std::min<unsigned>(unsubmitted_, static_cast<unsigned>(r));
      if (unsubmitted_ == 0 || wait_nr > 0) return 0;
    }
  }

  // Block until at least wait_nr completions are available, submitting
  // nothing.  0 or an errno.
  int wait_only(unsigned wait_nr) {
    for (;;) {
      const long r = syscall(__NR_io_uring_enter, fd_, 0, wait_nr, IORING_ENTER_GETEVENTS,
                             nullptr, 0);
      if (r >= 0) return 0;
      if (errno != EINTR) return errno ? errno : EIO;
    }
  }

  // Entries published since the last enter() handed them to the kernel.
  unsigned pending() const { return unsubmitted_; }

  // Entries published to the ring that the kernel has not taken yet.
  unsigned unconsumed() const { return tail_ - __atomic_load_n(sq_head_, __ATOMIC_ACQUIRE); }

  // Tear the ring down (entries the kernel never took are dropped).
  void shutdown() { reset(); }

  // Pass every available completion to fn(user_data, res); returns the count.
  template <class Fn>
  unsigned reap(Fn&& fn) {
    if (!enabled()) return 0;
    unsigned head = *cq_head_, n = 0;
    const unsigned tail = __atomic_load_n(cq_tail_, __ATOMIC_ACQUIRE);
    for (; head != tail; ++head, ++n) {
      const io_uring_cqe& c = cqes_[head & cq_mask_];
      fn(c.user_data, c.res);
    }
    __atomic_store_n(cq_head_, head, __ATOMIC_RELEASE);
    return n;
  }

 private:
  int fail_init() {
    const int e = errno ? errno : ENOMEM;
    reset();
    return e;
  }
  void reset() {
    if (sqes_) munmap(sqes_, sqes_len_);
    if (cq_ptr_ && cq_ptr_ != sq_ptr_) munmap(cq_ptr_, cq_len_);
    if (sq_ptr_ && sq_ptr_ != MAP_FAILED) munmap(sq_ptr_, sq_len_);
    if (fd_ >= 0) close(fd_);
    sqes_ = nullptr;
    sq_ptr_ = cq_ptr_ = nullptr;
    sq_head_ = sq_tail_ = sq_flags_ = sq_array_ = nullptr;
    cq_head_ = cq_tail_ = nullptr;
    cqes_ = nullptr;
    sq_mask_ = cq_mask_ = 0;
    fd_ = -1;
    depth_ = 0;
    tail_ = 0;
    unsubmitted_ = 0;
  }

  int fd_ = -1;
  unsigned flags_ = 0;
  void* sq_ptr_ = nullptr;
  void* cq_ptr_ = nullptr;
  size_t sq_len_ = 0, cq_len_ = 0, sqes_len_ = 0;
  io_uring_sqe* sqes_ = nullptr;
  unsigned *sq_head_ = nullptr, *sq_tail_ = nullptr, *sq_flags_ = nullptr, *sq_array_ = nullptr;
  unsigned *cq_head_ = nullptr, *cq_tail_ = nullptr;
  unsigned sq_mask_ = 0, cq_mask_ = 0;
  io_uring_cqe* cqes_ = nullptr;
  unsigned depth_ = 0;
  unsigned tail_ = 0;
  unsigned unsubmitted_ = 0;
};

// One file request: `bytes` at host `buf` <-> file `file` of `device` at `off`.
struct Request {
  int device = 0;
  int file = -1;
  char* buf = nullptr;
  int64_t off = 0, bytes = 0, first_block = 0;
};

// Everything a transfer call fixes: the per-device block lists and geometry.
struct Plan {
  int D = 0, F = 0, kv = 2;
  int start_layer = 0, num_layers = 0;
  char* base = nullptr;
  int64_t cpu_layer_stride = 0, cpu_kv_stride = 0, ssd_layer_stride = 0, ssd_kv_stride = 0;
  int64_t chunk = 0, block_stride = 0, max_request = 0;
  bool is_read = false, direct = false, block_major = false;
  std::vector<std::vector<int64_t>> dev_ssd, dev_cpu;   // [device][i]
};

// Build the merged requests for blocks [lo, hi) of device d, in the order
// that makes neighbours adjacent in both the file and the host cache: block
// by block when a block's layer window is contiguous on both sides
// (block-wise layouts, MLA), else layer by layer and K|V by K|V over the
// blocks (layer-wise layouts).  emit(const Request&) returns false to stop.
template <class Emit>
void for_each_request(const Plan& p, int d, size_t lo, size_t hi, Emit&& emit) {
  Request r;
  r.device = d;
  bool go = true;
  auto flush = [&]() {
    if (r.bytes > 0 && go) go = emit(r);
    r.bytes = 0;
  };
  auto add = [&](int64_t x, char* buf, int64_t off, int64_t bytes) {
    const int f = static_cast<int>(x % p.F);
    if (r.bytes > 0 && f == r.file && buf == r.buf + r.bytes && off == r.off + r.bytes &&
        r.bytes + bytes <= p.max_request) {
      r.bytes += bytes;
      return;
    }
    flush();
    r.file = f;
    r.buf = buf;
    r.off = off;
    r.bytes = bytes;
    r.first_block = x;
  };
  auto host_chunk = [&](size_t j, int l, int k) {
    return p.base + p.dev_cpu[d][j] * p.block_stride + static_cast<int64_t>(l) * p.cpu_layer_stride +
           k * p.cpu_kv_stride;
  };
  auto file_chunk = [&](size_t j, int l, int k) {
    return (p.dev_ssd[d][j] / p.F) * p.block_stride + static_cast<int64_t>(l) * p.ssd_layer_stride +
           k * p.ssd_kv_stride;
  };
  if (p.block_major) {
    const int64_t row = static_cast<int64_t>(p.num_layers) * p.kv * p.chunk;
    for (size_t j = lo; j < hi && go; ++j) {
      // a row longer than one request is issued in max_request pieces
      for (int64_t s = 0; s < row && go; s += p.max_request)
        add(p.dev_ssd[d][j], host_chunk(j, p.start_layer, 0) + s,
            file_chunk(j, p.start_layer, 0) + s, std::min(p.max_request, row - s));
    }
  } else {
    for (int l = p.start_layer; l < p.start_layer + p.num_layers && go; ++l)
      for (int k = 0; k < p.kv && go; ++k)
        for (size_t j = lo; j < hi && go; ++j)
          for (int64_t s = 0; s < p.chunk && go; s += p.max_request)
            add(p.dev_ssd[d][j], host_chunk(j, l, k) + s, file_chunk(j, l, k) + s,
                std::min(p.max_request, p.chunk - s));
  }
  flush();
}

// The first error of a call, kept across threads.
struct ErrorSlot {
  std::atomic<bool> failed{false};
  std::atomic<bool> have{false};
  std::string msg;
  void set(const char* text) {
    failed = true;
    bool expect = false;
    if (have.compare_exchange_strong(expect, true)) msg = text;
  }
  void record(bool is_read, const Request& r, int err) {
    char buf[256];
    snprintf(buf, sizeof(buf), "%s failed on device %d block %lld: %s",
             is_read ? "read" : "write", r.device, static_cast<long long>(r.first_block),
             err > 0 ? strerror(err) : "unexpected end of file");
    set(buf);
  }
  void ring(const char* what, int err) {
    char buf[256];
    snprintf(buf, sizeof(buf), "io_uring_enter (%s) failed: %s", what, strerror(err));
    set(buf);
  }
};

// O_DIRECT needs an aligned size and file offset (the bounce buffers that
// take the data are page aligned).
bool direct_ok(const Request& r) { return r.bytes % 4096 == 0 && r.off % 4096 == 0; }

// Bytes of one O_DIRECT read and of each bounce buffer.
// Measured on MI355X hosts (ext4, 1 GiB of O_DIRECT reads into random
// pinned host blocks, 32 threads): 4 MiB buffers read 4.9-5.3 GB/s, 1 MiB
// buffers 4.5 GB/s on the same boxes.
constexpr int64_t kBounceBytes = int64_t(4) << 20;

// Page-aligned bounce buffers of ordinary memory, kept for the handle's
// lifetime and shared by its calls.
class BouncePool {
 public:
  ~BouncePool() {
    for (char* b : free_) std::free(b);
  }
  char* get() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      if (!free_.empty()) {
        char* b = free_.back();
        free_.pop_back();
        return b;
      }
    }
    return static_cast<char*>(std::aligned_alloc(4096, kBounceBytes));
  }
  void put(char* b) {
    if (!b) return;
    std::lock_guard<std::mutex> lk(mu_);
    free_.push_back(b);
  }

 private:
  std::mutex mu_;
  std::vector<char*> free_;
};

int64_t max_request_bytes() {
  const char* e = getenv("FLEXKV_SSD_MAX_REQUEST_BYTES");
  int64_t v = e ? atoll(e) : (int64_t(1) << 30);
  v = std::max<int64_t>(v, 4096) & ~int64_t(4095);   // whole pages keep O_DIRECT pieces aligned
  return std::min<int64_t>(v, int64_t(1) << 30);     // an io_uring length is 32-bit
}

}  // namespace

struct fkv_ssd_s {
  int num_devices = 0;
  int files_per_device = 0;
  std::vector<std::vector<int>> fd_buffered;  // [device][file]
  std::vector<std::vector<int>> fd_direct;    // [device][file], -1 if unavailable
  std::mutex uring_mu;                        // one caller drives the ring at a time
  Uring uring;
  BouncePool bounce;                          // destinations of O_DIRECT reads (threads)
  // The ring's direct-read bounce memory: `ring_regions` regions of
  // `ring_piece` bytes, allocated on first use and kept (under uring_mu).
  char* ring_bounce = nullptr;
  int64_t ring_piece = 0;
  unsigned ring_regions = 0;
  ~fkv_ssd_s() { std::free(ring_bounce); }
  // cumulative counters (fkv_ssd_stats)
  std::atomic<int64_t> direct_read_bytes{0}, buffered_read_bytes{0}, write_bytes{0};
  std::atomic<int64_t> requests{0}, ring_entries{0}, fallbacks{0};
  void count_io(bool is_read, bool direct, int64_t bytes) {
    if (bytes <= 0) return;
    (is_read ? (direct ? direct_read_bytes : buffered_read_bytes) : write_bytes) += bytes;
  }
};

namespace {

// Blocking pread/pwrite of one request.  Direct reads go through `bounce`
// (kBounceBytes) piece by piece; what O_DIRECT cannot read (an error, a short
// read) is read through the page cache instead.
void run_sync(fkv_ssd_s* h, const Plan& p, const Request& r, char* bounce, ErrorSlot& err) {
  const int fd = h->fd_buffered[r.device][r.file];
  const int dfd = p.direct ? h->fd_direct[r.device][r.file] : -1;
  ++h->requests;
  int64_t done = 0;
  const bool direct = dfd >= 0 && bounce && direct_ok(r);
  if (direct) {
    while (done < r.bytes) {
      const int64_t n = std::min(kBounceBytes, r.bytes - done);
      if (io_all(dfd, bounce, n, r.off + done, true) != 0) break;
      memcpy(r.buf + done, bounce, static_cast<size_t>(n));
      done += n;
    }
    h->count_io(true, true, done);
  }
  if (done == r.bytes) return;
  if (direct) ++h->fallbacks;
  const int e = io_all(fd, r.buf + done, r.bytes - done, r.off + done, p.is_read);
  if (e)
    err.record(p.is_read, r, e);
  else
    h->count_io(p.is_read, false, r.bytes - done);
}

void run_threads(fkv_ssd_s* h, const Plan& p, int threads_per_device, ErrorSlot& err) {
  auto work = [&](int d, size_t lo, size_t hi) {
    char* bounce = p.direct ? h->bounce.get() : nullptr;
    for_each_request(p, d, lo, hi, [&](const Request& r) {
      if (err.failed) return false;
      run_sync(h, p, r, bounce, err);
      return !err.failed;
    });
    h->bounce.put(bounce);
  };
  std::vector<std::thread> threads;
  threads.reserve(static_cast<size_t>(p.D) * threads_per_device);
  for (int d = 0; d < p.D && !err.failed; ++d) {
    const size_t n = p.dev_ssd[d].size();
    if (n == 0) continue;
    const size_t per = (n + threads_per_device - 1) / threads_per_device;
    for (size_t lo = 0; lo < n && !err.failed; lo += per) {
      try {
        threads.emplace_back(work, d, lo, std::min(n, lo + per));
      } catch (const std::exception&) {
        work(d, lo, std::min(n, lo + per));  // no thread available: do this range here
      }
    }
  }
  for (auto& t : threads) t.join();
}

// Bounce memory of a ring: regions of FLEXKV_SSD_RING_PIECE_KIB (default
// 1024, a multiple of 4 KiB), at most one per ring slot and
// FLEXKV_SSD_RING_BOUNCE_MIB (default 256) in all, read when the ring first
// needs them.  The disk wants many bytes in flight: measured on MI355X hosts
// (ext4, 1 GiB of O_DIRECT reads into random pinned host blocks, depth 256),
// 1 MiB pieces with 256 MiB in all read 5.8-6.9 GB/s, 256 KiB pieces with
// 64 MiB in all 2.9-3.5 GB/s on the same boxes.
int64_t ring_piece_bytes() {
  const char* e = getenv("FLEXKV_SSD_RING_PIECE_KIB");
  int64_t v = (e ? atoll(e) : 1024) << 10;
  v = std::max<int64_t>(v, 4096) & ~int64_t(4095);   // O_DIRECT offsets stay page aligned
  return std::min<int64_t>(v, int64_t(1) << 30);      // an io_uring length is 32-bit
}
int64_t ring_bounce_total() {
  const char* e = getenv("FLEXKV_SSD_RING_BOUNCE_MIB");
  return std::max<int64_t>(1, e ? atoll(e) : 256) << 20;
}

// Every request of every device through the handle's ring, at most depth()
// entries in flight.  Direct reads are cut into bounce-region-sized pieces,
// each read into a free region and copied to the host cache when it
// completes.
void run_uring(fkv_ssd_s* h, const Plan& p, ErrorSlot& err) {
  Uring& u = h->uring;
  struct Entry {
    Request r;                 // the piece: host destination or source, file range
    char* bounce = nullptr;    // where a direct read lands, else nullptr
  };
  std::vector<Entry> slots(u.depth());
  std::vector<unsigned> free_slots(u.depth());
  for (unsigned i = 0; i < u.depth(); ++i) free_slots[i] = u.depth() - 1 - i;
  if (p.direct && !h->ring_bounce) {
    const int64_t piece = ring_piece_bytes();
    const unsigned regions = static_cast<unsigned>(
        std::max<int64_t>(1, std::min<int64_t>(u.depth(), ring_bounce_total() / piece)));
    h->ring_bounce = static_cast<char*>(
        std::aligned_alloc(4096, static_cast<size_t>(piece) * regions));
    h->ring_piece = h->ring_bounce ? piece : 0;
    h->ring_regions = h->ring_bounce ? regions : 0;
  }
  const int64_t piece_bytes = h->ring_piece;
  std::vector<char*> free_bounces;
  for (unsigned i = 0; i < h->ring_regions; ++i)
    free_bounces.push_back(h->ring_bounce + static_cast<int64_t>(i) * piece_bytes);
  unsigned in_flight = 0;
  auto complete = [&](uint64_t tag, int res) {
    const Entry s = slots[static_cast<size_t>(tag)];
    free_slots.push_back(static_cast<unsigned>(tag));
    --in_flight;
    ++h->ring_entries;
    int64_t done = 0;
    if (!err.failed && res > 0) {
      done = std::min<int64_t>(res, s.r.bytes);
      if (s.bounce) memcpy(s.r.buf, s.bounce, static_cast<size_t>(done));
      h->count_io(p.is_read, s.bounce != nullptr, done);
    }
    if (s.bounce) free_bounces.push_back(s.bounce);
    if (err.failed || done == s.r.bytes) return;
    if (res == 0 && p.is_read) {
      err.record(true, s.r, -1);
      return;
    }
    // A short transfer is finished, and a failed one (O_DIRECT refused, a
    // ring set up for polled I/O given a page-cache descriptor, ...) redone,
    // with blocking I/O through the page cache; an error there is the
    // request's error.
    ++h->fallbacks;
    const int fd = h->fd_buffered[s.r.device][s.r.file];
    const int e = io_all(fd, s.r.buf + done, s.r.bytes - done, s.r.off + done, p.is_read);
    if (e)
      err.record(p.is_read, s.r, e);
    else
      h->count_io(p.is_read, false, s.r.bytes - done);
  };
  auto wait_one = [&]() -> bool {
    const int e = u.enter(1);
    if (e) {
      err.ring("submit and wait", e);
      return false;
    }
    u.reap(complete);
    return true;
  };
  // Queue one ring entry for `r`, reading into a bounce buffer when `direct`.
  auto submit = [&](const Request& r, bool direct) -> bool {
    io_uring_sqe* e = nullptr;
    auto ready = [&]() {
      return !free_slots.empty() && (!direct || !free_bounces.empty()) &&
             (e = u.next_sqe()) != nullptr;
    };
    while (!ready()) {
      u.reap(complete);
      if (ready()) break;
      if (!wait_one()) return false;
    }
    const unsigned tag = free_slots.back();
    free_slots.pop_back();
    Entry& s = slots[tag];
    s.r = r;
    s.bounce = nullptr;
    if (direct) {
      s.bounce = free_bounces.back();
      free_bounces.pop_back();
    }
    e->opcode = p.is_read ? IORING_OP_READ : IORING_OP_WRITE;
    e->fd = direct ? h->fd_direct[r.device][r.file] : h->fd_buffered[r.device][r.file];
    e->addr = reinterpret_cast<uint64_t>(direct ? s.bounce : r.buf);
    e->len = static_cast<uint32_t>(r.bytes);
    e->off = static_cast<uint64_t>(r.off);
    e->user_data = tag;
    u.push();
    ++in_flight;
    // hand work to the kernel in batches of half the ring
    if (u.pending() >= std::max(1u, u.depth() / 2)) {
      const int ee = u.enter(0);
      if (ee) {
        err.ring("submit", ee);
        return false;
      }
    }
    return true;
  };
  for (int d = 0; d < p.D && !err.failed; ++d) {
    for_each_request(p, d, 0, p.dev_ssd[d].size(), [&](const Request& r) {
      if (err.failed) return false;
      ++h->requests;
      const bool direct =
          p.direct && piece_bytes > 0 && h->fd_direct[r.device][r.file] >= 0 && direct_ok(r);
      if (!direct) return submit(r, false);
      for (int64_t off = 0; off < r.bytes; off += piece_bytes) {
        Request piece = r;
        piece.buf += off;
        piece.off += off;
        piece.bytes = std::min(piece_bytes, r.bytes - off);
        if (!submit(piece, true)) return false;
      }
      return true;
    });
  }
  // Drain: no request the kernel has taken may still target the caller's
  // buffers when the call returns.  If submitting fails, wait only for the
  // requests the kernel took, then tear the ring down so that the entries it
  // never took are dropped (later calls use threads).
  bool broken = false;
  while (in_flight > 0) {
    u.reap(complete);
    if (in_flight == 0) break;
    // entries the kernel never took are dropped with the ring; under SQPOLL
    // the kernel's thread may still take them, so wait for every one
    if (broken && !u.sqpoll() && in_flight == u.unconsumed()) break;
    const int e = broken ? u.wait_only(1) : u.enter(1);
    if (e == 0) continue;
    if (!broken) {
      err.ring("submit and wait", e);
      broken = true;
    } else {
      std::this_thread::sleep_for(std::chrono::milliseconds(1));
    }
  }
  if (broken) {
    fprintf(stderr, "flexkv: io_uring failed (%s); SSD transfers use threads from now on\n",
            err.msg.c_str());
    u.shutdown();
  }
}

}  // namespace

extern "C" {

int fkv_ssd_open(const char* const* paths, int num_devices, int files_per_device,
                 int iouring_entries, int iouring_flags, fkv_ssd_t* out) try {
  fkv_detail::last_error().clear();
  if (!out || !paths || num_devices <= 0 || files_per_device <= 0 || iouring_entries < 0)
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
  if (iouring_entries > 0) {
    const int e = h->uring.init(static_cast<unsigned>(iouring_entries),
                                static_cast<unsigned>(iouring_flags));
    if (e)
      fprintf(stderr, "flexkv: io_uring setup (entries %d, flags %d) failed: %s; "
              "SSD transfers use threads\n", iouring_entries, iouring_flags, strerror(e));
  }
  *out = h;
  return 0;
} catch (const std::exception& e) {
  return ssd_fail("fkv_ssd_open: %s", e.what());
}

int fkv_ssd_iouring_depth(fkv_ssd_t h) {
  if (!h) {
    ssd_fail("null SSD context");
    return -1;
  }
  std::lock_guard<std::mutex> lk(h->uring_mu);
  return h->uring.enabled() ? static_cast<int>(h->uring.depth()) : 0;
}

int fkv_ssd_stats_read(fkv_ssd_t h, fkv_ssd_stats* out) {
  if (!h || !out) return ssd_fail("null SSD context or output");
  out->direct_read_bytes = h->direct_read_bytes.load();
  out->buffered_read_bytes = h->buffered_read_bytes.load();
  out->write_bytes = h->write_bytes.load();
  out->requests = h->requests.load();
  out->ring_entries = h->ring_entries.load();
  out->fallbacks = h->fallbacks.load();
  return 0;
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
  fkv_detail::last_unsafe_host_blocks().clear();
  if (!h) return ssd_fail("null SSD context");
  if (num_blocks <= 0 || num_layers <= 0) return 0;
  if (!cpu_ptr || !ssd_block_ids || !cpu_block_ids || chunk_size_bytes <= 0 || round_robin <= 0 ||
      start_layer < 0 || num_threads_per_device <= 0)
    return ssd_fail("bad arguments to fkv_transfer_kv_blocks_ssd");
  Plan p;
  p.D = h->num_devices;
  p.F = h->files_per_device;
  p.kv = is_mla ? 1 : 2;
  p.start_layer = start_layer;
  p.num_layers = num_layers;
  p.base = static_cast<char*>(cpu_ptr);
  p.cpu_layer_stride = cpu_layer_stride_bytes;
  p.cpu_kv_stride = cpu_kv_stride_bytes;
  p.ssd_layer_stride = ssd_layer_stride_bytes;
  p.ssd_kv_stride = ssd_kv_stride_bytes;
  p.chunk = chunk_size_bytes;
  p.block_stride = block_stride_bytes;
  p.max_request = max_request_bytes();
  p.is_read = is_read != 0;
  p.direct = p.is_read && chunk_size_bytes % 4096 == 0;
  p.block_major = (p.kv == 1 || (cpu_kv_stride_bytes == chunk_size_bytes &&
                                 ssd_kv_stride_bytes == chunk_size_bytes)) &&
                  (num_layers == 1 || (cpu_layer_stride_bytes == p.kv * chunk_size_bytes &&
                                       ssd_layer_stride_bytes == p.kv * chunk_size_bytes));
  // partition by device, keeping the id-list order within a device
  p.dev_ssd.resize(p.D);
  p.dev_cpu.resize(p.D);
  for (int i = 0; i < num_blocks; ++i) {
    const int64_t b = ssd_block_ids[i], c = cpu_block_ids[i];
    if (b < 0 || c < 0) return ssd_fail("negative block id at position %d", i);
    const int64_t q = b / round_robin;
    const int d = static_cast<int>(q % p.D);
    p.dev_ssd[d].push_back((q / p.D) * round_robin + b % round_robin);
    p.dev_cpu[d].push_back(c);
  }
  ErrorSlot err;
  // The ring is checked under its lock: a call on another thread whose ring
  // broke shuts the ring down under the same lock, and this call then runs on
  // threads instead of driving a ring that is gone.
  std::unique_lock<std::mutex> ring_lock(h->uring_mu);
  if (h->uring.enabled()) {
    run_uring(h, p, err);
  } else {
    ring_lock.unlock();
    run_threads(h, p, num_threads_per_device, err);
  }
  if (err.failed) return ssd_fail("%s", err.msg.c_str());
  return 0;
} catch (const std::exception& e) {
  return ssd_fail("fkv_transfer_kv_blocks_ssd: %s", e.what());
}

}  // extern "C"
