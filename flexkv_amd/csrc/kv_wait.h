// kv_wait.h - the bounded wait for copy-engine completion signals.
//
// Header-only and free of HIP, so a CPU-only test can drive it with stub
// signal operations.  Every copy the copy-engine path queues carries a
// completion signal that starts at 1 and drops to 0 when the engine is done.
// The wait blocks (or spins) on the few interrupt signals of each engine's
// last copy, then checks every copy's own signal by loading it, and gives up
// at a deadline instead of waiting forever on an engine that stalled.
#pragma once

#include <hsa/hsa.h>

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace fkv_detail {

// How long one host wait on a copy-engine half may take before the transfer
// fails (FLEXKV_SDMA_TIMEOUT_MS; default 20 s).  A staging half holds at most
// a few hundred MiB, which the link moves in milliseconds.
constexpr int64_t kDefaultSdmaTimeoutMs = 20000;

// The outcome of wait_copies: every signal reached 0, or the deadline passed
// with `stuck` still at 1 or more.
struct WaitOutcome {
  bool done = true;
  hsa_signal_t stuck{0};
  hsa_signal_value_t value = 0;
};

// Ops provides:
//   hsa_signal_value_t wait(hsa_signal_t s, uint64_t hint_ticks, bool spin)
//       one bounded host wait on an interrupt signal for its value to drop
//       below 1 (a blocking or spinning hsa_signal_wait_scacquire with a
//       finite timeout hint); returns the value observed;
//   hsa_signal_value_t load(hsa_signal_t s)   an acquire load;
//   uint64_t ticks_per_ms() const              timestamp ticks per millisecond.
// `deadline` bounds the whole call.
template <class Ops>
WaitOutcome wait_copies(Ops& ops, const std::vector<hsa_signal_t>& wake,
                        const std::vector<hsa_signal_t>& queued, bool spin,
                        std::chrono::steady_clock::time_point deadline) {
  using clock = std::chrono::steady_clock;
  WaitOutcome out;
  // Waits are cut into slices of at most 1 ms of the runtime's timestamp
  // clock; the timeout argument of an HSA wait is only a hint, so the clock
  // decides.
  const uint64_t slice = ops.ticks_per_ms() > 0 ? ops.ticks_per_ms() : 1;
  for (hsa_signal_t s : wake) {
    hsa_signal_value_t v;
    while ((v = ops.wait(s, slice, spin)) >= 1) {
      if (clock::now() >= deadline) {
        out.done = false;
        out.stuck = s;
        out.value = v;
        return out;
      }
    }
  }
  for (hsa_signal_t s : queued) {
    hsa_signal_value_t v;
    unsigned polls = 0;
    while ((v = ops.load(s)) >= 1) {
      if ((++polls & 63) == 0 && clock::now() >= deadline) {
        out.done = false;
        out.stuck = s;
        out.value = v;
        return out;
      }
      std::this_thread::yield();
    }
  }
  return out;
}

// Which host blocks the device-to-host copies of each staging half write.
// A half holds one piece at a time: queued() records the piece's host block
// ids when its copies are queued, finished() forgets them once the wait on
// the half succeeds, and abandoned() moves them to `unsafe` when the wait
// gives up: an engine may still write those blocks' rows of the host cache
// after the call has returned.  take_unsafe() hands the list to the caller
// and empties it.
struct HostRowLedger {
  std::vector<int64_t> pending[2];
  std::vector<int64_t> unsafe;

  void queued(int half, const int64_t* ids, size_t n) { pending[half].assign(ids, ids + n); }
  void finished(int half) { pending[half].clear(); }
  void abandoned(int half) {
    unsafe.insert(unsafe.end(), pending[half].begin(), pending[half].end());
    pending[half].clear();
  }
  std::vector<int64_t> take_unsafe() {
    std::vector<int64_t> out;
    out.swap(unsafe);
    return out;
  }
};

// One bounded wait on the copies of staging half `half`, keeping the ledger:
// the half's host blocks are forgotten when its copies have finished and
// become unsafe when the wait gives up.
template <class Ops>
WaitOutcome wait_half(Ops& ops, const std::vector<hsa_signal_t>& wake,
                      const std::vector<hsa_signal_t>& queued, bool spin,
                      std::chrono::steady_clock::time_point deadline, HostRowLedger& rows,
                      int half) {
  const WaitOutcome w = wait_copies(ops, wake, queued, spin, deadline);
  if (w.done)
    rows.finished(half);
  else
    rows.abandoned(half);
  return w;
}

}  // namespace fkv_detail
