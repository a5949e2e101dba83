// CPU-only check of the bounded copy-engine wait (flexkv_amd/csrc/kv_wait.h)
// with stub signal operations: no HSA runtime, no device.  Prints one line
// per case and exits non-zero on the first failure.
#include "kv_wait.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <thread>
#include <vector>

using fkv_detail::HostRowLedger;
using fkv_detail::wait_copies;
using fkv_detail::wait_half;
using fkv_detail::WaitOutcome;
using clk = std::chrono::steady_clock;

namespace {

// A signal drops to 0 after `remaining[s]` observations; -1 never drops.
struct StubOps {
  std::map<uint64_t, int> remaining;
  uint64_t max_hint = 0;
  int waits = 0, loads = 0;
  hsa_signal_value_t observe(hsa_signal_t s) {
    int& r = remaining[s.handle];
    if (r < 0) return 1;
    if (r == 0) return 0;
    --r;
    return 1;
  }
  hsa_signal_value_t wait(hsa_signal_t s, uint64_t hint, bool) {
    ++waits;
    if (hint > max_hint) max_hint = hint;
    const hsa_signal_value_t v = observe(s);
    if (v >= 1) std::this_thread::sleep_for(std::chrono::microseconds(200));   // a 'slice'
    return v;
  }
  hsa_signal_value_t load(hsa_signal_t s) {
    ++loads;
    return observe(s);
  }
  uint64_t ticks_per_ms() const { return 100000; }   // a 100 MHz timestamp clock
};

int failures = 0;
void check(bool ok, const char* what) {
  std::printf("%s: %s\n", ok ? "ok" : "FAIL", what);
  if (!ok) ++failures;
}

hsa_signal_t sig(uint64_t h) { return hsa_signal_t{h}; }

}  // namespace

int main() {
  {  // every signal finishes after a few observations
    StubOps ops;
    ops.remaining = {{1, 3}, {2, 0}, {3, 5}, {4, 2}};
    const WaitOutcome w = wait_copies(ops, {sig(1)}, {sig(1), sig(2), sig(3), sig(4)}, false,
                                      clk::now() + std::chrono::seconds(5));
    check(w.done, "copies that finish are waited for");
    check(ops.max_hint == 100000, "each blocking wait is one 1 ms slice of the timestamp clock");
  }
  {  // an interrupt signal that never drops: the deadline ends the wait
    StubOps ops;
    ops.remaining = {{7, -1}, {8, 0}};
    const auto t0 = clk::now();
    const WaitOutcome w = wait_copies(ops, {sig(7)}, {sig(8), sig(7)}, true,
                                      t0 + std::chrono::milliseconds(50));
    const double ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    check(!w.done && w.stuck.handle == 7 && w.value == 1, "a stalled interrupt signal times out");
    check(ms >= 50 && ms < 2000, "the stalled wait ends at the deadline");
  }
  {  // a polled signal that never drops behind interrupt signals that do
    StubOps ops;
    ops.remaining = {{1, 0}, {2, -1}, {3, 0}};
    const auto t0 = clk::now();
    const WaitOutcome w = wait_copies(ops, {sig(1)}, {sig(1), sig(2), sig(3)}, false,
                                      t0 + std::chrono::milliseconds(30));
    const double ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    check(!w.done && w.stuck.handle == 2, "a stalled polled signal times out");
    check(ms >= 30 && ms < 2000, "the polling loop ends at the deadline");
  }
  {  // no copies queued: nothing to wait for
    StubOps ops;
    const WaitOutcome w = wait_copies(ops, {}, {}, false, clk::now());
    check(w.done && ops.waits == 0 && ops.loads == 0, "an empty half returns at once");
  }
  {  // the host rows of a device-to-host transfer whose second half stalls
    StubOps ops;
    ops.remaining = {{1, 2}, {2, -1}, {3, -1}};   // half 0's copy finishes, 2 and 3 never
    HostRowLedger rows;
    const int64_t piece0[] = {10, 11, 12, 13}, piece1[] = {20, 21, 22}, piece2[] = {30, 31};
    const auto soon = [] { return clk::now() + std::chrono::milliseconds(20); };
    rows.queued(0, piece0, 4);
    rows.queued(1, piece1, 3);
    check(wait_half(ops, {sig(1)}, {sig(1)}, false, soon(), rows, 0).done,
          "the first half's copies finish");
    check(rows.unsafe.empty() && rows.pending[0].empty(),
          "a finished half leaves no unsafe rows");
    rows.queued(0, piece2, 2);   // the next piece reuses half 0
    check(!wait_half(ops, {sig(2)}, {sig(2)}, true, soon(), rows, 1).done,
          "the second half times out");
    check((rows.unsafe == std::vector<int64_t>{20, 21, 22}),
          "the timed-out half's host blocks are reported unsafe");
    // the failing call's drain waits for the other half too, which also stalls
    check(!wait_half(ops, {sig(3)}, {sig(3)}, false, soon(), rows, 0).done,
          "the drain's wait on the other half times out");
    const std::vector<int64_t> got = rows.take_unsafe();
    check((got == std::vector<int64_t>{20, 21, 22, 30, 31}),
          "both halves' host blocks are reported, in order");
    check(rows.unsafe.empty() && rows.pending[0].empty() && rows.pending[1].empty(),
          "the report empties the ledger");
  }
  return failures ? 1 : 0;
}
