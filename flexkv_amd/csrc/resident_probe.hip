// resident_probe.hip - a kernel that only occupies compute units.
//
// bench.py times whole-device GEMMs beside a transfer kernel.  To tell
// whether a kernel resident beside them costs the GEMMs through what it does
// (issue slots, memory traffic) or through being there at all, it also runs
// this kernel: each wavefront sleeps (s_sleep) between reads of the
// constant-rate wall clock until `ms` milliseconds have passed, touching no
// memory.  Launched from Python through ctypes on a torch stream:
//
//   int fkv_probe_resident(void* stream, double ms, int grid, int block);
//
// returns a hipError_t value (0 on success).
#include <hip/hip_runtime.h>

namespace {

__global__ void resident_sleep_kernel(long long ticks) {
  const long long t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(127);
}

}  // namespace

extern "C" int fkv_probe_resident(void* stream, double ms, int grid, int block) {
  int dev = 0, khz = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (grid < 1 || block < 1 || block > 1024 || ms < 0 || khz <= 0)
    return static_cast<int>(hipErrorInvalidValue);
  const long long ticks = static_cast<long long>(ms * khz);
  hipLaunchKernelGGL(resident_sleep_kernel, dim3(grid), dim3(block), 0,
                     static_cast<hipStream_t>(stream), ticks);
  return static_cast<int>(hipGetLastError());
}
