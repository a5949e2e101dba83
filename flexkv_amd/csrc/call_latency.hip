// call_latency: per-call latency of fkv_transfer_kv_blocks for small calls,
// beside the floors it sits on, in one process.  Every figure is the median
// of 400 timed calls (after 20 untimed), each call followed by
// hipStreamSynchronize on one stream of device 0:
//
//   empty_kernel            an empty kernel without arguments
//   args_kernel             an empty kernel with 1.6 KiB of arguments
//   args{160,640,2560}_kernel  the same with 160 B, 640 B and 2.5 KiB
//   copy_kernel_{h2d,d2h}   a plain 64 KiB copy kernel (16 workgroups, one
//                           16-byte load and store per lane)
//   memcpy_{h2d,d2h}        hipMemcpyAsync of one contiguous 64 KiB run
//   memcpy_2x32k_h2d        two 32 KiB hipMemcpyAsync on the stream
//   fkv_1x1_{h2d,d2h}       fkv_transfer_kv_blocks, kernel mode, 1 block x 1
//                           layer x K/V of 32 KiB chunks (64 KiB)
//   fkv_16x1_{h2d,d2h}      the same with 16 blocks (1 MiB)
//
// The device cache is one layer [K|V][64 blocks][32 KiB]; the host cache is
// 64 blocks of [K|V][32 KiB] in pinned memory.  Output: one JSON line.
// FLEXKV_SMALL_KERNEL=0 in the environment sends the library's small calls to
// its general kernel, for comparison.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "flexkv_hip.h"

#define CK(x)                                                                     \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

namespace {

constexpr int64_t kChunk = 32 << 10;
constexpr int64_t kBlocks = 64;
constexpr int64_t kCopyBytes = 64 << 10;

__global__ void empty_kernel() {}

template <int kWords>
struct Blob {
  uint64_t v[kWords];
};

template <int kWords>
__global__ void args_kernel(Blob<kWords> b, uint64_t* sink) {
  if (threadIdx.x == 0 && b.v[0] == 12345) sink[0] = b.v[kWords - 1];
}

// n 16-byte vectors, one per thread (the launch covers exactly n threads)
__global__ void copy_kernel(const int4* __restrict__ src, int4* __restrict__ dst, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

template <class F>
double median_us(F f, int reps = 400) {
  std::vector<double> t;
  t.reserve(reps);
  for (int i = 0; i < reps + 20; ++i) {
    const auto a = std::chrono::steady_clock::now();
    f();
    const auto b = std::chrono::steady_clock::now();
    if (i >= 20) t.push_back(std::chrono::duration<double, std::micro>(b - a).count());
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

// an empty kernel with kWords * 8 bytes of arguments, launched and synchronised
template <int kWords>
double args_us(hipStream_t s, uint64_t* sink) {
  const Blob<kWords> blob{};
  return median_us([&] {
    hipLaunchKernelGGL(args_kernel<kWords>, dim3(1), dim3(64), 0, s, blob, sink);
    CK(hipStreamSynchronize(s));
  });
}

}  // namespace

int main() {
  CK(hipSetDevice(0));
  hipStream_t s;
  CK(hipStreamCreate(&s));
  char* layer = nullptr;   // [K|V][kBlocks][kChunk]
  CK(hipMalloc(&layer, 2 * kBlocks * kChunk));
  char* host = nullptr;    // [kBlocks][K|V][kChunk]
  CK(hipHostMalloc(&host, kBlocks * 2 * kChunk, 0));
  char* dev64 = nullptr;
  CK(hipMalloc(&dev64, kCopyBytes));
  uint64_t* sink = nullptr;
  CK(hipMalloc(&sink, 64));
  int64_t* ids = nullptr;  // [0]: gpu id, [1]: cpu id of the 1-block call; 16 + 16 after
  CK(hipHostMalloc(reinterpret_cast<void**>(&ids), 64 * sizeof(int64_t), 0));
  ids[0] = 5;
  ids[1] = 7;
  int64_t* ids16 = ids + 16;
  for (int i = 0; i < 16; ++i) {   // distinct ids: 7 and 11 are coprime with 64
    ids16[i] = (i * 7 + 3) % kBlocks;
    ids16[16 + i] = (i * 11 + 5) % kBlocks;
  }
  void** ptrs = nullptr;
  CK(hipHostMalloc(reinterpret_cast<void**>(&ptrs), sizeof(void*), 0));
  ptrs[0] = layer;
  CK(hipMemset(layer, 1, 2 * kBlocks * kChunk));
  std::memset(host, 2, kBlocks * 2 * kChunk);

  const int nvec = static_cast<int>(kCopyBytes / 16);
  const double empty = median_us([&] {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s);
    CK(hipStreamSynchronize(s));
  });
  const double args = args_us<208>(s, sink);   // 1664 bytes
  const double args160 = args_us<20>(s, sink);
  const double args640 = args_us<80>(s, sink);
  const double args2560 = args_us<320>(s, sink);
  const double copy_h2d = median_us([&] {
    hipLaunchKernelGGL(copy_kernel, dim3(nvec / 256), dim3(256), 0, s,
                       reinterpret_cast<const int4*>(host), reinterpret_cast<int4*>(dev64), nvec);
    CK(hipStreamSynchronize(s));
  });
  const double copy_d2h = median_us([&] {
    hipLaunchKernelGGL(copy_kernel, dim3(nvec / 256), dim3(256), 0, s,
                       reinterpret_cast<const int4*>(dev64), reinterpret_cast<int4*>(host), nvec);
    CK(hipStreamSynchronize(s));
  });
  const double memcpy_h2d = median_us([&] {
    CK(hipMemcpyAsync(dev64, host, kCopyBytes, hipMemcpyHostToDevice, s));
    CK(hipStreamSynchronize(s));
  });
  const double memcpy_d2h = median_us([&] {
    CK(hipMemcpyAsync(host, dev64, kCopyBytes, hipMemcpyDeviceToHost, s));
    CK(hipStreamSynchronize(s));
  });
  const double memcpy_2x = median_us([&] {
    CK(hipMemcpyAsync(layer + 3 * kChunk, host, kChunk, hipMemcpyHostToDevice, s));
    CK(hipMemcpyAsync(layer + (kBlocks + 3) * kChunk, host + kChunk, kChunk,
                      hipMemcpyHostToDevice, s));
    CK(hipStreamSynchronize(s));
  });
  auto fkv = [&](int nb, const int64_t* gids, const int64_t* cids, int h2d) {
    const int rc = fkv_transfer_kv_blocks(nb, 0, 1, gids, ptrs, kBlocks * kChunk, kChunk, cids,
                                          host, kChunk, 2 * kChunk, 2 * kChunk, 0, kChunk, s,
                                          -1, h2d, FKV_XFER_KERNEL, 0);
    if (rc) {
      std::fprintf(stderr, "fkv_transfer_kv_blocks failed (%d): %s\n", rc, fkv_last_error());
      std::exit(1);
    }
  };
  const double f1h = median_us([&] { fkv(1, &ids[0], &ids[1], 1); });
  const double f1d = median_us([&] { fkv(1, &ids[0], &ids[1], 0); });
  const double f16h = median_us([&] { fkv(16, ids16, ids16 + 16, 1); });
  const double f16d = median_us([&] { fkv(16, ids16, ids16 + 16, 0); });
  const char* sk = std::getenv("FLEXKV_SMALL_KERNEL");
  std::printf("{\"small_kernel\": %s, \"empty_kernel_us\": %.2f, \"args_kernel_us\": %.2f, "
              "\"args160_kernel_us\": %.2f, \"args640_kernel_us\": %.2f, \"args2560_kernel_us\": %.2f, "
              "\"copy_kernel_h2d_us\": %.2f, \"copy_kernel_d2h_us\": %.2f, "
              "\"memcpy_h2d_us\": %.2f, \"memcpy_d2h_us\": %.2f, \"memcpy_2x32k_h2d_us\": %.2f, "
              "\"fkv_1x1_h2d_us\": %.2f, \"fkv_1x1_d2h_us\": %.2f, "
              "\"fkv_16x1_h2d_us\": %.2f, \"fkv_16x1_d2h_us\": %.2f}\n",
              (sk && std::atoi(sk) == 0) ? "false" : "true", empty, args, args160, args640,
              args2560, copy_h2d, copy_d2h,
              memcpy_h2d, memcpy_d2h, memcpy_2x, f1h, f1d, f16h, f16d);
  if (fkv_finalize() != 0) std::fprintf(stderr, "fkv_finalize: %s\n", fkv_last_error());
  CK(hipStreamDestroy(s));
  CK(hipFree(layer));
  CK(hipFree(dev64));
  CK(hipFree(sink));
  CK(hipHostFree(host));
  CK(hipHostFree(ids));
  CK(hipHostFree(ptrs));
  return 0;
}
