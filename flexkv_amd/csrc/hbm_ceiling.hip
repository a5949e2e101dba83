// hbm_ceiling.hip - measured HBM stream ceilings of one device.
//
// The KV gather/scatter kernels read and write every byte once, so the rate a
// plain device copy reaches bounds them, and a copy is bounded in turn by what
// the device sustains for reads alone and for writes alone.  This program
// measures all three over `bytes`-sized buffers (default 4 GiB) with 16-byte
// accesses per lane and prints one JSON line: the best rate of each kind, the
// launch shape that reached it, and every configuration tried.
//
//   ./hbm_ceiling [bytes]
//
// Rates are counted as bytes read plus bytes written per second (10^9 B/s);
// each configuration is timed as the best of 10 launches with HIP events.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 gvec;
constexpr int kThreads = 256;

#define CHECK(x)                                                                        \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      fprintf(stderr, "hbm_ceiling: %s failed: %s\n", #x, hipGetErrorString(e_));       \
      exit(1);                                                                          \
    }                                                                                   \
  } while (0)

// Every kernel walks vectors [0, nvec) in groups of kUnroll x 256 vectors per
// workgroup, grid-stride; a group is processed only when all of it is in
// range (nvec is a multiple of every group size used, up to 32 x 256 vectors
// = 128 KiB: the buffer size is a multiple of 1 MiB).

template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4* src0, u32x4* sink, size_t nvec) {
  const gvec* src = (const gvec*)src0;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads * kUnroll;
  u32x4 acc = {0, 0, 0, 0};
  for (; i + (kUnroll - 1) * kThreads < nvec; i += stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      v[u] = kNt ? __builtin_nontemporal_load(src + i + u * kThreads) : src[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  // one 16-byte result per thread keeps the loads live
  sink[static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kThreads) void write_kernel(u32x4* dst0, size_t nvec) {
  gvec* dst = (gvec*)dst0;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads * kUnroll;
  const u32x4 v = {static_cast<unsigned>(i), 1u, 2u, 3u};
  for (; i + (kUnroll - 1) * kThreads < nvec; i += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (kNt)
        __builtin_nontemporal_store(v, dst + i + u * kThreads);
      else
        dst[i + u * kThreads] = v;
    }
  }
}

template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kThreads) void copy_kernel(const u32x4* src0, u32x4* dst0, size_t nvec) {
  const gvec* src = (const gvec*)src0;
  gvec* dst = (gvec*)dst0;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads * kUnroll;
  for (; i + (kUnroll - 1) * kThreads < nvec; i += stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      v[u] = kNt ? __builtin_nontemporal_load(src + i + u * kThreads) : src[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (kNt)
        __builtin_nontemporal_store(v[u], dst + i + u * kThreads);
      else
        dst[i + u * kThreads] = v[u];
    }
  }
}

// Each wavefront copies kRows consecutive 1 KiB rows (64 lanes x 16 B): the
// access pattern of the KV gather, whose wavefronts stream whole chunks.
template <int kRows, bool kNt>
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(const u32x4* src0, u32x4* dst0,
                                                             size_t nvec) {
  const gvec* src = (const gvec*)src0;
  gvec* dst = (gvec*)dst0;
  constexpr int kWaves = kThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t nrows = nvec / 64;
  size_t row = (static_cast<size_t>(blockIdx.x) * kWaves + wave) * kRows;
  const size_t stride = static_cast<size_t>(gridDim.x) * kWaves * kRows;
  for (; row + kRows <= nrows; row += stride) {
    u32x4 v[kRows];
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const gvec* p = src + (row + u) * 64 + lane;
      v[u] = kNt ? __builtin_nontemporal_load(p) : *p;
    }
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      gvec* p = dst + (row + u) * 64 + lane;
      if (kNt)
        __builtin_nontemporal_store(v[u], p);
      else
        *p = v[u];
    }
  }
}

struct Best {
  double gbps = 0;
  std::string config;
};

hipEvent_t g_e0, g_e1;
std::string g_all;

template <class Launch>
void measure(const char* kind, const char* name, int grid, double bytes_counted, Best& best,
             Launch launch) {
  launch();
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  float best_ms = 1e30f;
  for (int r = 0; r < 10; ++r) {
    CHECK(hipEventRecord(g_e0));
    launch();
    CHECK(hipEventRecord(g_e1));
    CHECK(hipEventSynchronize(g_e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, g_e0, g_e1));
    if (ms < best_ms) best_ms = ms;
  }
  const double gbps = bytes_counted / (best_ms * 1e-3) / 1e9;
  char cfg[96];
  snprintf(cfg, sizeof(cfg), "%s grid %d", name, grid);
  if (gbps > best.gbps) {
    best.gbps = gbps;
    best.config = cfg;
  }
  char row[192];
  snprintf(row, sizeof(row), "%s{\"kind\": \"%s\", \"config\": \"%s\", \"gbps\": %.1f}",
           g_all.empty() ? "" : ", ", kind, cfg, gbps);
  g_all += row;
}

}  // namespace

int main(int argc, char** argv) {
  size_t bytes = size_t(4) << 30;
  if (argc > 1) bytes = strtoull(argv[1], nullptr, 10);
  bytes &= ~((size_t(1) << 20) - 1);   // whole MiB: every group size divides it
  if (bytes < (size_t(64) << 20)) {
    fprintf(stderr, "hbm_ceiling: buffer of at least 64 MiB required\n");
    return 2;
  }
  const size_t nvec = bytes / 16;
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, dev));
  const int max_mult = 64;
  u32x4 *a = nullptr, *b = nullptr, *sink = nullptr;
  CHECK(hipMalloc(&a, bytes));
  CHECK(hipMalloc(&b, bytes));
  CHECK(hipMalloc(&sink, static_cast<size_t>(cus) * max_mult * kThreads * sizeof(u32x4)));
  CHECK(hipMemset(a, 1, bytes));
  CHECK(hipMemset(b, 0, bytes));
  CHECK(hipEventCreate(&g_e0));
  CHECK(hipEventCreate(&g_e1));

  const double one = static_cast<double>(bytes), two = 2.0 * bytes;
  Best rd, wr, cp;
  for (int mult : {4, 8, 16, 32}) {
    const int grid = cus * mult;   // <= cus * max_mult: sink holds one vector per thread
    measure("read", "unroll 4 nt", grid, one, rd,
            [&] { read_kernel<4, true><<<grid, kThreads>>>(a, sink, nvec); });
    measure("read", "unroll 8 nt", grid, one, rd,
            [&] { read_kernel<8, true><<<grid, kThreads>>>(a, sink, nvec); });
    measure("write", "unroll 8", grid, one, wr,
            [&] { write_kernel<8, false><<<grid, kThreads>>>(b, nvec); });
    measure("write", "unroll 8 nt", grid, one, wr,
            [&] { write_kernel<8, true><<<grid, kThreads>>>(b, nvec); });
    measure("copy", "unroll 8 nt", grid, two, cp,
            [&] { copy_kernel<8, true><<<grid, kThreads>>>(a, b, nvec); });
    measure("copy", "unroll 32 nt", grid, two, cp,
            [&] { copy_kernel<32, true><<<grid, kThreads>>>(a, b, nvec); });
  }
  // one pass: a workgroup per group of vectors, no grid-stride loop
  auto one_pass = [&](int unroll) {
    return static_cast<int>(nvec / (static_cast<size_t>(kThreads) * unroll));
  };
  measure("write", "one pass, unroll 4", one_pass(4), one, wr,
          [&] { write_kernel<4, false><<<one_pass(4), kThreads>>>(b, nvec); });
  measure("write", "one pass, unroll 8", one_pass(8), one, wr,
          [&] { write_kernel<8, false><<<one_pass(8), kThreads>>>(b, nvec); });
  measure("copy", "one pass, unroll 4 nt", one_pass(4), two, cp,
          [&] { copy_kernel<4, true><<<one_pass(4), kThreads>>>(a, b, nvec); });
  measure("copy", "one pass, unroll 8 nt", one_pass(8), two, cp,
          [&] { copy_kernel<8, true><<<one_pass(8), kThreads>>>(a, b, nvec); });
  measure("copy", "one pass, unroll 16 nt", one_pass(16), two, cp,
          [&] { copy_kernel<16, true><<<one_pass(16), kThreads>>>(a, b, nvec); });
  measure("copy", "one pass, unroll 32 nt", one_pass(32), two, cp,
          [&] { copy_kernel<32, true><<<one_pass(32), kThreads>>>(a, b, nvec); });
  measure("copy", "one pass, unroll 32", one_pass(32), two, cp,
          [&] { copy_kernel<32, false><<<one_pass(32), kThreads>>>(a, b, nvec); });
  // wavefront-contiguous rows, one pass: a wavefront per kRows rows
  auto row_pass = [&](int rows) {
    return static_cast<int>(nvec / 64 / (static_cast<size_t>(kThreads / 64) * rows));
  };
  measure("copy", "rows per wave 16 nt, one pass", row_pass(16), two, cp,
          [&] { copy_rows_kernel<16, true><<<row_pass(16), kThreads>>>(a, b, nvec); });
  measure("copy", "rows per wave 32 nt, one pass", row_pass(32), two, cp,
          [&] { copy_rows_kernel<32, true><<<row_pass(32), kThreads>>>(a, b, nvec); });
  measure("copy", "rows per wave 32, one pass", row_pass(32), two, cp,
          [&] { copy_rows_kernel<32, false><<<row_pass(32), kThreads>>>(a, b, nvec); });
  for (int mult : {8, 16}) {
    const int grid = cus * mult;
    measure("copy", "rows per wave 32 nt", grid, two, cp,
            [&] { copy_rows_kernel<32, true><<<grid, kThreads>>>(a, b, nvec); });
  }
  printf("{\"device\": \"%s\", \"cus\": %d, \"bytes\": %zu, "
         "\"read_gbps\": %.1f, \"read_config\": \"%s\", "
         "\"write_gbps\": %.1f, \"write_config\": \"%s\", "
         "\"copy_gbps\": %.1f, \"copy_config\": \"%s\", \"runs\": [%s]}\n",
         prop.gcnArchName, cus, bytes, rd.gbps, rd.config.c_str(), wr.gbps, wr.config.c_str(),
         cp.gbps, cp.config.c_str(), g_all.c_str());
  CHECK(hipFree(a));
  CHECK(hipFree(b));
  CHECK(hipFree(sink));
  return 0;
}
