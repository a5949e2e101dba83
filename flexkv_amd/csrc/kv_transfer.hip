// kv_transfer.hip - GPU<->CPU KV-block transfer for MI355X (gfx950).
//
// One kernel template moves "chunks": the (layer, K|V, block) pieces of the
// KV cache, each `chunk_size` contiguous bytes on both sides
// (csrc/transfer.cu:39-53 gives the reference addressing).  It is used twice:
//   * zero-copy mode: the "CPU side" is the pinned host cache itself and the
//     kernel's 16-byte loads/stores travel over PCIe;
//   * copy-engine mode: the "CPU side" is a contiguous HBM staging buffer laid
//     out [block][layer][K|V][chunk]; the SDMA engines (queued through HSA)
//     then move maximal contiguous host runs between staging and the host
//     cache.
//
// Work decomposition: a workgroup (4 wavefronts) owns a tile of consecutive
// blocks; it stages the tile's (gpu_id, cpu_id) pairs in LDS, then its
// wavefronts stream the tile's rows (64 lanes x 16 B = 1 KiB) in groups of
// kUnroll rows, issuing all loads of a group before any store.  Rows are
// ordered block -> layer -> K|V -> offset, which is host-address order for the
// block-wise host layout.  Layer base pointers travel in the kernel argument
// block (scalar loads, no PCIe round trip per chunk).  Staging gathers whose
// chunks are whole groups of 32 rows address each group from one buffer
// resource per side instead of a 64-bit base per row.
//
// This file holds the kernels, the transfer paths that launch them and the
// transfer entry points of the C ABI; kv_host.cpp holds validation, id staging
// and the host-only entry points, kv_sdma.cpp the copy engines.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "kv_internal.h"

using namespace fkv_detail;

namespace {

// Rows (64 lanes x 16 B) each wavefront keeps in flight: the zero-copy
// kernel is PCIe bound, the staging gather/scatter HBM bound.  Measured on
// MI355X at the Llama-3-8B shape with 8 CUs: D2H best at 8 rows, H2D at 4.
#ifndef FKV_UNROLL_ZC_D2H
#define FKV_UNROLL_ZC_D2H 8
#endif
#ifndef FKV_UNROLL_ZC_H2D
#define FKV_UNROLL_ZC_H2D 4
#endif
#ifndef FKV_UNROLL_HBM
#define FKV_UNROLL_HBM 32
#endif
// Wave issue priority (s_setprio, 0-3) of the zero-copy kernel, which shares
// compute units with the caller's kernels when transfers overlap compute.
#ifndef FKV_ZC_PRIO
#define FKV_ZC_PRIO 0
#endif
// Staging gather/scatter launch shape: 1 = one workgroup per tile (grid =
// tiles), 0 = an occupancy-sized grid looping over tiles.
#ifndef FKV_HBM_ONEPASS
#define FKV_HBM_ONEPASS 1
#endif
// Tiles per occupancy slot the tiling aims for (zero-copy / staging).
#ifndef FKV_TILE_FACTOR
#define FKV_TILE_FACTOR 4
#endif
#ifndef FKV_TILE_FACTOR_HBM
#define FKV_TILE_FACTOR_HBM 16
#endif
// Staging gather / scatter: chunks of whole row groups take the kernel
// variant that addresses each group from one base (1) or the row-by-row one
// (0).  The whole-group variant keeps no per-row address and spills nothing.
// Measured on MI355X at the Llama-3-8B shape (TB/s of HBM traffic by launch
// size 128 MiB / 256 MiB / 512 MiB / 2 GiB): gather 5.41/5.71/5.89/6.07
// against 5.46/5.67/5.89/6.05 row by row; scatter 4.67/4.97/5.08/5.26
// against 4.01/4.67/5.10/5.42.  So the scatter takes the whole-group
// variant up to kWholeScatterMaxBytes per launch and the row-by-row one
// above, where kv_pack_span_kernel does not take it (a packed side that is
// not contiguous in row order; pack_shape).
#ifndef FKV_WHOLE_GATHER
#define FKV_WHOLE_GATHER 1
#endif
#ifndef FKV_WHOLE_SCATTER
#define FKV_WHOLE_SCATTER 1
#endif
// Zero-copy launches whose chunks are whole sub-groups (4 rows D2H, whose
// group of 8 rows in flight is addressed as two halves; 4 rows H2D) take the
// whole-group variant, which keeps one base per sub-group instead of one
// address per row (no spills).
#ifndef FKV_WHOLE_ZERO_COPY
#define FKV_WHOLE_ZERO_COPY 1
#endif
// Cache hints: loads are non-temporal everywhere; stores are non-temporal
// into HBM but plain into pinned host memory (about 2% faster D2H over PCIe).
#ifndef FKV_NT_LOAD
#define FKV_NT_LOAD 1
#endif
#ifndef FKV_NT_STORE_HBM
#define FKV_NT_STORE_HBM 1
#endif
#ifndef FKV_NT_STORE_HOST
#define FKV_NT_STORE_HOST 0
#endif
// The staging scatter (packed HBM -> scattered chunks) has its own knobs.
#ifndef FKV_UNROLL_SCATTER
#define FKV_UNROLL_SCATTER FKV_UNROLL_HBM
#endif
#ifndef FKV_TILE_FACTOR_SCATTER
#define FKV_TILE_FACTOR_SCATTER FKV_TILE_FACTOR_HBM
#endif
// Staging gather/scatter: hand each XCD a contiguous range of tiles instead
// of every eighth tile (workgroups are dispatched to the 8 XCDs round robin).
#ifndef FKV_XCD_REMAP
#define FKV_XCD_REMAP 0
#endif
// Tile order of the staging gather / scatter: 1 = block-major (consecutive
// workgroups take the layer windows of one block, so the packed side is
// walked in address order), 0 = layer-window-major (consecutive workgroups
// take one layer window of consecutive blocks).
#ifndef FKV_BLOCK_MAJOR_GATHER
#define FKV_BLOCK_MAJOR_GATHER 0
#endif
#ifndef FKV_BLOCK_MAJOR_SCATTER
#define FKV_BLOCK_MAJOR_SCATTER 0
#endif
// Dynamic LDS per staging workgroup (bytes), to cap its occupancy.
#ifndef FKV_HBM_LDS_PAD
#define FKV_HBM_LDS_PAD 0
#endif
#ifndef FKV_NT_LOAD_SCATTER
#define FKV_NT_LOAD_SCATTER FKV_NT_LOAD
#endif
#ifndef FKV_NT_STORE_SCATTER
#define FKV_NT_STORE_SCATTER FKV_NT_STORE_HBM
#endif

constexpr int kThreads = 256;               // 4 wavefronts of 64 lanes
constexpr int64_t kWholeScatterMaxBytes = int64_t(512) << 20;
constexpr int kWaves = kThreads / 64;
constexpr int kUnrollHbm = FKV_UNROLL_HBM;
// Sub-groups per group of the whole-group variant: the zero-copy D2H group of
// 8 rows in flight is two sub-groups of 4 rows, so chunks of 4 KiB (the
// Llama-3-70B TP-8 shard) take it; every other instantiation addresses its
// group as one.  Each sub-group lies inside one chunk.
template <bool kH2D, bool kIotaCpu>
constexpr int whole_sub_groups() { return (!kIotaCpu && !kH2D && FKV_UNROLL_ZC_D2H % 2 == 0) ? 2 : 1; }
constexpr int kMaxTileBlocks = 64;
// Transfers of at most this many blocks carry their (gpu_id, cpu_id) pairs in
// the kernel arguments, so no workgroup reads them over PCIe first (one host
// round trip less per call; a one-block zero-copy call is latency-bound).
constexpr int kInlineIds = 32;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
// Buffer resource word 3 for raw (unformatted, unswizzled) buffers on gfx9
// parts, and the cache-policy bit of buffer instructions meaning
// non-temporal on gfx94x/gfx950 (bit 1; bit 0 = sc0, bit 4 = sc1).
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kCachePolicyNt = 2;
// Every address the kernel touches is global memory (HBM or mapped pinned
// host memory); saying so lets the compiler emit global_* instead of flat_*.
typedef __attribute__((address_space(1))) u32x4 gvec;

struct CopyArgs {
  const int64_t* ids;        // device-visible (gpu_id, cpu_id) pairs (inline_n == 0)
  char* cpu_base;            // CPU side of launch layer 0, block index 0
  int64_t gpu_kv_stride;
  int64_t gpu_block_stride;
  int64_t cpu_kv_stride;
  int64_t cpu_layer_stride;
  int64_t cpu_block_stride;
  int64_t chunk_vec;         // 16-byte vectors per chunk
  int32_t rows_per_chunk;    // ceil(chunk_vec / 64)
  int32_t num_blocks;
  int32_t num_layers;        // layers in this launch (<= kMaxLayersPerLaunch)
  int32_t kv_dim;
  int32_t tile_blocks;       // a tile is tile_blocks blocks x tile_layers layers
  int32_t tile_layers;
  int32_t tiles_b;           // tiles along the block axis
  int32_t tiles_l;           // tiles along the layer axis
  int32_t block_major;       // tile order: layer windows of a block are consecutive tiles
  int32_t tiles_r;           // row ranges per tile (small transfers split a tile's rows)
  uint32_t split_rows;       // rows per range: a whole tile, or a multiple of the unroll
  int32_t num_tiles;
  int32_t ptrs_per_layer;    // 1: layer_ptr[l] + k*gpu_kv_stride; kv: layer_ptr[l*kv + k]
  int32_t inline_n;          // > 0: the launch's pairs are inline_ids, not ids
  int32_t ids_split;         // > 0: ids holds gpu ids, and cpu ids ids_split entries later
  uint64_t layer_ptr[kMaxLayersPerLaunch];
  int64_t inline_ids[2 * kInlineIds];
};

// A value every lane of the wavefront holds, moved to a scalar register.
__device__ inline int64_t wave_uniform(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// kH2D: copy CPU side -> GPU side.  kIotaCpu: the CPU side is staging and
// block i of the launch sits at CPU-side block index i (ids[2i+1] unused).
// Row addresses are wave-uniform (scalar registers); each lane adds its own
// 16-byte slot, so one 32-bit lane offset serves every access.
// kWhole: the launch's chunks are whole sub-groups of kUnroll / kSub full
// rows (kSub = whole_sub_groups(); the host checks rows_per_chunk % (kUnroll /
// kSub) == 0 and no partial row), so each sub-group lies inside one chunk and
// is addressed from one base per side.
template <bool kH2D, bool kIotaCpu, bool kWhole = false>
__global__ __launch_bounds__(kThreads) void kv_chunk_copy_kernel(CopyArgs a) {
  constexpr bool kScatter = kIotaCpu && kH2D;
  constexpr int kUnroll = kIotaCpu ? (kScatter ? FKV_UNROLL_SCATTER : kUnrollHbm)
                                   : (kH2D ? FKV_UNROLL_ZC_H2D : FKV_UNROLL_ZC_D2H);
  // only the zero-copy D2H instantiation stores into host memory
  constexpr bool kNtStore = kScatter ? FKV_NT_STORE_SCATTER
                                     : ((kIotaCpu || kH2D) ? FKV_NT_STORE_HBM : FKV_NT_STORE_HOST);
  constexpr bool kNtLoad = kScatter ? FKV_NT_LOAD_SCATTER : FKV_NT_LOAD;
  __shared__ int64_t s_gid[kMaxTileBlocks];
  __shared__ int64_t s_cid[kMaxTileBlocks];

  if (!kIotaCpu && FKV_ZC_PRIO > 0) __builtin_amdgcn_s_setprio(FKV_ZC_PRIO);
  const int lane = threadIdx.x & 63;
  const uint32_t lane_off = static_cast<uint32_t>(lane) * 16;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kv = static_cast<uint32_t>(a.kv_dim);
  const uint32_t rpc = static_cast<uint32_t>(a.rows_per_chunk);
  const uint32_t ppl = static_cast<uint32_t>(a.ptrs_per_layer);
  // true when every row of a chunk is a full 64-lane row
  const bool full_rows = (a.chunk_vec & 63) == 0;

  int first = blockIdx.x;
  if (kIotaCpu && FKV_XCD_REMAP && (gridDim.x & 7) == 0) {
    const int per = gridDim.x >> 3;
    first = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  for (int tile = first; tile < a.num_tiles; tile += gridDim.x) {
    const int tr = tile % a.tiles_r;
    const int tq = tile / a.tiles_r;
    const int tb = a.block_major ? tq / a.tiles_l : tq % a.tiles_b;
    const int tl = a.block_major ? tq % a.tiles_l : tq / a.tiles_b;
    const int b0 = tb * a.tile_blocks;
    const int nb = min(a.tile_blocks, a.num_blocks - b0);
    const int l0 = tl * a.tile_layers;
    const uint32_t nl = static_cast<uint32_t>(min(a.tile_layers, a.num_layers - l0));
    const uint32_t items_per_block = nl * kv;
    __syncthreads();  // previous tile's readers are done with the LDS ids
    if (threadIdx.x < nb) {
      const int j = b0 + threadIdx.x;
      int64_t gid, cid;
      if (a.inline_n) {
        gid = a.inline_ids[2 * j];
        cid = a.inline_ids[2 * j + 1];
      } else if (a.ids_split) {
        gid = a.ids[j];
        cid = a.ids[static_cast<int64_t>(a.ids_split) + j];
      } else {
        gid = a.ids[2 * static_cast<int64_t>(j)];
        cid = a.ids[2 * static_cast<int64_t>(j) + 1];
      }
      s_gid[threadIdx.x] = gid;
      s_cid[threadIdx.x] = kIotaCpu ? static_cast<int64_t>(j) : cid;
    }
    __syncthreads();

    // this workgroup's rows of the tile: [g_begin, g_end)
    const uint32_t rows = static_cast<uint32_t>(nb) * items_per_block * rpc;
    const uint32_t g_begin = static_cast<uint32_t>(tr) * a.split_rows;
    const uint32_t g_end = min(rows, g_begin + a.split_rows);
    if constexpr (kWhole) {
      // Groups start at multiples of kUnroll and sub-groups at multiples of
      // kR, so each sub-group lies inside one chunk: consecutive 1 KiB rows
      // on both sides.  A tile's rows are a multiple of kR, not always of
      // kUnroll, so a group's later sub-groups may lie past g_end.
      constexpr int kSub = whole_sub_groups<kH2D, kIotaCpu>();
      constexpr int kR = kUnroll / kSub;
      static_assert(kR * kSub == kUnroll, "a group is kSub sub-groups of kR rows");
      for (uint32_t g = g_begin + static_cast<uint32_t>(wave) * kUnroll; g < g_end;
           g += kWaves * kUnroll) {
        // Raw buffer accesses: the sub-group's base in a buffer resource
        // (scalar registers), the lane's 16-byte slot as the vector offset
        // and the row as a scalar offset, so no per-row 64-bit address is
        // kept.
        __amdgpu_buffer_rsrc_t rs[kSub], rd[kSub];
        bool live[kSub];
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
          const uint32_t gs = g + static_cast<uint32_t>(s * kR);
          live[s] = s == 0 || gs < g_end;
          // a sub-group past g_end takes the first one's row (never accessed)
          const uint32_t row = live[s] ? gs : g;
          const uint32_t item = row / rpc;
          const uint32_t rr = row - item * rpc;
          const uint32_t bi = item / items_per_block;
          const uint32_t rem = item - bi * items_per_block;
          const uint32_t l = rem / kv;
          const uint32_t k = rem - l * kv;
          const uint32_t layer = static_cast<uint32_t>(l0) + l;
          const int64_t gid = wave_uniform(s_gid[bi]);
          const int64_t cid = wave_uniform(s_cid[bi]);
          const int64_t row_off = static_cast<int64_t>(rr) * (64 * 16);
          char* gpu = reinterpret_cast<char*>(a.layer_ptr[layer * ppl + k * (ppl - 1)]) +
                      static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride +
                      row_off;
          char* cpu = a.cpu_base + static_cast<int64_t>(layer) * a.cpu_layer_stride +
                      static_cast<int64_t>(k) * a.cpu_kv_stride + cid * a.cpu_block_stride +
                      row_off;
          rs[s] = __builtin_amdgcn_make_buffer_rsrc(kH2D ? cpu : gpu, 0, -1, kBufferRsrcWord3);
          rd[s] = __builtin_amdgcn_make_buffer_rsrc(kH2D ? gpu : cpu, 0, -1, kBufferRsrcWord3);
        }
        i32x4 v[kUnroll];
#pragma unroll
        for (int s = 0; s < kSub; ++s)
          if (live[s]) {
#pragma unroll
            for (int u = 0; u < kR; ++u)
              v[s * kR + u] = __builtin_amdgcn_raw_buffer_load_b128(
                  rs[s], lane_off, u * (64 * 16), kNtLoad ? kCachePolicyNt : 0);
          }
#pragma unroll
        for (int s = 0; s < kSub; ++s)
          if (live[s]) {
#pragma unroll
            for (int u = 0; u < kR; ++u)
              __builtin_amdgcn_raw_buffer_store_b128(v[s * kR + u], rd[s], lane_off,
                                                     u * (64 * 16),
                                                     kNtStore ? kCachePolicyNt : 0);
          }
      }
    } else {
      for (uint32_t g = g_begin + static_cast<uint32_t>(wave) * kUnroll; g < g_end;
           g += kWaves * kUnroll) {
        if constexpr (kIotaCpu) {
          // Staging: the group's rows are walked twice from the same cursor
          // over (block, layer, K|V, row), once to issue the loads and once to
          // issue the stores.  No row address is held between the two walks,
          // so only the loaded data stays live: holding 2 x U 64-bit row
          // addresses spilled 358-387 scalar registers at U = 32.
          const uint32_t item0 = g / rpc;
          const uint32_t rr0 = g - item0 * rpc;
          const uint32_t bi0 = item0 / items_per_block;
          const uint32_t rem0 = item0 - bi0 * items_per_block;
          const uint32_t lw0 = rem0 / kv;
          const uint32_t kw0 = rem0 - lw0 * kv;
          u32x4 v[kUnroll];
#pragma unroll
          for (int pass = 0; pass < 2; ++pass) {
            uint32_t rr = rr0, bi = bi0, l = lw0, k = kw0;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
              const uint32_t bsafe = min(bi, static_cast<uint32_t>(nb - 1));
              const uint32_t layer = static_cast<uint32_t>(l0) + min(l, nl - 1);
              const int64_t gid = wave_uniform(s_gid[bsafe]);
              const int64_t cid = wave_uniform(s_cid[bsafe]);
              const int64_t row_off = static_cast<int64_t>(rr) * (64 * 16);
              char* gpu = reinterpret_cast<char*>(a.layer_ptr[layer * ppl + k * (ppl - 1)]) +
                          static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride +
                          row_off;
              char* cpu = a.cpu_base + static_cast<int64_t>(layer) * a.cpu_layer_stride +
                          static_cast<int64_t>(k) * a.cpu_kv_stride + cid * a.cpu_block_stride +
                          row_off;
              const bool live = (g + u < g_end) &&
                                (full_rows || static_cast<int64_t>(rr) * 64 + lane < a.chunk_vec);
              if (live) {
                if (pass == 0) {
                  const gvec* p = (const gvec*)((kH2D ? cpu : gpu) + lane_off);
                  v[u] = kNtLoad ? __builtin_nontemporal_load(p) : *p;
                } else {
                  gvec* p = (gvec*)((kH2D ? gpu : cpu) + lane_off);
                  if (kNtStore)
                    __builtin_nontemporal_store(v[u], p);
                  else
                    *p = v[u];
                }
              }
              // advance the cursor by one row
              if (++rr == rpc) {
                rr = 0;
                if (++k == kv) {
                  k = 0;
                  if (++l == nl) {
                    l = 0;
                    ++bi;
                  }
                }
              }
            }
          }
        } else {
          // Zero-copy: U is 4-8, so the group's row addresses are computed
          // once and held.  Walking twice made the host-to-device kernel on 2
          // compute units 35% slower (36.7 against 56.7 GB/s).
          uint32_t item = g / rpc;
          uint32_t rr = g - item * rpc;
          uint32_t bi = item / items_per_block;
          uint32_t rem = item - bi * items_per_block;
          uint32_t l = rem / kv;
          uint32_t k = rem - l * kv;
          const char* src[kUnroll];
          char* dst[kUnroll];
          bool live[kUnroll];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            const uint32_t bsafe = min(bi, static_cast<uint32_t>(nb - 1));
            const uint32_t layer = static_cast<uint32_t>(l0) + min(l, nl - 1);
            const int64_t gid = wave_uniform(s_gid[bsafe]);
            const int64_t cid = wave_uniform(s_cid[bsafe]);
            const int64_t row_off = static_cast<int64_t>(rr) * (64 * 16);
            char* gpu = reinterpret_cast<char*>(a.layer_ptr[layer * ppl + k * (ppl - 1)]) +
                        static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride +
                        row_off;
            char* cpu = a.cpu_base + static_cast<int64_t>(layer) * a.cpu_layer_stride +
                        static_cast<int64_t>(k) * a.cpu_kv_stride + cid * a.cpu_block_stride +
                        row_off;
            live[u] = (g + u < g_end) &&
                      (full_rows || static_cast<int64_t>(rr) * 64 + lane < a.chunk_vec);
            src[u] = kH2D ? cpu : gpu;
            dst[u] = kH2D ? gpu : cpu;
            // advance the cursor by one row
            if (++rr == rpc) {
              rr = 0;
              if (++k == kv) {
                k = 0;
                if (++l == nl) {
                  l = 0;
                  ++bi;
                }
              }
            }
          }
          u32x4 v[kUnroll];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            if (live[u]) {
              const gvec* p = (const gvec*)(src[u] + lane_off);
              v[u] = kNtLoad ? __builtin_nontemporal_load(p) : *p;
            }
          }
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            if (live[u]) {
              gvec* p = (gvec*)(dst[u] + lane_off);
              if (kNtStore)
                __builtin_nontemporal_store(v[u], p);
              else
                *p = v[u];
            }
          }
        }
      }
    }
  }
}

// The staging gather / scatter over packed rows.  The packed (staging)
// side of a launch is contiguous in row order, block -> layer -> K|V ->
// row, each row 1 KiB, so row r lies at packed + r KiB.  The launch's rows
// are cut into groups of kU consecutive rows and wavefront w of workgroup b
// moves group 4b + w: no tile, no LDS, no barrier, and every wavefront moves
// a full group.  A group is kC whole chunks of kU / kC rows (kC > 1: chunks
// of 4-16 KiB, e.g. the Llama-3-70B TP-8 shard's 4 KiB) or kU rows inside
// one chunk (kC == 1: 24 KiB chunks at kU = 24).  The host checks the
// shape: full 1 KiB
// rows, whole groups, a contiguous packed side, ids in device memory.
struct PackArgs {
  const int64_t* gids;       // device memory: gpu id of launch block i at gids[i]
  char* packed;              // staging address of launch row 0
  int64_t gpu_kv_stride;
  int64_t gpu_block_stride;
  uint32_t rows_per_chunk;
  uint32_t items_per_block;  // layers x kv of the launch
  uint32_t kv_dim;
  uint32_t num_layers;       // layers of the launch
  uint32_t num_groups;
  uint32_t num_rows;         // packed rows of the launch
  int32_t ptrs_per_layer;    // 1: layer_ptr[l] + k*gpu_kv_stride; kv: layer_ptr[l*kv + k]
  uint64_t layer_ptr[kMaxLayersPerLaunch];
};

template <bool kH2D, int kU, int kC>
__global__ __launch_bounds__(kThreads) void kv_pack_kernel(PackArgs a) {
  static_assert(kU % kC == 0, "a group is kC whole chunks");
  constexpr int kR = kU / kC;                 // rows per chunk when kC > 1
  constexpr int kRow = 64 * 16;               // bytes per row
  const uint32_t lane_off = (threadIdx.x & 63) * 16;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t g = blockIdx.x * kWaves + wave;
  if (g >= a.num_groups) return;
  const uint32_t kv = a.kv_dim;
  const uint32_t ppl = static_cast<uint32_t>(a.ptrs_per_layer);
  // the group's first chunk and its first row inside that chunk
  uint32_t c, rr;
  if constexpr (kC > 1) {
    c = g * kC;
    rr = 0;
  } else {
    const uint32_t row0 = g * kU;
    c = row0 / a.rows_per_chunk;
    rr = row0 - c * a.rows_per_chunk;
  }
  uint32_t bi = c / a.items_per_block;
  const uint32_t rem = c - bi * a.items_per_block;
  uint32_t l = rem / kv;
  uint32_t k = rem - l * kv;
  // The ids do not change during the launch: read them through the constant
  // address space, so the wave-uniform reads are scalar loads.
  const __attribute__((address_space(4))) int64_t* gids =
      (const __attribute__((address_space(4))) int64_t*)a.gids;
  int64_t gid = gids[bi];
  // scattered side: one base per chunk of the group
  char* chunk_base[kC];
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    chunk_base[j] = reinterpret_cast<char*>(a.layer_ptr[l * ppl + k * (ppl - 1)]) +
                    static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride +
                    static_cast<int64_t>(rr) * kRow;
    if (j + 1 < kC) {
      if (++k == kv) {
        k = 0;
        if (++l == a.num_layers) {
          l = 0;
          gid = gids[++bi];
        }
      }
    }
  }
  char* packed = a.packed + static_cast<int64_t>(g) * (kU * kRow);
  u32x4 v[kU];
#pragma unroll
  for (int j = 0; j < kC; ++j)
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const char* src = kH2D ? packed + (j * kR + r) * kRow : chunk_base[j] + r * kRow;
      v[j * kR + r] = __builtin_nontemporal_load((const gvec*)(src + lane_off));
    }
#pragma unroll
  for (int j = 0; j < kC; ++j)
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      char* dst = kH2D ? chunk_base[j] + r * kRow : packed + (j * kR + r) * kRow;
      __builtin_nontemporal_store(v[j * kR + r], (gvec*)(dst + lane_off));
    }
}

// 32-row packed groups over chunks of 8 rows or more: group g moves packed
// rows [32g, 32g + 32), fewer in the launch's last group.  They lie in chunk
// c = 32g / rows_per_chunk and the chunks after it, at most kB = 2 + 30 /
// rows_per_chunk chunks in all (2 from 31 rows per chunk, 3 from 16, 4 from
// 11, 5 from 8; span_bases), so a wavefront
// holds kB bases and picks one per row with wave-uniform compares (MLA's
// 72-row chunks: a group reads 32 rows of one chunk, or the tail of one and
// the head of the next).  Walk order, id reads and accesses as in
// kv_pack_kernel.
template <bool kH2D, int kB>
__global__ __launch_bounds__(kThreads) void kv_pack_span_kernel(PackArgs a) {
  constexpr int kU = 32;
  constexpr int kRow = 64 * 16;
  const uint32_t lane_off = (threadIdx.x & 63) * 16;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t g = blockIdx.x * kWaves + wave;
  if (g >= a.num_groups) return;
  const uint32_t rpc = a.rows_per_chunk;
  const uint32_t row0 = g * kU;
  const uint32_t c = row0 / rpc;
  const uint32_t rr = row0 - c * rpc;
  const uint32_t rows = min(static_cast<uint32_t>(kU), a.num_rows - row0);
  const uint32_t kv = a.kv_dim;
  const uint32_t ppl = static_cast<uint32_t>(a.ptrs_per_layer);
  uint32_t bi = c / a.items_per_block;
  const uint32_t rem = c - bi * a.items_per_block;
  uint32_t l = rem / kv;
  uint32_t k = rem - l * kv;
  const __attribute__((address_space(4))) int64_t* gids =
      (const __attribute__((address_space(4))) int64_t*)a.gids;
  int64_t gid = gids[bi];
  // Row r of the group lies at base[j] + r * kRow for the last j with
  // edge[j] <= r: chunk c + j starts at group row edge[j] (edge[0] = 0).
  char* base[kB];
  uint32_t edge[kB];
  base[0] = reinterpret_cast<char*>(a.layer_ptr[l * ppl + k * (ppl - 1)]) +
            static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride +
            static_cast<int64_t>(rr) * kRow;
  edge[0] = 0;
#pragma unroll
  for (int j = 1; j < kB; ++j) {
    edge[j] = rpc - rr + (j - 1) * rpc;
    base[j] = base[j - 1];
    if (edge[j] < rows) {
      if (++k == kv) {
        k = 0;
        if (++l == a.num_layers) {
          l = 0;
          gid = gids[++bi];
        }
      }
      base[j] = reinterpret_cast<char*>(a.layer_ptr[l * ppl + k * (ppl - 1)]) +
                static_cast<int64_t>(k) * a.gpu_kv_stride + gid * a.gpu_block_stride -
                static_cast<int64_t>(edge[j]) * kRow;
    }
  }
  char* packed = a.packed + static_cast<int64_t>(g) * (kU * kRow);
  u32x4 v[kU];
#pragma unroll
  for (int r = 0; r < kU; ++r) {
    if (r < rows) {
      char* b = base[0];
#pragma unroll
      for (int j = 1; j < kB; ++j)
        if (r >= edge[j]) b = base[j];
      const char* src = kH2D ? packed + r * kRow : b + r * kRow;
      v[r] = __builtin_nontemporal_load((const gvec*)(src + lane_off));
    }
  }
#pragma unroll
  for (int r = 0; r < kU; ++r) {
    if (r < rows) {
      char* b = base[0];
#pragma unroll
      for (int j = 1; j < kB; ++j)
        if (r >= edge[j]) b = base[j];
      char* dst = kH2D ? b + r * kRow : packed + r * kRow;
      __builtin_nontemporal_store(v[r], (gvec*)(dst + lane_off));
    }
  }
}

// Copies a transfer's (gpu_id, cpu_id) pairs from the pinned buffer into a
// device buffer laid out [gpu ids | cpu ids], n entries each, which the
// staging kernels then read with ids_split = n.
__global__ __launch_bounds__(256) void stage_ids_kernel(const int64_t* pairs, int64_t* out,
                                                        int n) {
  const int i = blockIdx.x * 256 + static_cast<int>(threadIdx.x);
  if (i < n) {
    out[i] = pairs[2 * static_cast<int64_t>(i)];
    out[static_cast<int64_t>(n) + i] = pairs[2 * static_cast<int64_t>(i) + 1];
  }
}

// A system-scope acquire in every workgroup.  Launched with a workgroup per
// compute unit (so every XCD's L2 takes part) before a kernel reads memory
// the copy engines wrote outside any HIP stream: no stale line survives it.
__global__ __launch_bounds__(64) void acquire_system_kernel() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
}

// Small zero-copy transfers: the host cuts the call's chunks into pieces of
// at most small_piece_rows 1 KiB rows, resolves each piece's two addresses
// and passes them in the kernel arguments, indexed by workgroup.  A
// workgroup's first scalar loads fetch its piece, and its data loads follow
// at once.  The general kernel first walks its ids, layer table and tiling,
// four rounds of dependent loads from the argument segment before the first
// data load; in a kernel trace on MI355X it took 5.3 / 6.1 us (H2D / D2H) for
// one 64 KiB block row, against 3.0 us for a plain 64 KiB copy kernel.
constexpr int kSmallPieces = 128;
// 1 KiB rows per wavefront (a piece is 4 wavefronts' rows).  Measured on
// MI355X through the C-ABI, one block of 64 KiB / 16 blocks (1 MiB), one
// layer: device-to-host 2 / 4 / 8 rows 13.3 / 13.4 / 13.6 us and 34.3 / 30.7
// / 30.9 us; host-to-device 1 / 2 / 4 rows 14.4 / 14.2 / 14.4 us and (1 row:
// too many pieces, general kernel) 35.1 / 35.1 / 36.5 us.
#ifndef FKV_SMALL_U_D2H
#define FKV_SMALL_U_D2H 4
#endif
#ifndef FKV_SMALL_U_H2D
#define FKV_SMALL_U_H2D 2
#endif
// rows per wavefront and rows per piece, by direction
template <bool kH2D>
constexpr int small_rows_per_wave() { return kH2D ? FKV_SMALL_U_H2D : FKV_SMALL_U_D2H; }
template <bool kH2D>
constexpr int small_piece_rows() { return kWaves * small_rows_per_wave<kH2D>(); }
constexpr int64_t kSmallMaxBytes = int64_t(4) << 20;   // bytes moved per call

struct SmallArgs {
  uint64_t src[kSmallPieces];
  uint64_t dst[kSmallPieces];
  int32_t nvec[kSmallPieces];   // 16-byte vectors of each piece
};

// One workgroup per piece (the host launches exactly as many as there are
// pieces, at most kSmallPieces): wavefront `wave` of workgroup w takes rows
// wave + j * kWaves of piece w, j < small_rows_per_wave.  No branch sits
// between the argument loads and the data loads, so the piece's length and
// both addresses arrive in one round.
template <bool kH2D>
__global__ __launch_bounds__(kThreads) void kv_small_copy_kernel(SmallArgs a) {
  constexpr bool kNtStore = kH2D ? FKV_NT_STORE_HBM : FKV_NT_STORE_HOST;
  constexpr int kU = small_rows_per_wave<kH2D>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = blockIdx.x;
  const int n = a.nvec[w];
  const gvec* src = reinterpret_cast<const gvec*>(a.src[w]);
  gvec* dst = reinterpret_cast<gvec*>(a.dst[w]);
  // Every lane loads (past the piece's end it reloads the last vector, n >= 1),
  // so the loads carry no branch and all issue before the first wait.
  u32x4 v[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int vi = min((u * kWaves + wave) * 64 + lane, n - 1);
    v[u] = FKV_NT_LOAD ? __builtin_nontemporal_load(src + vi) : src[vi];
  }
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int vi = (u * kWaves + wave) * 64 + lane;
    if (vi < n) {
      if (kNtStore)
        __builtin_nontemporal_store(v[u], dst + vi);
      else
        dst[vi] = v[u];
    }
  }
}

std::mutex g_init_mu;

// ---------------------------------------------------------------------------
// Host-side policy of the transfer paths

// Compute units of the zero-copy kernel when the caller passes -1: enough
// loads/stores in flight to saturate the PCIe Gen5 x16 link (measured on
// MI355X: 8 CUs reach the link's copy rate; more add contention).
constexpr int kAutoZeroCopyCus = 8;
// The whole-group variant of the device-to-host zero-copy kernel fills the
// link with fewer compute units and loses rate with more (MI355X, Llama-3-8B
// shape, 2 GiB: 56.4 / 56.7 / 56.2 / 55.8 GB/s on 3 / 4 / 6 / 8 CUs, against
// 56.6 GB/s for the row-by-row variant on 8), for calls of at least
// kZeroCopyFewCusMinBytes.
constexpr int kAutoZeroCopyCusWholeD2H = 4;
// Layer-wise host-to-device transfers run beside the caller's compute.  Two
// CUs still fill the link for reads from host memory (56.9 vs 57.2 GB/s with
// 8) and leave the rest of the chip to the compute kernels: a 32-layer
// Llama-3-8B load overlapped with per-layer GEMMs finishes in 42.8 ms on 2
// CUs against 46.1 ms on 8.
constexpr int kAutoLayerwiseH2DCus = 2;
// Copy-engine size policy: smallest transfer, and smallest bytes per engine
// copy, worth handing to the SDMA engines (ce_pays_off).  Measured on MI355X
// (block-wise host caches, random ids, GB/s zero-copy kernel / engines): the
// kernel is as fast or faster up to 32 MiB in both directions at every shape
// (16 MiB of 256 KiB rows: D2H 48.9 / 46.1, H2D 53.8 / 49.5; 8 MiB of 2 MiB
// rows: 46.1 / 45.9, 50.0 / 45.8), and from 32-64 MiB the engines come
// within 1-3% (32 MiB of 2 MiB rows: D2H 53.1 / 53.5, H2D 55.2 / 53.5; 64 MiB:
// 54.8 / 55.2, 56.2 / 55.2).  Below 32 MiB the kernel holds its compute units
// for at most about 0.6 ms per transfer.
constexpr int64_t kCeMinBytesDefault = int64_t(32) << 20;
constexpr int64_t kCeMinRunBytes = int64_t(128) << 10;
// The copy-engine policy set through fkv_set_copy_engine_policy; -1: unset,
// so FLEXKV_CE_MIN_BYTES / FLEXKV_CE_RECT_COPIES, else the defaults, apply.
std::atomic<int64_t> g_ce_min_bytes{-1};
std::atomic<int> g_ce_rect_copies{-1};

int64_t ce_min_bytes() {
  const int64_t v = g_ce_min_bytes.load(std::memory_order_relaxed);
  if (v >= 0) return v;
  const char* e = getenv("FLEXKV_CE_MIN_BYTES");
  return e ? std::max<int64_t>(0, atoll(e)) : kCeMinBytesDefault;
}

// Whether a layer-wise host cache with scattered ids stays on the engines
// (rect copies) in copy-engine mode; default no (the zero-copy kernel).
bool ce_rect_copies() {
  const int v = g_ce_rect_copies.load(std::memory_order_relaxed);
  if (v >= 0) return v == 1;
  const char* r = getenv("FLEXKV_CE_RECT_COPIES");
  return r && atoi(r) == 1;
}
// The piece of a copy-engine transfer that runs without engine copies beside
// it (the first gather, the last scatter) is cut to 1 / kEdgePieceDiv of a
// staging half when it moves at least kEdgePieceMinBytes.
constexpr int kEdgePieceDiv = 8;
constexpr int64_t kEdgePieceMinBytes = int64_t(128) << 20;
// Default smallest engine copy per block of the copy-engine layer-wise
// pipeline (see layerwise_min_copy_bytes).  Measured on MI355X, Llama-3-8B
// one-layer groups (64 KiB per block), 1024 random blocks, engines 0-7:
// 37.6 / 47.2 / 50.5 / 51.1 / 51.1 GB/s with windows up to 64 KiB / 128 KiB /
// 256 KiB / 512 KiB / 1 MiB per block; per-layer GEMMs overlapped with it end
// within 0.0 / 0.5 / 0.6 / 8.3 / 8.3% of the transfer plus one layer's
// compute, and GEMMs beside it slow by the same few percent at every size.
constexpr int64_t kLayerwiseCeMinCopyBytes = int64_t(256) << 10;
// Average host run (bytes per (layer, K|V) run of consecutive blocks) from
// which a layer-wise host cache is staged layer-major and copied run by run
// instead of one rect copy per block.  Measured on MI355X at the Llama-3-8B
// shape, layer-major against rect copies (46.8 GB/s either way): runs of
// 128 KiB 41.2 / 32.4 GB/s (D2H / H2D), 256 KiB 51.1 / 42.0, 512 KiB
// 55.3 / 51.7.
constexpr int64_t kLayerRunBytes[2] = {int64_t(192) << 10, int64_t(384) << 10};   // [D2H, H2D]
// The average run from which layer-major staging is used;
// FLEXKV_CE_LAYER_RUN_BYTES overrides kLayerRunBytes.
int64_t layer_run_bytes(bool h2d) {
  const char* lr = getenv("FLEXKV_CE_LAYER_RUN_BYTES");
  return lr ? std::max<int64_t>(1, atoll(lr)) : kLayerRunBytes[h2d ? 1 : 0];
}
// transfer_staged's return when the copy engines cannot be set up (nothing
// was queued); not a hipError_t value
constexpr int kSdmaUnavailable = -1000;

template <bool H, bool I, bool W = false>
void* kernel_ptr() {
  return reinterpret_cast<void*>(&kv_chunk_copy_kernel<H, I, W>);
}

int ensure_device_basics(int dev) {
  DeviceState& d = g_dev[dev];
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (d.init) return 0;
  FKV_HIP(hipDeviceGetAttribute(&d.num_cus, hipDeviceAttributeMultiprocessorCount, dev));
  int o = 0;
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &o, reinterpret_cast<void*>(&kv_small_copy_kernel<false>), kThreads, 0));
  d.occ_small[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &o, reinterpret_cast<void*>(&kv_small_copy_kernel<true>), kThreads, 0));
  d.occ_small[1] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<false, false>(), kThreads, 0));
  d.occ_zero_copy[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<true, false>(), kThreads, 0));
  d.occ_zero_copy[1] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<false, true>(), kThreads, 0));
  d.occ_staged[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<true, true>(), kThreads, 0));
  d.occ_staged[1] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<false, true, true>(),
                                                       kThreads, 0));
  d.occ_whole[0] = std::max(1, o);
  FKV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel_ptr<true, true, true>(),
                                                       kThreads, 0));
  d.occ_whole[1] = std::max(1, o);
  d.init = true;
  return 0;
}

// Staging launches take kv_pack_kernel / kv_pack_span_kernel where their
// shape allows (1), or the row-by-row / whole-group kv_chunk_copy_kernel
// throughout (0).
#ifndef FKV_PACK_KERNEL
#define FKV_PACK_KERNEL 1
#endif

// Staging kernels read their tile's ids from a device copy of the pairs
// (stage_ids_on_device) rather than the pinned buffer: every workgroup of a
// staging launch starts with that read, and over PCIe it costs a host round
// trip per tile.
#ifndef FKV_STAGE_IDS_ON_DEVICE
#define FKV_STAGE_IDS_ON_DEVICE 1
#endif

// Queue a copy of the n pairs in `ids` (pinned) into a device buffer held by
// `lease`, on `stream`, and describe it in `out` (the pinned pairs stay its
// host side, for launches that take their ids inline) with `split` = n.
// Without FKV_STAGE_IDS_ON_DEVICE, `out` is `ids` and `split` 0.
int stage_ids_on_device(const IdBuf& ids, int n, int dev, hipStream_t stream, DevIdLease& lease,
                        IdBuf* out, int32_t* split) {
  *out = ids;
  *split = 0;
  if (!FKV_STAGE_IDS_ON_DEVICE || n <= 0) return 0;
  lease.dev = dev;
  int rc = dev_ids_acquire(dev, static_cast<size_t>(n) * 16, &lease.buf);
  if (rc) return rc;
  (void)hipGetLastError();  // a stale error from elsewhere must not be blamed on this launch
  hipLaunchKernelGGL(stage_ids_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                     reinterpret_cast<const int64_t*>(ids.dev),
                     reinterpret_cast<int64_t*>(lease.buf.dev), n);
  FKV_HIP(hipGetLastError());
  out->dev = lease.buf.dev;
  *split = n;
  return 0;
}

// Tiles are tb blocks x tl layers.  Start from whole block rows (one block,
// every layer) and halve the layer window until there are about `factor`
// tiles per occupancy slot of the grid; when blocks are plentiful, group
// several per tile so one LDS id load serves more rows.  Rows per tile stay
// below 2^31.  Measured on MI355X (2 GiB gather at the Llama-3-8B shape):
// 32 rows in flight per wavefront with one workgroup per tile and 16 tiles
// per slot is the best shape (6.0 TB/s with whole-group addressing; 4 and 8
// tiles per slot 5.93 / 6.00, 32 tiles 5.44).
//
// `balanced` (the HBM-bound staging kernels): a workgroup's wavefronts take
// the tile's unrolled row groups in turn, so a tile whose rows are not a
// multiple of kWaves * unroll leaves some wavefronts idle while the others
// finish (a one-layer Llama-3-8B tile, 64 rows, keeps two of four busy; a
// one-layer MLA tile, 72 rows, fills 56% of the group slots).  The layer
// window is then halved only while that fill does not drop, and row ranges
// (below) are whole multiples of kWaves * unroll.  Measured on MI355X, 128 MiB
// launches: Llama-3-8B gather 5.08 -> 5.40 TB/s, 70B-shard (4 KiB chunks)
// gather 2.39 -> 3.66 TB/s.
//
// A transfer too small for that many tiles even one (block, layer) per tile
// splits each tile's rows into up to `factor`-filling ranges of at least one
// `unroll`-row group per wavefront, so more wavefronts share its few chunks:
// one block of one layer moves in one round of loads instead of several
// (zero-copy latency is bound by PCIe round trips).
void choose_tiles(int nb, int nl, int kv, int rpc, int grid_cap, int factor, int unroll,
                  bool balanced, CopyArgs* a) {
  const int64_t target = factor * static_cast<int64_t>(std::max(1, grid_cap));
  auto tiles = [&](int tb, int tl) {
    return static_cast<int64_t>((nb + tb - 1) / tb) * ((nl + tl - 1) / tl);
  };
  auto rows_of = [&](int tb_, int tl_) { return static_cast<int64_t>(tb_) * tl_ * kv * rpc; };
  const int64_t wave_groups = static_cast<int64_t>(unroll) * kWaves;   // rows of one round
  // rows of a tile over the row slots its wavefronts' rounds provide
  auto fill_below = [&](int64_t ra, int64_t rb) {   // fill(ra) < fill(rb)
    const int64_t ca = (ra + wave_groups - 1) / wave_groups * wave_groups;
    const int64_t cb = (rb + wave_groups - 1) / wave_groups * wave_groups;
    return static_cast<__int128>(ra) * cb < static_cast<__int128>(rb) * ca;
  };
  int tb = 1, tl = nl;
  while (tl > 1 && tiles(tb, tl) < target) {
    const int half = (tl + 1) / 2;
    if (balanced && fill_below(rows_of(tb, half), rows_of(tb, tl))) break;
    tl = half;
  }
  while (tb < kMaxTileBlocks && tiles(tb * 2, tl) >= target) tb *= 2;
  while (tb > 1 && static_cast<int64_t>(tb) * tl * kv * rpc >= (int64_t(1) << 31)) tb /= 2;
  while (tl > 1 && static_cast<int64_t>(tb) * tl * kv * rpc >= (int64_t(1) << 31)) tl = (tl + 1) / 2;
  const int64_t t = tiles(tb, tl);
  const int64_t tile_rows = static_cast<int64_t>(tb) * tl * kv * rpc;
  int64_t tr = 1, split = tile_rows;
  if (t < target) {
    const int64_t min_split = wave_groups;
    const int64_t quantum = balanced ? wave_groups : unroll;
    tr = std::min<int64_t>(std::max<int64_t>(1, tile_rows / min_split), (target + t - 1) / t);
    split = ((tile_rows + tr - 1) / tr + quantum - 1) / quantum * quantum;
    tr = (tile_rows + split - 1) / split;
  }
  a->tile_blocks = tb;
  a->tile_layers = tl;
  a->tiles_b = (nb + tb - 1) / tb;
  a->tiles_l = (nl + tl - 1) / tl;
  a->tiles_r = static_cast<int32_t>(tr);
  a->split_rows = static_cast<uint32_t>(split);
  a->num_tiles = static_cast<int32_t>(t * tr);
}

int64_t op_bytes(const Geometry& g) {
  return static_cast<int64_t>(g.num_blocks) * g.num_layers * g.kv * g.chunk;
}

// Whether the zero-copy launches of a transfer take the whole-group kernel
// variant (launch_copy: full 1 KiB rows, chunks of whole sub-groups).
// Host-to-device calls under kZeroCopyWholeH2DMinBytes keep the row-by-row
// variant, which measured faster on short calls and slower on long ones
// (MI355X, Llama-3-8B chunks, kernel mode, whole-group against row by row:
// 1 block, 2 MiB, 34.4-34.6 against 35.6-36.1 GB/s; 16 blocks x 1 layer,
// 36.2-36.7 against 34.5-34.7 us per call; 16 MiB equal; 64 MiB 56.33
// against 56.21-56.22 GB/s; 2 GiB 57.34-57.35 against 57.19-57.20).
constexpr int64_t kZeroCopyWholeH2DMinBytes = int64_t(32) << 20;
bool zero_copy_whole(const Geometry& g, bool h2d) {
  const int64_t sub_rows = h2d ? FKV_UNROLL_ZC_H2D / whole_sub_groups<true, false>()
                               : FKV_UNROLL_ZC_D2H / whole_sub_groups<false, false>();
  return FKV_WHOLE_ZERO_COPY && g.chunk % (64 * 16) == 0 &&
         (g.chunk / (64 * 16)) % sub_rows == 0 &&
         (!h2d || op_bytes(g) >= kZeroCopyWholeH2DMinBytes);
}

// Compute units of a zero-copy transfer when the caller passes -1.
// The whole-group device-to-host kernel's fewer compute units pay from this
// many bytes per call; below it the ramp of a short call wants more (MI355X,
// 4 / 8 / 16 CUs: 16 MiB ops 51.3 / 52.1 / 52.8 GB/s, 32 MiB 53.6 / 53.9 /
// 53.9, 2 GiB 56.7 / 55.6 / 55.2).
constexpr int64_t kZeroCopyFewCusMinBytes = int64_t(64) << 20;
int auto_zero_copy_cus(const Geometry& g, bool h2d) {
  return !h2d && zero_copy_whole(g, h2d) && op_bytes(g) >= kZeroCopyFewCusMinBytes
             ? kAutoZeroCopyCusWholeD2H
             : kAutoZeroCopyCus;
}

// The packed-row kernel for a staging launch of chunks of `rpc` full rows:
// kv_pack_kernel<kU, kC>, kv_pack_span_kernel ({32, 0}), or {0, 0} when the
// row-by-row or whole-group kv_chunk_copy_kernel takes it.
struct PackShape {
  int u = 0, c = 0;
};
// Measured on MI355X (HBM TB/s, interleaved A/B in one process):
// - chunks of whole 32-row groups (32 KiB, 64 KiB, ...): gathers keep the
//   tiled whole-group kernel (Llama-3-8B, 2 GiB: 6.07-6.10 against 6.01-6.08
//   for 32-row span groups); scatters take the span kernel (5.53-5.54 against
//   5.47-5.50; the copy-engine path's pieces 0.628 -> 0.650 of 8 TB/s);
// - longer chunks that are not (MLA's 72 rows): 32-row span groups gather
//   6.15-6.20 and scatter 5.70 against 5.60-5.62 and 5.48-5.49 for 36-row
//   kv_pack_kernel groups (pieces: gather 0.695 -> 0.731, scatter 0.665 ->
//   0.682);
// - 4-16 KiB chunks: groups of 32 / rpc whole chunks;
// - other chunks of 8-31 rows: span groups with 3-5 bases (DeepSeek MLA at
//   16 tokens per block, 18 KiB chunks: gather 6.03-6.07 and scatter
//   5.41-5.43 against 5.48-5.49 and 5.14-5.15 for the two-walk kernel;
//   pieces 0.656 -> 0.712 and 0.614 -> 0.644).
PackShape pack_shape(int64_t rpc, int64_t chunks, bool h2d) {
  if (rpc % 32 == 0) return h2d ? PackShape{32, 0} : PackShape{};
  if (rpc > 32) return {32, 0};
  for (int c : {2, 4, 8})
    if (rpc * c == 32 && chunks % c == 0) return {32, c};
  if (rpc == 24) return {24, 1};
  if (rpc >= 8) return {32, 0};
  return {};
}

// Chunks a 32-row span group can touch with chunks of `rpc` rows (rpc >= 8).
int span_bases(int64_t rpc) { return 2 + static_cast<int>(30 / rpc); }

// Dynamic LDS (unused by the kernels) that holds the span kernel and the
// 24-row variant to one workgroup per compute unit.  Measured on MI355X,
// capped / uncapped HBM TB/s: span groups gather 6.15-6.20 / 5.94-5.96 (MLA)
// and 6.01-6.08 / 5.77-5.83 (Llama-3-8B), scatter 5.70-5.71 / 5.61-5.65 and
// 5.53-5.54 / 5.37-5.43; two workgroups per CU (64 KiB) fall between; 24-row
// groups gather 5.53 / 5.47.  The 4-16 KiB chunk groups gain nothing from it
// (the Llama-3-70B TP-8 shard: gather 5.92-5.98 / 5.96-6.02, scatter 5.29 /
// 5.24-5.28).
constexpr unsigned kPackLdsOneGroup = 84 << 10;

// Launch kv_pack_kernel<kH2D, kU, kC> over the launch's groups.
template <bool kH2D, int kU, int kC>
void launch_pack(const PackArgs& pa, hipStream_t stream, hipEvent_t ea, hipEvent_t eb) {
  const uint32_t grid = (pa.num_groups + kWaves - 1) / kWaves;
  hipExtLaunchKernelGGL((kv_pack_kernel<kH2D, kU, kC>), dim3(grid), dim3(kThreads),
                        kU != 32 ? kPackLdsOneGroup : 0u, stream, ea, eb, 0, pa);
}

// Launch kv_pack_span_kernel<kH2D, kB> over the launch's groups.
template <bool kH2D, int kB>
void launch_pack_span(const PackArgs& pa, hipStream_t stream, hipEvent_t ea, hipEvent_t eb) {
  const uint32_t grid = (pa.num_groups + kWaves - 1) / kWaves;
  hipExtLaunchKernelGGL((kv_pack_span_kernel<kH2D, kB>), dim3(grid), dim3(kThreads),
                        kPackLdsOneGroup, stream, ea, eb, 0, pa);
}

// Fill the per-launch part of CopyArgs and launch over `nb` blocks starting at
// block `b0` of the (already packed) id list, for GPU layers [l0, l0 + nl).
// `cpu_base` is the CPU-side address of launch layer 0 of block index 0.
// `ids` holds the packed pairs: `host` for the host's view, `dev` for the
// device's (the same pinned buffer).  With `split` > 0, `dev` instead holds
// the gpu ids and, `split` entries later, the cpu ids (device memory), and
// `host` is null.  `grid_cap` is compute units x occupancy of the kernel the
// launch takes; staging launches that take the whole-group variant use
// `whole_grid_cap` instead when it is given.
template <bool kH2D, bool kIota>
int launch_copy(const Geometry& g, const IdBuf& ids, char* cpu_base, int64_t cks, int64_t cls,
                int64_t cbs, int b0, int nb, int l0, int nl, int grid_cap,
                hipStream_t stream, ProfRecorder& prof, int32_t split = 0,
                int whole_grid_cap = 0) {
  if (nl < 1 || static_cast<int64_t>(nl) * g.ptrs_per_layer > kMaxLayersPerLaunch)
    return fail(kInval, "internal: a launch of %d layers exceeds the %d layer pointers of the "
                "kernel arguments", nl, kMaxLayersPerLaunch / g.ptrs_per_layer);
  // Staging launches whose packed side is contiguous in row order, with full
  // rows and ids in device memory, take kv_pack_kernel or kv_pack_span_kernel
  // where pack_shape says so.
  if constexpr (kIota) {
    const int64_t rpc = g.chunk / (64 * 16);
    const bool packed_rows = FKV_PACK_KERNEL && split > 0 && g.chunk % (64 * 16) == 0 &&
                             (g.kv == 1 || cks == g.chunk) && cls == g.kv * g.chunk &&
                             cbs == static_cast<int64_t>(nl) * cls;
    const int64_t chunks = static_cast<int64_t>(nb) * nl * g.kv;
    const PackShape shape = packed_rows ? pack_shape(rpc, chunks, kH2D) : PackShape{};
    if (shape.u > 0 && chunks * rpc + shape.u <= UINT32_MAX) {
      PackArgs pa;
      memset(&pa, 0, sizeof(pa));
      pa.gids = reinterpret_cast<const int64_t*>(ids.dev) + b0;
      pa.packed = cpu_base;
      pa.gpu_kv_stride = g.gks;
      pa.gpu_block_stride = g.gbs;
      pa.rows_per_chunk = static_cast<uint32_t>(rpc);
      pa.items_per_block = static_cast<uint32_t>(nl * g.kv);
      pa.kv_dim = static_cast<uint32_t>(g.kv);
      pa.num_layers = static_cast<uint32_t>(nl);
      pa.num_rows = static_cast<uint32_t>(chunks * rpc);
      pa.num_groups = (pa.num_rows + shape.u - 1) / shape.u;   // whole groups but for span launches
      pa.ptrs_per_layer = g.ptrs_per_layer;
      for (int i = 0; i < nl * g.ptrs_per_layer; ++i)
        pa.layer_ptr[i] = reinterpret_cast<uint64_t>(g.layer_ptrs[l0 * g.ptrs_per_layer + i]);
      hipEvent_t ea = nullptr, eb = nullptr;
      int rc = prof.kernel_events(&ea, &eb);
      if (rc) return rc;
      prof.kernel_span(ea, eb, chunks * g.chunk);   // owns the events from here on
      (void)hipGetLastError();  // a stale error from elsewhere must not be blamed on this launch
      switch (shape.u * 16 + shape.c) {
        case 32 * 16 + 2: launch_pack<kH2D, 32, 2>(pa, stream, ea, eb); break;
        case 32 * 16 + 4: launch_pack<kH2D, 32, 4>(pa, stream, ea, eb); break;
        case 32 * 16 + 8: launch_pack<kH2D, 32, 8>(pa, stream, ea, eb); break;
        case 24 * 16 + 1: launch_pack<kH2D, 24, 1>(pa, stream, ea, eb); break;
        default:
          switch (span_bases(rpc)) {
            case 2: launch_pack_span<kH2D, 2>(pa, stream, ea, eb); break;
            case 3: launch_pack_span<kH2D, 3>(pa, stream, ea, eb); break;
            case 4: launch_pack_span<kH2D, 4>(pa, stream, ea, eb); break;
            default: launch_pack_span<kH2D, 5>(pa, stream, ea, eb); break;
          }
          break;
      }
      FKV_HIP(hipGetLastError());
      return 0;
    }
  }
  CopyArgs a;
  memset(&a, 0, sizeof(a));
  a.ids = reinterpret_cast<const int64_t*>(ids.dev) + (split ? 1 : 2) * static_cast<int64_t>(b0);
  a.ids_split = split;
  if (nb <= kInlineIds && ids.host) {
    a.inline_n = nb;
    memcpy(a.inline_ids, ids.host + 2 * static_cast<int64_t>(b0), sizeof(int64_t) * 2 * nb);
  }
  a.cpu_base = cpu_base;
  a.gpu_kv_stride = g.gks;
  a.gpu_block_stride = g.gbs;
  a.cpu_kv_stride = cks;
  a.cpu_layer_stride = cls;
  a.cpu_block_stride = cbs;
  a.chunk_vec = g.chunk / 16;
  a.rows_per_chunk = static_cast<int32_t>((a.chunk_vec + 63) / 64);
  a.num_blocks = nb;
  a.num_layers = nl;
  a.kv_dim = g.kv;
  a.ptrs_per_layer = g.ptrs_per_layer;
  for (int i = 0; i < nl * g.ptrs_per_layer; ++i)
    a.layer_ptr[i] = reinterpret_cast<uint64_t>(g.layer_ptrs[l0 * g.ptrs_per_layer + i]);
  constexpr int kLaunchUnroll = kIota ? (kH2D ? FKV_UNROLL_SCATTER : kUnrollHbm)
                                     : (kH2D ? FKV_UNROLL_ZC_H2D : FKV_UNROLL_ZC_D2H);
  // staging launches whose chunks are whole groups of full rows take the
  // kernel variant that addresses each group from one base; its occupancy
  // sizes the tiling
  constexpr int kStagedUnroll = kH2D ? FKV_UNROLL_SCATTER : kUnrollHbm;
  const bool whole_variant =
      kH2D ? (FKV_WHOLE_SCATTER &&
              static_cast<int64_t>(nb) * nl * g.kv * g.chunk <= kWholeScatterMaxBytes)
           : FKV_WHOLE_GATHER;
  // zero-copy launches whose chunks are whole groups of the launch's unroll
  // take it too (FKV_WHOLE_ZERO_COPY)
  const bool whole = kIota ? a.chunk_vec % 64 == 0 && whole_variant &&
                                 a.rows_per_chunk % kStagedUnroll == 0
                           : zero_copy_whole(g, kH2D);
  if (whole && whole_grid_cap > 0) grid_cap = whole_grid_cap;
  choose_tiles(nb, nl, g.kv, a.rows_per_chunk, grid_cap,
               kIota ? (kH2D ? FKV_TILE_FACTOR_SCATTER : FKV_TILE_FACTOR_HBM) : FKV_TILE_FACTOR,
               kLaunchUnroll, /*balanced=*/kIota, &a);
  a.block_major = kIota && (kH2D ? FKV_BLOCK_MAJOR_SCATTER : FKV_BLOCK_MAJOR_GATHER);
  int grid = std::max(1, std::min(grid_cap, a.num_tiles));
  if (kIota && FKV_HBM_ONEPASS) grid = a.num_tiles;
  hipEvent_t ea = nullptr, eb = nullptr;
  int rc = prof.kernel_events(&ea, &eb);
  if (rc) return rc;
  prof.kernel_span(ea, eb, static_cast<int64_t>(nb) * nl * g.kv * g.chunk);
  (void)hipGetLastError();  // a stale error from elsewhere must not be blamed on this launch
  const unsigned lds = kIota ? FKV_HBM_LDS_PAD : 0;
  if (whole)
    hipExtLaunchKernelGGL((kv_chunk_copy_kernel<kH2D, kIota, true>), dim3(grid), dim3(kThreads),
                          lds, stream, ea, eb, 0, a);
  else
    hipExtLaunchKernelGGL((kv_chunk_copy_kernel<kH2D, kIota>), dim3(grid), dim3(kThreads), lds,
                          stream, ea, eb, 0, a);
  FKV_HIP(hipGetLastError());
  return 0;
}

// Pieces a call takes in kv_small_copy_kernel when it fits (at most
// kSmallPieces pieces, kSmallMaxBytes, and one workgroup per piece within
// the call's `grid_cap` workgroups), else 0.  FLEXKV_SMALL_KERNEL=0 sends
// every call to the general kernel.
int small_pieces(const Geometry& g, int grid_cap, bool h2d) {
  if (const char* e = getenv("FLEXKV_SMALL_KERNEL"))
    if (atoi(e) == 0) return 0;
  const int64_t chunks = static_cast<int64_t>(g.num_blocks) * g.num_layers * g.kv;
  if (chunks < 1 || chunks > kSmallPieces || chunks * g.chunk > kSmallMaxBytes) return 0;
  const int64_t piece_bytes =
      int64_t(h2d ? small_piece_rows<true>() : small_piece_rows<false>()) * 64 * 16;
  const int64_t n = chunks * ((g.chunk + piece_bytes - 1) / piece_bytes);
  return n > std::min(kSmallPieces, grid_cap) ? 0 : static_cast<int>(n);
}

// One launch of kv_small_copy_kernel over the whole call.  `cpu_dev` is the
// device-visible address of the host cache at call layer 0 (start layer and
// start offset applied).  Chunk sizes are multiples of 16 bytes here.
template <bool kH2D>
int transfer_small(const Geometry& g, char* cpu_dev, int n_pieces, hipStream_t stream,
                   ProfRecorder& prof) {
  SmallArgs a;
  const int64_t piece_bytes = int64_t(small_piece_rows<kH2D>()) * 64 * 16;
  int p = 0;
  for (int l = 0; l < g.num_layers; ++l)
    for (int k = 0; k < g.kv; ++k)
      for (int i = 0; i < g.num_blocks; ++i) {
        char* gpu = g.gpu_base(l, k) + g.gids[i] * g.gbs;
        char* cpu = cpu_dev + static_cast<int64_t>(l) * g.cls + k * g.cks + g.cids[i] * g.cbs;
        for (int64_t off = 0; off < g.chunk; off += piece_bytes, ++p) {
          a.src[p] = reinterpret_cast<uint64_t>((kH2D ? cpu : gpu) + off);
          a.dst[p] = reinterpret_cast<uint64_t>((kH2D ? gpu : cpu) + off);
          a.nvec[p] = static_cast<int32_t>(std::min(piece_bytes, g.chunk - off) / 16);
        }
      }
  if (p != n_pieces) return fail(kInval, "internal: %d small-transfer pieces, expected %d", p,
                                 n_pieces);
  hipEvent_t ea = nullptr, eb = nullptr;
  int rc = prof.kernel_events(&ea, &eb);
  if (rc) return rc;
  prof.kernel_span(ea, eb, op_bytes(g));
  (void)hipGetLastError();  // a stale error from elsewhere must not be blamed on this launch
  hipExtLaunchKernelGGL(kv_small_copy_kernel<kH2D>, dim3(n_pieces), dim3(kThreads), 0, stream,
                        ea, eb, 0, a);
  FKV_HIP(hipGetLastError());
  return 0;
}

int transfer_zero_copy(const Geometry& g, hipStream_t stream, int dev, int transfer_cus,
                       bool h2d) {
  DeviceState& d = g_dev[dev];
  const int small_cus = transfer_cus <= 0 ? std::min(kAutoZeroCopyCus, d.num_cus)
                                          : std::min(transfer_cus, d.num_cus);
  if (const int n = small_pieces(g, small_cus * (h2d ? d.occ_small[1] : d.occ_small[0]), h2d)) {
    DrainOnError drain{stream};
    char* cpu_dev = g.cpu_info.dev_ptr + g.startoff +
                    static_cast<int64_t>(g.start_layer) * g.cls;
    ProfRecorder prof;
    const int rc = h2d ? transfer_small<true>(g, cpu_dev, n, stream, prof)
                       : transfer_small<false>(g, cpu_dev, n, stream, prof);
    if (rc) return rc;
    FKV_HIP(hipStreamSynchronize(stream));
    drain.armed = false;
    prof.flush();
    return 0;
  }
  IdLease ids;
  int rc = pack_ids(g, ids);
  if (rc) return rc;
  DrainOnError drain{stream};
  int cus = transfer_cus <= 0 ? std::min(auto_zero_copy_cus(g, h2d), d.num_cus)
                              : std::min(transfer_cus, d.num_cus);
  const int grid_cap = cus * (h2d ? d.occ_zero_copy[1] : d.occ_zero_copy[0]);
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff +
                  static_cast<int64_t>(g.start_layer) * g.cls;
  ProfRecorder prof;
  const int per_launch = g.layers_per_launch();
  for (int l0 = 0; l0 < g.num_layers; l0 += per_launch) {
    const int nl = std::min(per_launch, g.num_layers - l0);
    char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
    rc = h2d ? launch_copy<true, false>(g, ids.buf, base, g.cks, g.cls, g.cbs, 0,
                                        g.num_blocks, l0, nl, grid_cap, stream, prof)
             : launch_copy<false, false>(g, ids.buf, base, g.cks, g.cls, g.cbs, 0,
                                         g.num_blocks, l0, nl, grid_cap, stream, prof);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

// ---------------------------------------------------------------------------
// The entry point that allocates nothing (fkv_transfer_kv_blocks_noalloc):
// the zero-copy transfer with its id lists staged in `scratch`, a fixed
// device array, instead of a pinned buffer the library allocates.  Each GPU
// holds its own copy of the array; host code reaches it only through the
// address hipGetSymbolAddress returns for the device (the array's name is a
// host-side stand-in, not a device address).  Every call on a device shares
// that device's array, so a call holds the device's scratch mutex from the
// copy of its ids into the array until its kernels have finished: calls
// from several threads on one device take turns instead of racing.

constexpr size_t kScratchBytes = size_t(1) << 20;
// gpu ids in the first half, cpu ids in the second
constexpr int kScratchMaxBlocks = static_cast<int>(kScratchBytes / (2 * sizeof(int64_t)));

static __device__ __align__(256) int64_t scratch[kScratchBytes / sizeof(int64_t)];

std::mutex g_scratch_mu;
int64_t* g_scratch_dev[kMaxDevices];   // scratch's address on each device, once resolved
// held by a call from its scratch copy until its stream is synchronised
std::mutex g_scratch_use_mu[kMaxDevices];

// scratch's device address on `dev` (resolved once per device, with the
// device current).
int scratch_address(int dev, int64_t** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    DeviceGuard guard;
    int rc = guard.set(dev);
    if (rc) return rc;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(static_cast<int>(e == hipSuccess ? hipErrorInvalidSymbol : e),
                  "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<int64_t*>(p);
  }
  *out = g_scratch_dev[dev];
  return 0;
}

int transfer_zero_copy_noalloc(const Geometry& g, hipStream_t stream, int dev, int transfer_cus,
                               bool h2d) {
  DeviceState& d = g_dev[dev];
  if (g.num_blocks > kScratchMaxBlocks)
    return fail(kInval, "fkv_transfer_kv_blocks_noalloc moves at most %d blocks per call "
                "(its id scratch is %zu bytes), got %d", kScratchMaxBlocks, kScratchBytes,
                g.num_blocks);
  const int small_cus = transfer_cus <= 0 ? std::min(kAutoZeroCopyCus, d.num_cus)
                                          : std::min(transfer_cus, d.num_cus);
  if (const int n = small_pieces(g, small_cus * (h2d ? d.occ_small[1] : d.occ_small[0]), h2d)) {
    DrainOnError drain{stream};
    char* cpu_dev = g.cpu_info.dev_ptr + g.startoff + static_cast<int64_t>(g.start_layer) * g.cls;
    ProfRecorder prof;
    prof.on = false;   // profiling events are allocations
    const int rc = h2d ? transfer_small<true>(g, cpu_dev, n, stream, prof)
                       : transfer_small<false>(g, cpu_dev, n, stream, prof);
    if (rc) return rc;
    FKV_HIP(hipStreamSynchronize(stream));
    drain.armed = false;
    return 0;
  }
  int64_t pairs[2 * kInlineIds];
  IdBuf ids;
  int32_t split = 0;
  // Declared before the DrainOnError below, so an error path drains the
  // stream before the next call may overwrite the scratch.
  std::unique_lock<std::mutex> scratch_use(g_scratch_use_mu[dev], std::defer_lock);
  if (g.num_blocks <= kInlineIds) {
    // the ids travel in the kernel arguments
    pack_ids_into(g, pairs);
    ids.host = pairs;
  } else {
    int64_t* sp = nullptr;
    int rc = scratch_address(dev, &sp);
    if (rc) return rc;
    scratch_use.lock();
    const size_t n = static_cast<size_t>(g.num_blocks) * sizeof(int64_t);
    DrainOnError copy_drain{stream};   // a failed second copy still waits for the first
    FKV_HIP(hipMemcpyAsync(sp, g.gids, n, hipMemcpyHostToDevice, stream));
    FKV_HIP(hipMemcpyAsync(sp + kScratchMaxBlocks, g.cids, n, hipMemcpyHostToDevice, stream));
    copy_drain.armed = false;
    ids.dev = reinterpret_cast<char*>(sp);
    split = kScratchMaxBlocks;
  }
  DrainOnError drain{stream};
  const int cus = transfer_cus <= 0 ? std::min(auto_zero_copy_cus(g, h2d), d.num_cus)
                                    : std::min(transfer_cus, d.num_cus);
  const int grid_cap = cus * (h2d ? d.occ_zero_copy[1] : d.occ_zero_copy[0]);
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff + static_cast<int64_t>(g.start_layer) * g.cls;
  ProfRecorder prof;
  prof.on = false;   // profiling events are allocations
  const int per_launch = g.layers_per_launch();
  for (int l0 = 0; l0 < g.num_layers; l0 += per_launch) {
    const int nl = std::min(per_launch, g.num_layers - l0);
    char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
    const int rc = h2d ? launch_copy<true, false>(g, ids, base, g.cks, g.cls, g.cbs, 0,
                                                  g.num_blocks, l0, nl, grid_cap, stream, prof,
                                                  split)
                       : launch_copy<false, false>(g, ids, base, g.cks, g.cls, g.cbs, 0,
                                                   g.num_blocks, l0, nl, grid_cap, stream, prof,
                                                   split);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  return 0;
}

// Copy-engine transfer: the SDMA engines move whole-block runs between the
// host cache and double-buffered HBM staging; a gather (D2H) or scatter
// (H2D) kernel on the caller's stream moves them between staging and the
// per-layer cache.  The host thread orders the two, so no compute unit
// takes part in the PCIe copies.
//  D2H, per piece: wait for the half's previous copies -> gather kernel ->
//  wait for it -> queue the half's copies.
//  H2D: queue the copies of the first two pieces; per piece: wait for its
//  copies -> system-scope acquire -> scatter kernel; once that has read the
//  half, queue the copies of the piece two ahead into it.
// fkv_prepare: polled completion signals it creates per staging half (one
// per block of a 1024-block layer-wise window; the pools grow on demand),
// and the pinned host buffer of its warm-up copies (4 KiB per engine).
constexpr size_t kPrepareSignalsPerHalf = 1024;
constexpr size_t kPrepareHostBytes = size_t(64) << 10;

// Staging for a copy-engine transfer (ensure_staging): 0; kSdmaUnavailable
// when the device has no memory left for it, so the transfer moves with the
// zero-copy kernel instead (warned once per device; later transfers try the
// allocation again); or another error.
int staging_or_fallback(DeviceState& d, int dev, CopyLane& ln, size_t need_half) {
  const int rc = ensure_staging(ln, need_half);
  if (rc != static_cast<int>(hipErrorOutOfMemory)) return rc;
  (void)hipGetLastError();
  if (!d.staging_oom_warned.exchange(true))
    fprintf(stderr, "flexkv: no device memory for copy-engine staging on device %d (%s); "
            "such transfers use the zero-copy kernel until the allocation succeeds\n", dev,
            last_error().c_str());
  last_error().clear();
  return kSdmaUnavailable;
}

// Edge pieces below kEdgePieceMinBytes: one of at least edge_small_min_bytes()
// (FLEXKV_CE_EDGE_MIN_BYTES, default 32 MiB) gives 1 / kEdgeSmallDiv of its
// blocks to a piece of its own.  Measured on MI355X, Llama-3-8B block rows
// (2 MiB), copy-engine transfers with / without the cut: 16 blocks 628.8 /
// 631.5 us D2H, 627.3 / 637.9 us H2D; 32 blocks 1216 / 1236 us D2H, 1214 /
// 1237 us H2D; 4 blocks (8 MiB) 181 / 183 us D2H but 198 / 183 us H2D, where
// the extra piece's host round trip is not hidden behind 2 MiB of copies.
constexpr int kEdgeSmallDiv = 4;
constexpr int64_t kEdgeSmallMinBytesDefault = int64_t(32) << 20;

int64_t edge_small_min_bytes() {
  const char* e = getenv("FLEXKV_CE_EDGE_MIN_BYTES");
  return e ? std::max<int64_t>(1, atoll(e)) : kEdgeSmallMinBytesDefault;
}

// Host-to-device engine copies shorter than this on average spread over the
// synchronous wide set (engines 0-5) instead of the direction's four (0-3).
// Measured on MI355X: 256 KiB copies 51.7 GB/s on 0-3, 56.1 on 0-5; 640 KiB
// copies (Llama-3-70B TP-8 shard) 57.0 on 0-3, 56.4 on 0-5.  While a D2H is
// in flight, host-to-device copies of any size take the duplex split
// instead (issue_sdma).
constexpr int64_t kWideCopyBytes = int64_t(384) << 10;
// Host-to-device copies on the wide set run beside the scatter of the
// previous piece, and every engine in flight slows that scatter (MI355X,
// Llama-3-70B TP-8 shard, 640 KiB copies: 512 MiB scatter pieces 4.26 /
// 4.65 / 4.90 TB/s beside 8 / 6 / 4 engines).  So the engines of the set
// beyond the first kHoldKeepEngines take their share of a piece only once
// that scatter is done (issue_sdma, SdmaHold).  held_fraction is the
// scatter's expected time, plus the host's wake-up, over the piece's time on
// the link; FLEXKV_SDMA_HOLD_SCALE scales it (0: no engine is held).
double held_fraction(int64_t prev_piece_bytes, int64_t piece_bytes) {
  const char* e = getenv("FLEXKV_SDMA_HOLD_SCALE");
  const double scale = e ? std::max(0.0, atof(e)) : 1.0;
  if (scale <= 0 || piece_bytes <= 0) return 0.0;
  constexpr double kScatterBytesPerS = 4.9e12;   // HBM bytes, read + write
  constexpr double kLinkBytesPerS = 56e9;
  constexpr double kWakeS = 20e-6;
  const double d = 2.0 * static_cast<double>(prev_piece_bytes) / kScatterBytesPerS + kWakeS;
  return scale * d / (static_cast<double>(piece_bytes) / kLinkBytesPerS);
}

int transfer_staged(const Geometry& g, hipStream_t stream, int dev, bool h2d) {
  DeviceState& d = g_dev[dev];
  CopyLane& ln = d.lane[h2d ? 1 : 0];
  // Staging order: block-major [block][layer][K|V][chunk] (contiguous block
  // rows, or one rect copy per block of a layer-wise cache), or layer-major
  // [layer][K|V][block][chunk] when a layer-wise cache's ids come in runs of
  // consecutive blocks long enough to copy each (layer, K|V) run linearly.
  const bool layer_major = layer_major_pays_off(g, layer_run_bytes(h2d));
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) &&
                          (g.num_layers == 1 || g.cls == g.kv * g.chunk);
  // A transfer of rect copies runs alone on the device: those go to the
  // engine the runtime picks, and the runtime must not see them beside copies
  // pinned to engines.  Other transfers hold their direction's lane only.
  const bool rect_copies = !row_contig && !layer_major;
  std::unique_lock<std::mutex> own(ln.mu, std::defer_lock);
  std::unique_lock<std::mutex> other(d.lane[h2d ? 0 : 1].mu, std::defer_lock);
  if (rect_copies)
    std::lock(own, other);
  else
    own.lock();
  BusyMark busy(d.busy[h2d ? 1 : 0]);
  DeviceGuard guard;
  int rc = guard.set(dev);
  if (rc) return rc;
  IdLease ids;
  rc = pack_ids(g, ids);
  if (rc) return rc;
  DevIdLease dev_ids;   // released after the drain below
  IdBuf kids;           // the ids the staging kernels read
  int32_t kids_split = 0;

  // A piece is a run of whole blocks over a layer window; the window covers
  // all layers unless one block row would not fit a staging half.
  const size_t req = g_staging_request.load();
  const size_t half_default = (req ? req : kDefaultStagingBytes) / 2;
  int nl_piece = std::min(g.num_layers, g.layers_per_launch());
  while (nl_piece > 1 && static_cast<size_t>(nl_piece) * g.kv * g.chunk > half_default) nl_piece /= 2;
  const size_t row_bytes = static_cast<size_t>(nl_piece) * g.kv * g.chunk;
  rc = staging_or_fallback(d, dev, ln, row_bytes);
  if (rc) return rc;   // kSdmaUnavailable: the caller moves it with the zero-copy kernel
  if ((rc = ensure_sdma(d, dev, ln.staging))) {
    // nothing has been queued yet: the caller moves this transfer, and every
    // later one on the device, with the zero-copy kernel
    if (!d.sdma_failed.exchange(true))
      fprintf(stderr, "flexkv: copy engines unavailable on device %d (%s); copy-engine "
              "transfers use the zero-copy kernel\n", dev, last_error().c_str());
    last_error().clear();
    return kSdmaUnavailable;
  }
  const size_t half = ln.staging_bytes / 2;
  const int blocks_per_piece = static_cast<int>(std::max<size_t>(1, half / row_bytes));
  const int grid_cap = d.num_cus * (h2d ? d.occ_staged[1] : d.occ_staged[0]);
  const int whole_cap = d.num_cus * (h2d ? d.occ_whole[1] : d.occ_whole[0]);
  const hsa_agent_t host_agent = d.cpu_agent;   // device-resident caches never get here

  struct Piece {
    int l0, nl, b0, nb;
  };
  std::vector<Piece> pieces;
  for (int l0 = 0; l0 < g.num_layers; l0 += nl_piece)
    for (int b0 = 0; b0 < g.num_blocks; b0 += blocks_per_piece)
      pieces.push_back({l0, std::min(nl_piece, g.num_layers - l0), b0,
                        std::min(blocks_per_piece, g.num_blocks - b0)});
  // The first piece's gather (D2H) and the last piece's scatter (H2D) run
  // with no engine copies beside them.  When that piece is large, an eighth
  // of a half is cut off it, so the engines start, or the transfer ends,
  // after a short kernel.  A smaller edge piece of at least
  // edge_small_min_bytes() gives a quarter of its blocks instead; below that
  // it is not cut, since every piece costs a host round trip.
  if (!pieces.empty()) {
    const size_t edge = h2d ? pieces.size() - 1 : 0;
    const Piece p = pieces[edge];
    const int64_t bytes = static_cast<int64_t>(p.nb) * p.nl * g.kv * g.chunk;
    int cut = 0;
    if (bytes >= kEdgePieceMinBytes)
      cut = std::min(p.nb - 1, std::max(1, blocks_per_piece / kEdgePieceDiv));
    else if (bytes >= edge_small_min_bytes())
      cut = std::min(p.nb - 1, std::max(1, p.nb / kEdgeSmallDiv));
    if (cut >= 1) {
      Piece first = p, second = p;
      first.nb = h2d ? p.nb - cut : cut;
      second.b0 = p.b0 + first.nb;
      second.nb = p.nb - first.nb;
      pieces[edge] = first;
      pieces.insert(pieces.begin() + static_cast<std::ptrdiff_t>(edge) + 1, second);
    }
  }
  const int np = static_cast<int>(pieces.size());

  // Host-side waits order everything below against the caller's stream, so
  // work already queued on it comes first.
  FKV_HIP(hipStreamSynchronize(stream));
  // After the drain below (declared later, so it runs first), hand the host
  // blocks of device-to-host copies given up on to the calling thread
  // (fkv_last_unsafe_host_blocks).
  struct PublishUnsafeRows {
    CopyLane& ln;
    ~PublishUnsafeRows() {
      std::vector<int64_t> ids = ln.rows.take_unsafe();
      if (!ids.empty()) last_unsafe_host_blocks() = std::move(ids);
    }
  } publish{ln};
  DrainOnError drain{stream, &d, &ln};
  if ((rc = stage_ids_on_device(ids.buf, g.num_blocks, dev, stream, dev_ids, &kids, &kids_split)))
    return rc;
  ProfRecorder prof;
  std::vector<Run> runs;
  bool pending[2] = {false, false};
  int64_t dma_copies = 0, dma_bytes = 0, held_copies = 0;
  const auto t0 = std::chrono::steady_clock::now();
  // Host-to-device copies into one half run beside the scatter of the other
  // half's previous piece; the held engines' share of them waits for that
  // scatter (issue_sdma, SdmaHold) and is queued by release_held.
  SdmaHold hold[2];
  auto piece_bytes_of = [&](int pi) {
    const Piece& p = pieces[pi];
    return static_cast<int64_t>(p.nb) * p.nl * g.kv * g.chunk;
  };
  auto queue_copies = [&](int pi) -> int {
    const Piece& p = pieces[pi];
    const int h = pi & 1;
    build_runs(g, p.b0, p.nb, p.l0, p.nl, sdma_rect_available(), layer_major, runs);
    int64_t piece_bytes = 0;
    for (const Run& r : runs) piece_bytes += r.bytes * std::max<int64_t>(1, r.slices);
    dma_bytes += piece_bytes;
    dma_copies += static_cast<int64_t>(runs.size());
    pending[h] = true;
    if (!h2d) ln.rows.queued(h, g.cids + p.b0, static_cast<size_t>(p.nb));
    // Host-to-device copies shorter than kWideCopyBytes on average are bound
    // by the engines' per-copy cost and spread over the wide set
    const bool wide = h2d && !runs.empty() &&
                      piece_bytes < kWideCopyBytes * static_cast<int64_t>(runs.size());
    hold[h].held_fraction = wide && pi > 0 ? held_fraction(piece_bytes_of(pi - 1), piece_bytes)
                                           : 0.0;
    return issue_sdma(d, ln, runs, ln.staging + h * half, h2d, h, host_agent,
                      wide ? kEnginesWideSync : kEnginesOwn, &hold[h]);
  };
  auto release_held = [&](int pi) -> int {
    const int h = pi & 1;
    if (hold[h].deferred.empty()) return 0;
    held_copies += static_cast<int64_t>(hold[h].deferred.size());
    const int rc2 = issue_sdma(d, ln, hold[h].deferred, ln.staging + h * half, h2d, h,
                               host_agent, kEnginesWideSync, nullptr, /*held_part=*/true);
    hold[h].deferred.clear();
    return rc2;
  };
  auto launch = [&](int pi) -> int {
    const Piece& p = pieces[pi];
    // staging strides (K|V, layer, block) of the piece
    int64_t cks, cls, cbs;
    if (layer_major) {
      cbs = g.chunk;
      cks = g.kv == 1 ? 0 : static_cast<int64_t>(p.nb) * g.chunk;
      cls = static_cast<int64_t>(g.kv) * p.nb * g.chunk;
    } else {
      cks = g.kv == 1 ? 0 : g.chunk;
      cls = static_cast<int64_t>(g.kv) * g.chunk;
      cbs = static_cast<int64_t>(p.nl) * cls;
    }
    char* stg = ln.staging + (pi & 1) * half;
    return h2d ? launch_copy<true, true>(g, kids, stg, cks, cls, cbs, p.b0, p.nb, p.l0, p.nl,
                                         grid_cap, stream, prof, kids_split, whole_cap)
               : launch_copy<false, true>(g, kids, stg, cks, cls, cbs, p.b0, p.nb, p.l0, p.nl,
                                          grid_cap, stream, prof, kids_split, whole_cap);
  };
  if (!h2d) {
    for (int pi = 0; pi < np; ++pi) {
      const int h = pi & 1;
      if (pending[h]) {
        pending[h] = false;
        if ((rc = sdma_wait(d, ln, h))) return rc;
      }
      if ((rc = launch(pi))) return rc;
      FKV_HIP(hipEventRecord(ln.ev_compute[h], stream));
      FKV_HIP(hipEventSynchronize(ln.ev_compute[h]));
      if ((rc = queue_copies(pi))) return rc;
    }
  } else {
    for (int pi = 0; pi < std::min(np, 2); ++pi)
      if ((rc = queue_copies(pi))) return rc;
    for (int pi = 0; pi < np; ++pi) {
      const int h = pi & 1;
      pending[h] = false;
      // the last piece has nothing behind it
      if ((rc = sdma_wait(d, ln, h, /*spin=*/pi + 1 == np))) return rc;
      hipLaunchKernelGGL(acquire_system_kernel, dim3(d.num_cus), dim3(64), 0, stream);
      FKV_HIP(hipGetLastError());
      if ((rc = launch(pi))) return rc;
      if (pi + 1 < np) {
        FKV_HIP(hipEventRecord(ln.ev_compute[h], stream));
        FKV_HIP(hipEventSynchronize(ln.ev_compute[h]));
        // the scatter of piece pi is done: the held engines take their share
        // of piece pi + 1, and piece pi + 2 goes into the half it read
        if ((rc = release_held(pi + 1))) return rc;
        if (pi + 2 < np && (rc = queue_copies(pi + 2))) return rc;
      }
    }
  }
  for (int h = 0; h < 2; ++h)
    if (pending[h]) {
      pending[h] = false;
      if ((rc = sdma_wait(d, ln, h, /*spin=*/true))) return rc;
    }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  if (prof.on) {
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    prof_add_dma(ms, dma_copies, dma_bytes, held_copies);
  }
  prof.flush();
  return 0;
}

// Gather (to_gpu = false) or scatter between the GPU cache and a contiguous
// buffer laid out [block][layer][K|V][chunk]; g.cpu_ptr is the buffer and
// g.cids is 0..n-1.  Uses every compute unit: the copy is HBM-bound.
int transfer_contiguous(const Geometry& g, hipStream_t stream, int dev, bool to_gpu) {
  DeviceState& d = g_dev[dev];
  IdLease ids;
  int rc = pack_ids(g, ids);
  if (rc) return rc;
  const int grid_cap = d.num_cus * (to_gpu ? d.occ_staged[1] : d.occ_staged[0]);
  const int whole_cap = d.num_cus * (to_gpu ? d.occ_whole[1] : d.occ_whole[0]);
  DevIdLease dev_ids;
  IdBuf kids;
  int32_t kids_split = 0;
  DrainOnError drain{stream};
  if ((rc = stage_ids_on_device(ids.buf, g.num_blocks, dev, stream, dev_ids, &kids, &kids_split)))
    return rc;
  ProfRecorder prof;
  const int per_launch = g.layers_per_launch();
  for (int l0 = 0; l0 < g.num_layers; l0 += per_launch) {
    const int nl = std::min(per_launch, g.num_layers - l0);
    char* base = g.cpu_info.dev_ptr + static_cast<int64_t>(l0) * g.cls;
    rc = to_gpu ? launch_copy<true, true>(g, kids, base, g.cks, g.cls, g.cbs, 0, g.num_blocks,
                                          l0, nl, grid_cap, stream, prof, kids_split, whole_cap)
                : launch_copy<false, true>(g, kids, base, g.cks, g.cls, g.cbs, 0, g.num_blocks,
                                           l0, nl, grid_cap, stream, prof, kids_split,
                                           whole_cap);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

int contiguous_entry(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                     void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                     int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes, void* buffer,
                     size_t buffer_bytes, fkv_stream_t stream, int is_mla, bool to_gpu) {
  try {
    last_error().clear();
    last_unsafe_host_blocks().clear();
    if (num_blocks == 0 || num_layers == 0) return 0;
    if (num_blocks < 0 || num_layers < 0)
      return fail(kInval, "negative count: num_blocks=%d num_layers=%d", num_blocks, num_layers);
    std::vector<int64_t> iota(static_cast<size_t>(num_blocks));
    for (int i = 0; i < num_blocks; ++i) iota[i] = i;
    Geometry g;
    g.num_blocks = num_blocks;
    g.start_layer = 0;
    g.num_layers = num_layers;
    g.kv = is_mla ? 1 : 2;
    g.gids = gpu_block_ids;
    g.cids = iota.data();
    g.layer_ptrs = gpu_layer_ptrs;
    g.gks = gpu_kv_stride_bytes;
    g.gbs = gpu_block_stride_bytes;
    g.chunk = chunk_size_bytes;
    g.cks = g.kv == 1 ? 0 : chunk_size_bytes;
    g.cls = static_cast<int64_t>(g.kv) * chunk_size_bytes;
    g.cbs = static_cast<int64_t>(num_layers) * g.cls;
    g.startoff = 0;
    g.cpu_ptr = static_cast<char*>(buffer);
    const __int128 need = static_cast<__int128>(num_blocks) * g.cbs;
    if (need > static_cast<__int128>(buffer_bytes))
      return fail(kInval, "buffer holds %zu bytes, the blocks need %lld", buffer_bytes,
                  static_cast<long long>(need));
    int rc = validate(g, FKV_XFER_KERNEL);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    if ((rc = stream_device(s, &dev))) return rc;
    if ((rc = ensure_device_basics(dev))) return rc;
    return transfer_contiguous(g, s, dev, to_gpu);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

// The reference copy-engine loop, csrc/transfer.cu:97-121: one async copy per
// (layer, K|V, block) chunk, issued layer-major then K|V then block.
int transfer_ce_per_chunk(const Geometry& g, hipStream_t stream, bool h2d) {
  DrainOnError drain{stream};
  ProfRecorder prof;
  hipEvent_t ev = nullptr;
  int rc = prof.begin(stream, &ev);
  if (rc) return rc;
  for (int l = 0; l < g.num_layers; ++l) {
    for (int k = 0; k < g.kv; ++k) {
      char* gk = g.gpu_base(l, k);
      for (int i = 0; i < g.num_blocks; ++i) {
        char* cpu = g.cpu_ptr + static_cast<int64_t>(l + g.start_layer) * g.cls + k * g.cks +
                    g.cids[i] * g.cbs + g.startoff;
        char* gpu = gk + g.gids[i] * g.gbs;
        if (h2d) {
          FKV_HIP(hipMemcpyAsync(gpu, cpu, g.chunk, hipMemcpyHostToDevice, stream));
        } else {
          FKV_HIP(hipMemcpyAsync(cpu, gpu, g.chunk, hipMemcpyDeviceToHost, stream));
        }
      }
    }
  }
  const int64_t copies = static_cast<int64_t>(g.num_layers) * g.kv * g.num_blocks;
  if ((rc = prof.end(stream, ev, copies * g.chunk, copies, true))) return rc;
  FKV_HIP(hipStreamSynchronize(stream));
  drain.armed = false;
  prof.flush();
  return 0;
}

// ---------------------------------------------------------------------------
// Asynchronous layer-grouped transfers.  A handle owns a pinned id buffer
// from the id pool (returned at release) and one event per group.  Live
// handles are registered, so a stale or released handle is refused and
// fkv_finalize can release the ones left.

}  // namespace

struct fkv_transfer_handle_s {
  int dev = 0;
  hipStream_t stream = nullptr;
  std::vector<hipEvent_t> done;   // one per layer group, in order
  IdBuf ids;
  ProfRecorder prof;
  bool enqueued = false;          // every group was enqueued
  // Copy-engine pipeline: a driver thread queues each layer group's SDMA
  // copies into staging and, once they have landed, the group's scatter on
  // the lane's pipeline stream, then records done[g] there.  `recorded`
  // counts the events recorded so far; a caller that waits on a group (on
  // the host or through another stream) first waits for its event to exist.
  bool ce = false;
  std::thread driver;
  hipEvent_t start = nullptr;     // the caller's stream at the call
  std::mutex mu;
  std::condition_variable cv;
  int recorded = 0;
  int err = 0;
  std::string err_msg;
  int granularity = 1;
  Geometry geo;                   // points at the copies below
  std::vector<int64_t> gids, cids;
  std::vector<void*> ptrs;
};

namespace {

std::mutex g_handles_mu;
std::vector<fkv_transfer_handle_s*> g_handles;   // live handles

void handle_register(fkv_transfer_handle_s* h) {
  std::lock_guard<std::mutex> lk(g_handles_mu);
  g_handles.push_back(h);
}

// Removes h from the registry; false when it is not a live handle.
bool handle_unregister(fkv_transfer_handle_s* h) {
  std::lock_guard<std::mutex> lk(g_handles_mu);
  auto it = std::find(g_handles.begin(), g_handles.end(), h);
  if (it == g_handles.end()) return false;
  g_handles.erase(it);
  return true;
}

bool handle_live(fkv_transfer_handle_s* h) {
  std::lock_guard<std::mutex> lk(g_handles_mu);
  return std::find(g_handles.begin(), g_handles.end(), h) != g_handles.end();
}

int layerwise_enqueue(const Geometry& g, hipStream_t stream, int dev, int transfer_cus, bool h2d,
                      int granularity, fkv_transfer_handle_s* h) {
  DeviceState& d = g_dev[dev];
  int rc = ids_acquire(static_cast<size_t>(g.num_blocks) * 16, &h->ids);
  if (rc) return rc;
  pack_ids_into(g, h->ids.host);
  const int automatic = h2d ? kAutoLayerwiseH2DCus : auto_zero_copy_cus(g, h2d);
  const int cus = transfer_cus <= 0 ? std::min(automatic, d.num_cus)
                                    : std::min(transfer_cus, d.num_cus);
  const int grid_cap = cus * (h2d ? d.occ_zero_copy[1] : d.occ_zero_copy[0]);
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff + static_cast<int64_t>(g.start_layer) * g.cls;
  for (int g0 = 0; g0 < g.num_layers; g0 += granularity) {
    const int gend = std::min(g.num_layers, g0 + granularity);
    for (int l0 = g0; l0 < gend; l0 += g.layers_per_launch()) {
      const int nl = std::min(g.layers_per_launch(), gend - l0);
      char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
      rc = h2d ? launch_copy<true, false>(g, h->ids, base, g.cks, g.cls, g.cbs, 0,
                                          g.num_blocks, l0, nl, grid_cap, stream, h->prof)
               : launch_copy<false, false>(g, h->ids, base, g.cks, g.cls, g.cbs, 0,
                                           g.num_blocks, l0, nl, grid_cap, stream, h->prof);
      if (rc) return rc;
    }
    hipEvent_t ev = nullptr;
    FKV_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    h->done.push_back(ev);
    FKV_HIP(hipEventRecord(ev, stream));
  }
  h->enqueued = true;
  return 0;
}

// Wait for everything the handle enqueued, then free it.  Safe on a handle
// whose enqueue failed part-way.
int handle_destroy(fkv_transfer_handle_s* h) {
  int rc = 0;
  if (h->driver.joinable()) h->driver.join();   // every event is recorded once it ends
  if (h->ce && h->err) rc = fail(h->err, "%s", h->err_msg.c_str());
  if (h->enqueued && !h->done.empty()) {
    hipError_t e = hipEventSynchronize(h->done.back());
    if (e != hipSuccess) rc = fail(static_cast<int>(e), "hipEventSynchronize: %s", hipGetErrorString(e));
  } else if (h->ids.host) {  // enqueue failed after taking ids: drain what was issued
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) rc = fail(static_cast<int>(e), "hipStreamSynchronize: %s", hipGetErrorString(e));
  }
  h->prof.flush();
  for (hipEvent_t ev : h->done) (void)hipEventDestroy(ev);
  if (h->start) (void)hipEventDestroy(h->start);
  if (h->ids.host) ids_release(h->ids);
  delete h;
  return rc;
}

// Whether the copy-engine layer-wise pipeline takes this transfer: host to
// device from pinned host memory whose layer groups are contiguous per block
// (block-wise host rows), on a device whose engines work.  Anything else
// moves with the zero-copy kernel, as the synchronous path's policy would.
bool layerwise_ce_fits(const Geometry& g, int dev, bool h2d, int granularity) {
  if (!h2d || g.cpu_info.device || g_dev[dev].sdma_failed.load()) return false;
  const int nl = std::min(granularity, g.num_layers);
  return (g.kv == 1 || g.cks == g.chunk) && (nl == 1 || g.cls == g.kv * g.chunk);
}

// Smallest engine copy per block the copy-engine layer-wise pipeline aims for
// (bytes; FLEXKV_LAYERWISE_CE_MIN_COPY_BYTES), by carrying several layer
// groups in one window.  0 or 1: one group per window.
size_t layerwise_min_copy_bytes() {
  const char* e = getenv("FLEXKV_LAYERWISE_CE_MIN_COPY_BYTES");
  const long long v = e ? atoll(e) : static_cast<long long>(kLayerwiseCeMinCopyBytes);
  return v > 0 ? static_cast<size_t>(v) : 1;
}

constexpr int kLayerwiseCeKernelGroups = 0;

// Leading layer groups a copy-engine layer-wise handle moves with the
// zero-copy kernel before its engines start (FLEXKV_LAYERWISE_CE_KERNEL_GROUPS,
// default 0: every group on the engines; at most all groups but one).  A
// one-group window is bound by the engines' per-copy cost (one copy per block
// of one group's rows), while a consumer waiting for the first group has
// nothing else to run, so the kernel's compute units cost it little then.
// Measured on MI355X at the Llama-3-8B shape with one layer per group, one
// kernel group brings the first group in after 1.3 ms instead of 2.1 ms and
// ends a prefill overlapped with 8 or 12 bf16 GEMMs per layer 1.1-1.7%
// sooner, but one with 4 GEMMs per layer, which the transfer outlasts,
// 0.5% later.
int layerwise_kernel_lead_groups(int ngroups) {
  const char* e = getenv("FLEXKV_LAYERWISE_CE_KERNEL_GROUPS");
  const int v = e ? atoi(e) : kLayerwiseCeKernelGroups;
  return std::max(0, std::min(v, ngroups - 1));
}

// The lane's pipeline stream: a stream with a full CU mask, so it has a
// hardware queue of its own and its scatters never wait behind compute
// kernels queued on a shared queue.
int pipeline_stream(CopyLane& ln, int dev, hipStream_t* out) {
  std::lock_guard<std::mutex> lk(ln.stream_mu);
  if (!ln.pipeline_stream) {
    DeviceGuard guard;
    int rc = guard.set(dev);
    if (rc) return rc;
    int ncu = 0;
    FKV_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    std::vector<uint32_t> mask(static_cast<size_t>((ncu + 31) / 32), 0u);
    for (int c = 0; c < ncu; ++c) mask[c / 32] |= 1u << (c % 32);
    FKV_HIP(hipExtStreamCreateWithCUMask(&ln.pipeline_stream, static_cast<uint32_t>(mask.size()),
                                         mask.data()));
  }
  *out = ln.pipeline_stream;
  return 0;
}

// Groups [first_group, end_group) of a copy-engine handle (all groups when
// end_group < 0) move host-to-device with the zero-copy kernel on the
// pipeline stream (the layer-wise kernel path's compute units), each group's
// event recorded after it: every group on a device whose engines cannot be
// set up, and the leading groups a handle moves before its engines start.
int layerwise_kernel_groups(fkv_transfer_handle_s* h, hipStream_t work, int first_group = 0,
                            int end_group = -1) {
  const Geometry& g = h->geo;
  DeviceState& d = g_dev[h->dev];
  const int cus = std::min(kAutoLayerwiseH2DCus, d.num_cus);
  const int grid_cap = cus * d.occ_zero_copy[1];
  char* cpu_dev = g.cpu_info.dev_ptr + g.startoff + static_cast<int64_t>(g.start_layer) * g.cls;
  const int end_layer = end_group < 0 ? g.num_layers
                                      : std::min(g.num_layers, end_group * h->granularity);
  int group = first_group;
  for (int g0 = first_group * h->granularity; g0 < end_layer; g0 += h->granularity, ++group) {
    const int gend = std::min(g.num_layers, g0 + h->granularity);
    for (int l0 = g0; l0 < gend; l0 += g.layers_per_launch()) {
      const int nl = std::min(g.layers_per_launch(), gend - l0);
      char* base = cpu_dev + static_cast<int64_t>(l0) * g.cls;
      int rc = launch_copy<true, false>(g, h->ids, base, g.cks, g.cls, g.cbs, 0, g.num_blocks,
                                        l0, nl, grid_cap, work, h->prof);
      if (rc) return rc;
    }
    FKV_HIP(hipEventRecord(h->done[group], work));
    std::lock_guard<std::mutex> lk(h->mu);
    h->recorded = group + 1;
    h->cv.notify_all();
  }
  return 0;
}

// The driver's work: the leading group(s) with the zero-copy kernel (see
// layerwise_kernel_lead_groups), then the other layer groups in order, each
// cut into pieces of whole blocks that fit a staging half; SDMA copies (one per block: the group's
// rows are contiguous in block-wise host memory) on the wide engine set,
// double-buffered; each piece's scatter on the pipeline stream after a
// system-scope acquire; done[g] after the group's last piece.  The host
// waits for a piece's scatter before reusing its half.
int layerwise_ce_run(fkv_transfer_handle_s* h, CopyLane& ln, hipStream_t work) {
  DeviceState& d = g_dev[h->dev];
  const Geometry& g = h->geo;
  DeviceGuard guard;
  int rc = guard.set(h->dev);
  if (rc) return rc;
  FKV_HIP(hipEventSynchronize(h->start));   // the caller's earlier work is done
  const int G = h->granularity;
  const size_t req = g_staging_request.load();
  const size_t half_default = (req ? req : kDefaultStagingBytes) / 2;
  const int nl_max = std::min({G, g.num_layers, g.layers_per_launch()});
  const size_t row_max = static_cast<size_t>(nl_max) * g.kv * g.chunk;
  // a half holds at least one block's row of one layer, so every window fits
  const size_t one_layer = static_cast<size_t>(g.kv) * g.chunk;
  rc = staging_or_fallback(d, h->dev, ln, std::max(std::min(row_max, half_default), one_layer));
  if (rc == kSdmaUnavailable) return layerwise_kernel_groups(h, work);
  if (rc) return rc;
  if ((rc = ensure_sdma(d, h->dev, ln.staging))) {
    // nothing has been queued yet: this handle, and every later copy-engine
    // transfer on the device, moves with the zero-copy kernel
    if (!d.sdma_failed.exchange(true))
      fprintf(stderr, "flexkv: copy engines unavailable on device %d (%s); copy-engine "
              "transfers use the zero-copy kernel\n", h->dev, last_error().c_str());
    last_error().clear();
    return layerwise_kernel_groups(h, work);
  }
  BusyMark busy(d.busy[1]);
  const size_t half = ln.staging_bytes / 2;
  struct Piece {
    int l0, nl, b0, nb, group;   // group: the last layer group the piece completes
    bool last;
  };
  // Consecutive groups share engine copies when a block's rows of several
  // layers are contiguous in host memory: a full window carries at least
  // layerwise_min_copy_bytes() per block, which the engines move faster than
  // one-group copies.  Every group's event is recorded when the window
  // holding it has landed.  Windows grow from one group (1, 2, 4, ...), so
  // the first group arrives early, and near the end hold at most half of the
  // groups left, so the compute a window releases ends while the rest
  // arrive: a consumer that keeps up waits for one group's compute after the
  // last transfer, as with one group per window.
  const int lpl = g.layers_per_launch();
  const int ngroups = (g.num_layers + G - 1) / G;
  const size_t group_row = static_cast<size_t>(std::min(G, g.num_layers)) * g.kv * g.chunk;
  const size_t min_copy = layerwise_min_copy_bytes();
  int gpw = 1;   // groups per window
  if (G <= lpl && g.cls == static_cast<int64_t>(g.kv) * g.chunk) {
    gpw = static_cast<int>(std::max<size_t>(1, (min_copy + group_row - 1) / group_row));
    gpw = std::max(1, std::min(gpw, lpl / G));
    while (gpw > 1 && static_cast<size_t>(gpw) * group_row > half) --gpw;
  }
  // The leading groups move with the zero-copy kernel, alone on the link;
  // the engines start on the next group once they have landed.
  const int lead = layerwise_kernel_lead_groups(ngroups);
  std::vector<Piece> pieces;
  for (int grp = lead, ramp = 1; grp < ngroups; ramp = std::min(2 * ramp, gpw)) {
    const int take = std::min({gpw, ramp, std::max(1, (ngroups - grp) / 2)});
    const int l0 = grp * G;
    const int nl = std::min(take * G, g.num_layers - l0);
    grp += take;
    // a window moves in layer windows whose block rows fit a staging half
    // and whose layer pointers fit one launch's kernel arguments
    int win = std::min(nl, lpl);
    while (win > 1 && static_cast<size_t>(win) * g.kv * g.chunk > half) win = (win + 1) / 2;
    for (int w0 = l0; w0 < l0 + nl; w0 += win) {
      const int wn = std::min(win, l0 + nl - w0);
      const size_t row = static_cast<size_t>(wn) * g.kv * g.chunk;
      const int bpp = static_cast<int>(std::max<size_t>(1, half / row));
      for (int b0 = 0; b0 < g.num_blocks; b0 += bpp)
        pieces.push_back({w0, wn, b0, std::min(bpp, g.num_blocks - b0), grp - 1, false});
    }
    pieces.back().last = true;
  }
  const int np = static_cast<int>(pieces.size());
  const int grid_cap = d.num_cus * d.occ_staged[1];
  const int whole_cap = d.num_cus * d.occ_whole[1];
  std::vector<Run> runs;
  bool pending[2] = {false, false};
  int next_group = 0;   // the first group whose event is not yet recorded
  int64_t dma_copies = 0, dma_bytes = 0;
  const auto t0 = std::chrono::steady_clock::now();
  DrainOnError drain{work, &d, &ln};
  auto queue_copies = [&](int pi) -> int {
    const Piece& p = pieces[pi];
    build_runs(g, p.b0, p.nb, p.l0, p.nl, false, false, runs);
    for (const Run& r : runs) dma_bytes += r.bytes;
    dma_copies += static_cast<int64_t>(runs.size());
    pending[pi & 1] = true;
    // Copies of one block's window are bound by the engines' per-copy cost,
    // so every window spreads over the wide engine set.
    return issue_sdma(d, ln, runs, ln.staging + (pi & 1) * half, true, pi & 1, d.cpu_agent,
                      kEnginesWide);
  };
  if (lead > 0) {
    if ((rc = layerwise_kernel_groups(h, work, 0, lead))) return rc;
    next_group = lead;
    // engine copies started beside the kernel share the link with it, and the
    // first group lands no earlier than with the engines alone
    FKV_HIP(hipEventSynchronize(h->done[lead - 1]));
  }
  for (int pi = 0; pi < std::min(np, 2); ++pi)
    if ((rc = queue_copies(pi))) return rc;
  for (int pi = 0; pi < np; ++pi) {
    const Piece& p = pieces[pi];
    const int hf = pi & 1;
    pending[hf] = false;
    // The host sleeps while the other half's copies keep the engines busy;
    // only the last wait, which nothing overlaps, spins (a wake from a sleep
    // costs 15-30 us).  Spinning throughout would hold a host core for the
    // whole transfer.
    if ((rc = sdma_wait(d, ln, hf, /*spin=*/pi + 1 == np))) return rc;
    hipLaunchKernelGGL(acquire_system_kernel, dim3(d.num_cus), dim3(64), 0, work);
    FKV_HIP(hipGetLastError());
    const int64_t cks = g.kv == 1 ? 0 : g.chunk;
    const int64_t cls = static_cast<int64_t>(g.kv) * g.chunk;
    const int64_t cbs = static_cast<int64_t>(p.nl) * cls;
    // launch_copy reads the group's layer pointers from call layer p.l0 on
    if ((rc = launch_copy<true, true>(g, h->ids, ln.staging + hf * half, cks, cls, cbs, p.b0,
                                      p.nb, p.l0, p.nl, grid_cap, work, h->prof, 0,
                                      whole_cap)))
      return rc;
    if (p.last) {
      for (int gi = next_group; gi <= p.group; ++gi) FKV_HIP(hipEventRecord(h->done[gi], work));
      next_group = p.group + 1;
      std::lock_guard<std::mutex> lk(h->mu);
      h->recorded = next_group;
      h->cv.notify_all();
    }
    if (pi + 2 < np) {
      FKV_HIP(hipEventRecord(ln.ev_compute[hf], work));
      FKV_HIP(hipEventSynchronize(ln.ev_compute[hf]));
      if ((rc = queue_copies(pi + 2))) return rc;
    }
  }
  drain.armed = false;
  if (h->prof.on) {
    FKV_HIP(hipStreamSynchronize(work));
    prof_add_dma(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                     .count(),
                 dma_copies, dma_bytes);
  }
  return 0;
}

void layerwise_ce_drive(fkv_transfer_handle_s* h, hipStream_t work) {
  CopyLane& ln = g_dev[h->dev].lane[1];
  int rc = 0;
  std::string msg;
  {
    std::lock_guard<std::mutex> own(ln.mu);
    try {
      rc = layerwise_ce_run(h, ln, work);
    } catch (const std::exception& e) {
      rc = fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
    }
    if (rc) msg = last_error();
  }
  std::lock_guard<std::mutex> lk(h->mu);
  if (rc) {
    // every group's event is recorded even on failure, so no waiter blocks
    // for good; the handle reports the error
    h->err = rc;
    h->err_msg = msg;
    (void)hipSetDevice(h->dev);
    for (size_t gi = static_cast<size_t>(h->recorded); gi < h->done.size(); ++gi)
      (void)hipEventRecord(h->done[gi], work);
  }
  h->recorded = static_cast<int>(h->done.size());
  h->cv.notify_all();
}

// Set up the copy-engine pipeline of a handle and start its driver.  The
// caller's id lists and layer pointers are copied, since the driver reads
// them after the call returns.
int layerwise_ce_start(const Geometry& g, hipStream_t stream, int dev, int granularity,
                       fkv_transfer_handle_s* h) {
  h->ce = true;
  h->granularity = granularity;
  h->gids.assign(g.gids, g.gids + g.num_blocks);
  h->cids.assign(g.cids, g.cids + g.num_blocks);
  h->ptrs.assign(g.layer_ptrs, g.layer_ptrs + static_cast<int64_t>(g.num_layers) * g.ptrs_per_layer);
  h->geo = g;
  h->geo.gids = h->gids.data();
  h->geo.cids = h->cids.data();
  h->geo.layer_ptrs = h->ptrs.data();
  int rc = ids_acquire(static_cast<size_t>(g.num_blocks) * 16, &h->ids);
  if (rc) return rc;
  pack_ids_into(h->geo, h->ids.host);
  hipStream_t work = nullptr;
  if ((rc = pipeline_stream(g_dev[dev].lane[1], dev, &work))) return rc;
  for (int g0 = 0; g0 < g.num_layers; g0 += granularity) {
    hipEvent_t ev = nullptr;
    FKV_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    h->done.push_back(ev);
  }
  FKV_HIP(hipEventCreateWithFlags(&h->start, hipEventDisableTiming));
  FKV_HIP(hipEventRecord(h->start, stream));
  FKV_HIP(hipStreamWaitEvent(work, h->start, 0));
  h->driver = std::thread(layerwise_ce_drive, h, work);
  h->enqueued = true;
  return 0;
}

// A copy-engine handle's group g: wait until its event is recorded.  0, or
// the pipeline's error.
int ce_group_recorded(fkv_transfer_handle_s* h, int group) {
  std::unique_lock<std::mutex> lk(h->mu);
  h->cv.wait(lk, [&] { return h->recorded > group; });
  if (h->err) return fail(h->err, "%s", h->err_msg.c_str());
  return 0;
}

Geometry make_geometry(int num_blocks, int start_layer_id, int num_layers,
                       const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                       int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                       const int64_t* cpu_block_ids, void* cpu_ptr, int64_t cpu_kv_stride_bytes,
                       int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
                       int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes, int is_mla) {
  Geometry g;
  g.num_blocks = num_blocks;
  g.start_layer = start_layer_id;
  g.num_layers = num_layers;
  g.kv = is_mla ? 1 : 2;
  g.gids = gpu_block_ids;
  g.cids = cpu_block_ids;
  g.layer_ptrs = gpu_layer_ptrs;
  g.gks = gpu_kv_stride_bytes;
  g.gbs = gpu_block_stride_bytes;
  g.cks = cpu_kv_stride_bytes;
  g.cls = cpu_layer_stride_bytes;
  g.cbs = cpu_block_stride_bytes;
  g.startoff = cpu_startoff_inside_chunks;
  g.chunk = chunk_size_bytes;
  g.cpu_ptr = static_cast<char*>(cpu_ptr);
  return g;
}

// Copy-engine mode hands a transfer to the SDMA engines only when the
// engines pay off: the op moves at least ce_min_bytes() (default 32 MiB)
// and each engine copy moves at least 128 KiB: a contiguous host run, or one
// block's layer window as a rect copy when the host layout puts its chunks at
// one stride (layer-wise).  Each engine copy costs about 6 us and the
// host-side ordering about 40 us per call (MI355X: a 1 MiB op of 64 KiB runs
// takes 77 us on the engines, 39 us in the zero-copy kernel); smaller or
// finer-grained transfers, and caches in device memory, go to the zero-copy
// kernel, with identical results.
//
// A layer-wise host cache whose ids do not come in runs long enough for
// layer-major staging needs one rect copy per block, and the runtime runs
// every rect copy on a single engine per direction: 46.8 / 47.0 GB/s
// (D2H / H2D) at the Llama-3-8B shape, 82% of the link, against 56.5 /
// 57.2 GB/s for the zero-copy kernel.  Such transfers therefore move with
// the zero-copy kernel, which holds compute units for the whole transfer
// (160 bf16 GEMMs queued after a 2 GiB D2H starts take 71 ms instead of
// 36 ms beside the rect copies); fkv_set_copy_engine_policy (or
// FLEXKV_CE_RECT_COPIES=1) keeps them on the engines.
bool ce_pays_off(const Geometry& g, bool h2d) {
  // a "host" cache that is device memory has no PCIe copy to offload
  if (g.cpu_info.device) return false;
  const int64_t min_bytes = ce_min_bytes();
  const int64_t total = op_bytes(g);
  const bool row_contig = (g.kv == 1 || g.cks == g.chunk) &&
                          (g.num_layers == 1 || g.cls == g.kv * g.chunk);
  const int64_t row = static_cast<int64_t>(g.num_layers) * g.kv * g.chunk;
  const bool rect = !row_contig && host_slice_pitch(g, g.num_layers) > 0;
  if (rect && !layer_major_pays_off(g, layer_run_bytes(h2d)) && !ce_rect_copies()) return false;
  const int64_t run = (row_contig || rect) ? row : g.chunk;
  return total >= min_bytes && (min_bytes == 0 || run >= kCeMinRunBytes);
}

// Validate, then run one synchronous transfer in the requested mode.
// Copy-engine mode copies exact bytes for any geometry, as the reference's
// CE loop does (csrc/transfer.cu:97-121): a chunk size, stride, offset or
// pointer that is not a multiple of 16 bytes, which the kernels' 16-byte
// accesses cannot take, sends the transfer to the per-chunk engine loop.
int transfer_entry(Geometry& g, hipStream_t s, int transfer_cus, bool h2d, int mode) {
  if (mode == FKV_XFER_CE && !geometry_vec16(g)) mode = FKV_XFER_CE_PER_CHUNK;
  int rc = validate(g, mode);
  if (rc) return rc;
  int dev = 0;
  if ((rc = stream_device(s, &dev))) return rc;
  if ((rc = ensure_device_basics(dev))) return rc;
  switch (mode) {
    case FKV_XFER_KERNEL:
      return transfer_zero_copy(g, s, dev, transfer_cus, h2d);
    case FKV_XFER_CE:
      if (!ce_pays_off(g, h2d) || g_dev[dev].sdma_failed.load())
        return transfer_zero_copy(g, s, dev, transfer_cus, h2d);
      rc = transfer_staged(g, s, dev, h2d);
      return rc == kSdmaUnavailable ? transfer_zero_copy(g, s, dev, transfer_cus, h2d) : rc;
    default:
      return transfer_ce_per_chunk(g, s, h2d);
  }
}
}  // namespace

extern "C" {

int fkv_transfer_kv_blocks(int num_blocks, int start_layer_id, int num_layers,
                           const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                           int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                           const int64_t* cpu_block_ids, void* cpu_ptr,
                           int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                           int64_t cpu_block_stride_bytes, int64_t cpu_startoff_inside_chunks,
                           int64_t chunk_size_bytes, fkv_stream_t stream, int transfer_cus,
                           int is_host_to_device, int use_ce_transfer, int is_mla) {
  try {
    last_error().clear();
    last_unsafe_host_blocks().clear();
    if (use_ce_transfer < FKV_XFER_KERNEL || use_ce_transfer > FKV_XFER_CE_PER_CHUNK)
      return fail(kInval, "use_ce_transfer must be 0 (kernel), 1 (CE) or 2 (CE per chunk), got %d",
                  use_ce_transfer);
    if (num_blocks == 0 || num_layers == 0) return 0;
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids,
                               gpu_layer_ptrs, gpu_kv_stride_bytes, gpu_block_stride_bytes,
                               cpu_block_ids, cpu_ptr, cpu_kv_stride_bytes,
                               cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    return transfer_entry(g, static_cast<hipStream_t>(stream), transfer_cus,
                          is_host_to_device != 0, use_ce_transfer);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_transfer_kv_blocks_kv_ptrs(int num_blocks, int start_layer_id, int num_layers,
                                   const int64_t* gpu_block_ids, void* const* gpu_kv_ptrs,
                                   int64_t gpu_block_stride_bytes, const int64_t* cpu_block_ids,
                                   void* cpu_ptr, int64_t cpu_kv_stride_bytes,
                                   int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
                                   int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes,
                                   fkv_stream_t stream, int transfer_cus, int is_host_to_device,
                                   int use_ce_transfer, int is_mla) {
  try {
    last_error().clear();
    last_unsafe_host_blocks().clear();
    if (use_ce_transfer < FKV_XFER_KERNEL || use_ce_transfer > FKV_XFER_CE_PER_CHUNK)
      return fail(kInval, "use_ce_transfer must be 0 (kernel), 1 (CE) or 2 (CE per chunk), got %d",
                  use_ce_transfer);
    if (num_blocks == 0 || num_layers == 0) return 0;
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids, gpu_kv_ptrs,
                               0, gpu_block_stride_bytes, cpu_block_ids, cpu_ptr,
                               cpu_kv_stride_bytes, cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    g.ptrs_per_layer = g.kv;
    return transfer_entry(g, static_cast<hipStream_t>(stream), transfer_cus,
                          is_host_to_device != 0, use_ce_transfer);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_transfer_kv_blocks_noalloc(int num_blocks, int start_layer_id, int num_layers,
                                   const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs,
                                   int64_t gpu_kv_stride_bytes, int64_t gpu_block_stride_bytes,
                                   const int64_t* cpu_block_ids, void* cpu_ptr,
                                   int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes,
                                   int64_t cpu_block_stride_bytes,
                                   int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes,
                                   fkv_stream_t stream, int transfer_cus, int is_host_to_device,
                                   int is_mla) {
  try {
    last_error().clear();
    last_unsafe_host_blocks().clear();
    if (num_blocks == 0 || num_layers == 0) return 0;
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids,
                               gpu_layer_ptrs, gpu_kv_stride_bytes, gpu_block_stride_bytes,
                               cpu_block_ids, cpu_ptr, cpu_kv_stride_bytes,
                               cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The call is synchronous and resolves its ids and addresses on the host
    // while it runs, so a captured call could not replay: refuse capture
    // before anything reaches the stream (the null stream is never captured).
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (s) FKV_HIP(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return fail(static_cast<int>(hipErrorStreamCaptureUnsupported),
                  "fkv_transfer_kv_blocks_noalloc cannot run on a stream under HIP graph "
                  "capture (it synchronises the stream and stages ids from host memory)");
    int rc = validate(g, FKV_XFER_KERNEL);
    if (rc) return rc;
    int dev = 0;
    if ((rc = stream_device(s, &dev))) return rc;
    if ((rc = ensure_device_basics(dev))) return rc;
    return transfer_zero_copy_noalloc(g, s, dev, transfer_cus, is_host_to_device != 0);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_gather_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                         void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                         int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes, void* buffer,
                         size_t buffer_bytes, fkv_stream_t stream, int is_mla) {
  return contiguous_entry(num_blocks, num_layers, gpu_block_ids, gpu_layer_ptrs,
                          gpu_kv_stride_bytes, gpu_block_stride_bytes, chunk_size_bytes, buffer,
                          buffer_bytes, stream, is_mla, false);
}

int fkv_scatter_kv_blocks(int num_blocks, int num_layers, const int64_t* gpu_block_ids,
                          void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
                          int64_t gpu_block_stride_bytes, int64_t chunk_size_bytes,
                          const void* buffer, size_t buffer_bytes, fkv_stream_t stream,
                          int is_mla) {
  return contiguous_entry(num_blocks, num_layers, gpu_block_ids, gpu_layer_ptrs,
                          gpu_kv_stride_bytes, gpu_block_stride_bytes, chunk_size_bytes,
                          const_cast<void*>(buffer), buffer_bytes, stream, is_mla, true);
}

int fkv_transfer_kv_blocks_layerwise(
    int num_blocks, int start_layer_id, int num_layers, int layer_granularity,
    const int64_t* gpu_block_ids, void* const* gpu_layer_ptrs, int64_t gpu_kv_stride_bytes,
    int64_t gpu_block_stride_bytes, const int64_t* cpu_block_ids, void* cpu_ptr,
    int64_t cpu_kv_stride_bytes, int64_t cpu_layer_stride_bytes, int64_t cpu_block_stride_bytes,
    int64_t cpu_startoff_inside_chunks, int64_t chunk_size_bytes, fkv_stream_t stream,
    int transfer_cus, int is_host_to_device, int use_ce_transfer, int is_mla,
    fkv_transfer_handle* out) {
  try {
    last_error().clear();
    last_unsafe_host_blocks().clear();
    if (!out) return fail(kInval, "out handle pointer is null");
    if (use_ce_transfer != FKV_XFER_KERNEL && use_ce_transfer != FKV_XFER_CE)
      return fail(kInval, "use_ce_transfer must be 0 (kernel) or 1 (copy engines), got %d",
                  use_ce_transfer);
    *out = nullptr;
    if (layer_granularity < 1) return fail(kInval, "layer_granularity must be >= 1");
    if (num_blocks < 0 || num_layers < 0)
      return fail(kInval, "negative count: num_blocks=%d num_layers=%d", num_blocks, num_layers);
    Geometry g = make_geometry(num_blocks, start_layer_id, num_layers, gpu_block_ids,
                               gpu_layer_ptrs, gpu_kv_stride_bytes, gpu_block_stride_bytes,
                               cpu_block_ids, cpu_ptr, cpu_kv_stride_bytes,
                               cpu_layer_stride_bytes, cpu_block_stride_bytes,
                               cpu_startoff_inside_chunks, chunk_size_bytes, is_mla);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* h = new fkv_transfer_handle_s();
    h->stream = s;
    int rc = 0;
    if (num_blocks > 0 && num_layers > 0) {
      const bool h2d = is_host_to_device != 0;
      if ((rc = validate(g, FKV_XFER_KERNEL)) || (rc = stream_device(s, &h->dev)) ||
          (rc = ensure_device_basics(h->dev)) ||
          (rc = (use_ce_transfer == FKV_XFER_CE &&
                 layerwise_ce_fits(g, h->dev, h2d, layer_granularity))
                    ? layerwise_ce_start(g, s, h->dev, layer_granularity, h)
                    : layerwise_enqueue(g, s, h->dev, transfer_cus, h2d, layer_granularity, h))) {
        const std::string msg = last_error();
        (void)handle_destroy(h);
        last_error() = msg;
        return rc;
      }
    }
    handle_register(h);
    *out = h;
    return 0;
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_handle_num_groups(fkv_transfer_handle h) {
  last_error().clear();
  if (!h || !handle_live(h)) return fail(-1, "null, released or unknown handle");
  return static_cast<int>(h->done.size());
}

int fkv_handle_query(fkv_transfer_handle h, int group) {
  last_error().clear();
  if (!h || !handle_live(h) || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(-1, "bad handle or group %d", group);
  if (h->ce) {
    std::lock_guard<std::mutex> lk(h->mu);
    if (h->recorded <= group) return 0;
    if (h->err) return fail(-h->err, "%s", h->err_msg.c_str());
  }
  hipError_t e = hipEventQuery(h->done[group]);
  if (e == hipSuccess) return 1;
  (void)hipGetLastError();
  if (e == hipErrorNotReady) return 0;
  return fail(-static_cast<int>(e), "hipEventQuery: %s", hipGetErrorString(e));
}

int fkv_handle_wait(fkv_transfer_handle h, int group) {
  last_error().clear();
  if (!h || !handle_live(h) || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(kInval, "bad handle or group %d", group);
  if (h->ce) {
    const int rc = ce_group_recorded(h, group);
    if (rc) return rc;
  }
  FKV_HIP(hipEventSynchronize(h->done[group]));
  return 0;
}

int fkv_handle_stream_wait(fkv_transfer_handle h, int group, fkv_stream_t other) {
  last_error().clear();
  if (!h || !handle_live(h) || group < 0 || group >= static_cast<int>(h->done.size()))
    return fail(kInval, "bad handle or group %d", group);
  if (h->ce) {
    // the group's event exists once its copies have landed and its scatter
    // is queued; only then can another stream wait on it
    const int rc = ce_group_recorded(h, group);
    if (rc) return rc;
  }
  FKV_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(other), h->done[group], 0));
  return 0;
}

int fkv_handle_release(fkv_transfer_handle h) {
  last_error().clear();
  if (!h) return 0;
  if (!handle_unregister(h)) return fail(kInval, "handle %p is released or unknown", (void*)h);
  return handle_destroy(h);
}

int fkv_set_copy_engine_policy(int64_t min_bytes, int rect_copies) {
  last_error().clear();
  if (min_bytes < -2)
    return fail(kInval, "min_bytes must be >= 0, -1 to unset or -2 to keep, got %lld",
                static_cast<long long>(min_bytes));
  if (rect_copies < -2 || rect_copies > 1)
    return fail(kInval, "rect_copies must be 0, 1, -1 to unset or -2 to keep, got %d",
                rect_copies);
  if (min_bytes != -2) g_ce_min_bytes.store(min_bytes);
  if (rect_copies != -2) g_ce_rect_copies.store(rect_copies);
  return 0;
}

int fkv_get_copy_engine_policy(int64_t* min_bytes, int* rect_copies) {
  last_error().clear();
  if (!min_bytes || !rect_copies) return fail(kInval, "null output pointer");
  *min_bytes = ce_min_bytes();
  *rect_copies = ce_rect_copies() ? 1 : 0;
  return 0;
}

int fkv_prepare(int device) {
  try {
    last_error().clear();
    int dev = device;
    if (dev < 0) FKV_HIP(hipGetDevice(&dev));
    int count = 0;
    FKV_HIP(hipGetDeviceCount(&count));
    if (dev >= count || dev >= kMaxDevices)
      return fail(kInval, "device %d out of range (%d devices)", dev, count);
    DeviceGuard guard;
    int rc = guard.set(dev);
    if (rc) return rc;
    if ((rc = ensure_device_basics(dev))) return rc;
    // the library's code object is loaded with its first kernel launch
    hipLaunchKernelGGL(acquire_system_kernel, dim3(1), dim3(64), 0, nullptr);
    FKV_HIP(hipGetLastError());
    FKV_HIP(hipStreamSynchronize(nullptr));
    DeviceState& d = g_dev[dev];
    if (d.sdma_failed.load()) return 0;   // copy-engine transfers use the zero-copy kernel
    IdLease host;
    if ((rc = ids_acquire(kPrepareHostBytes, &host.buf))) return rc;
    for (int dir = 0; dir < 2; ++dir) {
      CopyLane& ln = d.lane[dir];
      std::lock_guard<std::mutex> lk(ln.mu);
      rc = staging_or_fallback(d, dev, ln, 0);
      if (rc == kSdmaUnavailable) return 0;   // no memory for staging: the transfer falls back
      if (rc) return rc;
      if ((rc = ensure_sdma(d, dev, ln.staging))) {
        if (!d.sdma_failed.exchange(true))
          fprintf(stderr, "flexkv: copy engines unavailable on device %d (%s); copy-engine "
                  "transfers use the zero-copy kernel\n", dev, last_error().c_str());
        last_error().clear();
        return 0;
      }
      if ((rc = sdma_prepare_lane(d, ln, dir == 1, kPrepareSignalsPerHalf,
                                  reinterpret_cast<char*>(host.buf.host), kPrepareHostBytes)))
        return rc;
    }
    // the stream of the copy-engine layer-wise pipeline's scatters
    hipStream_t work = nullptr;
    return pipeline_stream(d.lane[1], dev, &work);
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}

int fkv_finalize(void) {
  try {
    last_error().clear();
    int rc = 0;
    auto keep = [&rc](int r) {
      if (r && !rc) rc = r;
    };
    // 1. layer-wise handles the caller never released: wait for their groups
    std::vector<fkv_transfer_handle_s*> handles;
    {
      std::lock_guard<std::mutex> lk(g_handles_mu);
      handles.swap(g_handles);
    }
    for (fkv_transfer_handle_s* h : handles) keep(handle_destroy(h));
    // TP groups: their rank threads and streams
    keep(tp_groups_destroy_all());
    // 2. streams made by fkv_stream_create (each is synchronised first)
    keep(streams_destroy_all());
    // 3. copy-engine lanes: queued copies, signals, events, staging
    for (int dev = 0; dev < kMaxDevices; ++dev) {
      DeviceState& d = g_dev[dev];
      for (CopyLane& ln : d.lane) {
        std::lock_guard<std::mutex> lk(ln.mu);
        const bool used = ln.staging || ln.ev_compute[0] || ln.ev_compute[1] ||
                          ln.pipeline_stream ||
                          !ln.polled_pool[0].empty() || !ln.irq_pool[0].empty() ||
                          !ln.polled_pool[1].empty() || !ln.irq_pool[1].empty();
        if (!used) continue;
        DeviceGuard guard;
        const int r = guard.set(dev);
        if (r) {
          keep(r);
          continue;
        }
        keep(lane_release(d, ln));
      }
    }
    // 4. pinned and device id buffers
    keep(ids_pool_free());
    keep(dev_ids_pool_free());
    return rc;
  } catch (const std::exception& e) {
    return fail(static_cast<int>(hipErrorUnknown), "exception: %s", e.what());
  } catch (...) {
    return fail(static_cast<int>(hipErrorUnknown), "unknown exception");
  }
}


}  // extern "C"
