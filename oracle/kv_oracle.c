/*
 * kv_oracle.c - CPU restatement of FlexKV's GPU<->CPU KV-block transfer.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle for the HIP transfer
 * library and the CPU baseline that bench.py times; it is never linked into
 * or called by the product path (flexkv_amd), which fails loudly when its
 * HIP library is missing.
 *
 * Every "GPU" pointer here is host memory: a host-resident copy of the
 * engine's per-layer KV tensors.  The arithmetic follows the reference:
 *   - stride conversion to int64 units by truncating division,
 *     csrc/transfer.cu:84-93;
 *   - chunk index decomposition layer -> K|V -> block and the two chunk
 *     addresses, csrc/transfer.cu:37-50 (kernel) and :98-111 (copy engine);
 *   - kernel mode copies floor(chunk/16) 16-byte vectors (the int64 -> float4
 *     conversion at csrc/transfer.cu:35, loop at :55-59) and reads block ids
 *     through `int` (csrc/transfer.cu:41-42); copy-engine mode copies exactly
 *     chunk bytes with 64-bit ids (csrc/transfer.cu:104-117);
 *   - the multi-threaded variant partitions blocks into contiguous ranges of
 *     ceil(n / threads) and each thread loops block -> layer -> K then V, the
 *     structure of the reference's CPU fan-out, csrc/transfer_ssd.cpp:120-179
 *     and :215-284, with memcpy in place of pread/pwrite;
 *   - oracle_transfer_kv_blocks_ssd restates the SSD tier's block mapping and
 *     offsets over in-memory file images (end of this file).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int num_blocks, start_layer_id, num_layers, kv_dim;
  const int64_t *gpu_block_ids, *cpu_block_ids;
  void *const *gpu_layer_ptrs;
  int64_t gpu_kv, gpu_block;            /* int64 units */
  int64_t cpu_kv, cpu_layer, cpu_block; /* int64 units */
  int64_t startoff;                     /* int64 units */
  int64_t copy_bytes;
  int64_t *cpu_ptr;
  int h2d, kernel_mode;
  int b_begin, b_end;
} job_t;

static void copy_one(const job_t *j, int layer_idx, int kv_idx, int i) {
  int64_t gid, cid;
  if (j->kernel_mode) {
    /* csrc/transfer.cu:41-42 stores the ids in `int` */
    gid = (int)j->gpu_block_ids[i];
    cid = (int)j->cpu_block_ids[i];
  } else {
    gid = j->gpu_block_ids[i];
    cid = j->cpu_block_ids[i];
  }
  int64_t *cpu_chunk = j->cpu_ptr + (int64_t)(layer_idx + j->start_layer_id) * j->cpu_layer +
                       (int64_t)kv_idx * j->cpu_kv + cid * j->cpu_block + j->startoff;
  int64_t *gpu_chunk = (int64_t *)j->gpu_layer_ptrs[layer_idx] + (int64_t)kv_idx * j->gpu_kv +
                       gid * j->gpu_block;
  if (j->h2d)
    memcpy(gpu_chunk, cpu_chunk, (size_t)j->copy_bytes);
  else
    memcpy(cpu_chunk, gpu_chunk, (size_t)j->copy_bytes);
}

/* Reference chunk order: chunk = (layer * kv_dim + kv) * num_blocks + block. */
static void run_reference_order(const job_t *j) {
  for (int l = 0; l < j->num_layers; ++l)
    for (int k = 0; k < j->kv_dim; ++k)
      for (int i = 0; i < j->num_blocks; ++i) copy_one(j, l, k, i);
}

/* Thread body: blocks [b_begin, b_end), block -> layer -> K then V. */
static void *run_block_range(void *arg) {
  const job_t *j = (const job_t *)arg;
  for (int i = j->b_begin; i < j->b_end; ++i)
    for (int l = 0; l < j->num_layers; ++l)
      for (int k = 0; k < j->kv_dim; ++k) copy_one(j, l, k, i);
  return NULL;
}

/*
 * Same argument list and meaning as flexkv::transfer_kv_blocks
 * (csrc/transfer.cu:63-70) minus the stream and transfer_sms, plus
 * num_threads: 1 = the reference's sequential chunk order, > 1 = block-range
 * fan-out over that many threads.  Returns 0, or -1 on bad arguments.
 */
int oracle_transfer_kv_blocks(int num_blocks, int start_layer_id, int num_layers,
                              const int64_t *gpu_block_ids, void *const *gpu_layer_ptrs,
                              int64_t gpu_kv_stride_in_bytes, int64_t gpu_block_stride_in_bytes,
                              const int64_t *cpu_block_ids, void *cpu_ptr,
                              int64_t cpu_kv_stride_in_bytes, int64_t cpu_layer_stride_in_bytes,
                              int64_t cpu_block_stride_in_bytes,
                              int64_t cpu_startoff_inside_chunks, int64_t chunk_size_in_bytes,
                              int is_host_to_device, int use_ce_transfer, int is_mla,
                              int num_threads) {
  if (num_blocks < 0 || num_layers < 0 || num_threads < 1) return -1;
  if (num_blocks == 0 || num_layers == 0) return 0;
  job_t j;
  memset(&j, 0, sizeof(j));
  j.num_blocks = num_blocks;
  j.start_layer_id = start_layer_id;
  j.num_layers = num_layers;
  j.kv_dim = is_mla ? 1 : 2;
  j.gpu_block_ids = gpu_block_ids;
  j.cpu_block_ids = cpu_block_ids;
  j.gpu_layer_ptrs = gpu_layer_ptrs;
  j.gpu_kv = gpu_kv_stride_in_bytes / (int64_t)sizeof(int64_t);
  j.gpu_block = gpu_block_stride_in_bytes / (int64_t)sizeof(int64_t);
  j.cpu_kv = cpu_kv_stride_in_bytes / (int64_t)sizeof(int64_t);
  j.cpu_layer = cpu_layer_stride_in_bytes / (int64_t)sizeof(int64_t);
  j.cpu_block = cpu_block_stride_in_bytes / (int64_t)sizeof(int64_t);
  j.startoff = cpu_startoff_inside_chunks / (int64_t)sizeof(int64_t);
  j.cpu_ptr = (int64_t *)cpu_ptr;
  j.h2d = is_host_to_device != 0;
  j.kernel_mode = use_ce_transfer == 0;
  if (j.kernel_mode) {
    /* copy_size (int64 units) * 8 / 16 float4 elements of 16 bytes */
    int64_t chunk_int64 = chunk_size_in_bytes / (int64_t)sizeof(int64_t);
    j.copy_bytes = (chunk_int64 * (int64_t)sizeof(int64_t) / 16) * 16;
  } else {
    j.copy_bytes = chunk_size_in_bytes;
  }
  if (num_threads == 1) {
    run_reference_order(&j);
    return 0;
  }
  int per = (num_blocks + num_threads - 1) / num_threads;
  pthread_t *tids = (pthread_t *)calloc((size_t)num_threads, sizeof(pthread_t));
  job_t *jobs = (job_t *)calloc((size_t)num_threads, sizeof(job_t));
  int *started = (int *)calloc((size_t)num_threads, sizeof(int));
  if (!tids || !jobs || !started) {
    free(tids);
    free(jobs);
    free(started);
    return -1;
  }
  for (int t = 0; t < num_threads; ++t) {
    jobs[t] = j;
    jobs[t].b_begin = t * per;
    jobs[t].b_end = (t + 1) * per < num_blocks ? (t + 1) * per : num_blocks;
    if (jobs[t].b_begin >= jobs[t].b_end) continue;
    if (pthread_create(&tids[t], NULL, run_block_range, &jobs[t]) == 0)
      started[t] = 1;
    else
      run_block_range(&jobs[t]);
  }
  for (int t = 0; t < num_threads; ++t)
    if (started[t]) pthread_join(tids[t], NULL);
  free(tids);
  free(jobs);
  free(started);
  return 0;
}

/*
 * SSD tier restated (csrc/transfer_ssd.cpp:17-32 partition_and_remap,
 * :120-179 single-thread loop): `files` holds num_devices * files_per_device
 * in-memory file images, device-major.  For each block i in list order:
 * device d = (b / rr) % D, device block x = ((b / rr) / D) * rr + b % rr,
 * file x % F, in-file block x / F; then for each layer of the window, K then
 * V: chunk_size bytes between
 *   file + in_file*block_stride + l*ssd_layer_stride (+ ssd_kv_stride for V)
 *   cpu  + cpu_id*block_stride + l*cpu_layer_stride (+ cpu_kv_stride for V).
 * is_read: file -> cpu.  Returns 0, or -1 on bad arguments.
 */
int oracle_transfer_kv_blocks_ssd(void *const *files, int num_devices, int files_per_device,
                                  int start_layer, int num_layers, void *cpu_ptr,
                                  const int64_t *ssd_block_ids, const int64_t *cpu_block_ids,
                                  int num_blocks, int64_t cpu_layer_stride, int64_t cpu_kv_stride,
                                  int64_t ssd_layer_stride, int64_t ssd_kv_stride,
                                  int64_t chunk_size, int64_t block_stride, int is_read,
                                  int round_robin, int is_mla) {
  if (num_devices <= 0 || files_per_device <= 0 || round_robin <= 0 || num_blocks < 0)
    return -1;
  for (int i = 0; i < num_blocks; ++i) {
    int64_t b = ssd_block_ids[i];
    int64_t d = (b / round_robin) % num_devices;
    int64_t x = ((b / round_robin) / num_devices) * round_robin + (b % round_robin);
    char *file = (char *)files[d * files_per_device + (x % files_per_device)];
    int64_t in_file = x / files_per_device;
    for (int l = start_layer; l < start_layer + num_layers; ++l) {
      for (int k = 0; k < (is_mla ? 1 : 2); ++k) {
        char *s = file + in_file * block_stride + l * ssd_layer_stride + k * ssd_kv_stride;
        char *c = (char *)cpu_ptr + cpu_block_ids[i] * block_stride + l * cpu_layer_stride +
                  k * cpu_kv_stride;
        if (is_read)
          memcpy(c, s, (size_t)chunk_size);
        else
          memcpy(s, c, (size_t)chunk_size);
      }
    }
  }
  return 0;
}
