/*
 * A plain C consumer of libkvx: no Python, no torch. It allocates a small
 * paged KV pool with HIP, saves two blocks to FP8 entries and restores them
 * into two other blocks (kvx_save_blocks / kvx_restore_blocks), moves two
 * blocks through the copy engine to pinned host slots and back in BF16 mode
 * (kvx_cache_*), and checks that bad arguments come back as error codes.
 *
 * Usage: roundtrip OUT.bin
 * OUT.bin receives the pool before, the FP8 entries, the pool after the FP8
 * restore and the pool after the BF16 round trip; tests/test_gpu_c_abi.py
 * checks them against the oracle. Exit status 0 means every call succeeded
 * and the checks done here (BF16 bytes, error codes) passed.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kvx.h"

#define L 2
#define NB 6
#define BS 16
#define H 2
#define HD 128

static void hip_check(hipError_t err, const char* what) {
  if (err != hipSuccess) {
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(err));
    exit(2);
  }
}

static void kvx_check(int rc, const char* what) {
  if (rc != KVX_OK) {
    fprintf(stderr, "%s: %d (%s)\n", what, rc, kvx_last_error());
    exit(3);
  }
}

static uint32_t lcg(uint32_t* state) {
  *state = *state * 1664525u + 1013904223u;
  return *state >> 8;
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s OUT.bin\n", argv[0]);
    return 1;
  }
  if (kvx_abi_version() != KVX_ABI_VERSION) {
    fprintf(stderr, "ABI version %d, header %d\n", kvx_abi_version(), KVX_ABI_VERSION);
    return 4;
  }
  const size_t block_elems = (size_t)2 * L * BS * H * HD;
  const size_t elems = block_elems * NB;
  const size_t bytes = elems * sizeof(uint16_t);
  uint16_t* host = (uint16_t*)malloc(bytes);
  uint16_t* after_fp8 = (uint16_t*)malloc(bytes);
  uint16_t* after_raw = (uint16_t*)malloc(bytes);
  if (!host || !after_fp8 || !after_raw) return 5;
  uint32_t state = 12345u;
  for (size_t i = 0; i < elems; ++i) {  /* finite bf16: sign, exponent 112..135, 7 mantissa bits */
    const uint32_t r = lcg(&state);
    host[i] = (uint16_t)(((r & 1u) << 15) | ((112u + (r >> 1) % 24u) << 7) | ((r >> 6) & 0x7Fu));
  }

  hip_check(hipSetDevice(0), "hipSetDevice");
  void* pool = NULL;
  hip_check(hipMalloc(&pool, bytes), "hipMalloc pool");
  hip_check(hipMemcpy(pool, host, bytes, hipMemcpyHostToDevice), "upload pool");
  hipStream_t compute, save, restore;
  hip_check(hipStreamCreate(&compute), "hipStreamCreate");
  hip_check(hipStreamCreate(&save), "hipStreamCreate");
  hip_check(hipStreamCreate(&restore), "hipStreamCreate");

  kvx_block_layout layout;
  layout.plane_stride = (int64_t)NB * BS * H * HD;
  layout.block_stride = (int64_t)BS * H * HD;
  layout.planes = 2 * L;
  layout.plane_rows = BS * H;
  layout.head_dim = HD;
  layout.num_blocks = NB;
  layout.elem_bytes = 2;
  layout.scale_dtype = KVX_SCALE_FP32;

  /* 1. FP8: save blocks 4 and 1 to device entries, restore them into blocks 0 and 3. */
  int64_t logical = 0, scale_offset = 0, stride = 0;
  kvx_check(kvx_entry_layout(&layout, KVX_FORMAT_FP8, &logical, &scale_offset, &stride), "kvx_entry_layout");
  uint8_t* staging = NULL;
  hip_check(hipMalloc((void**)&staging, (size_t)(2 * stride)), "hipMalloc staging");
  const int32_t sources[2] = {4, 1}, dests[2] = {0, 3};
  const uint64_t entries[2] = {(uint64_t)(uintptr_t)staging, (uint64_t)(uintptr_t)(staging + stride)};
  kvx_check(kvx_save_blocks(pool, &layout, KVX_FORMAT_FP8, sources, entries, 2, scale_offset, compute),
            "kvx_save_blocks");
  kvx_check(kvx_restore_blocks(pool, &layout, KVX_FORMAT_FP8, dests, entries, 2, scale_offset, compute),
            "kvx_restore_blocks");
  hip_check(hipStreamSynchronize(compute), "sync");
  uint8_t* staged = (uint8_t*)malloc((size_t)(2 * stride));
  if (!staged) return 5;
  hip_check(hipMemcpy(staged, staging, (size_t)(2 * stride), hipMemcpyDeviceToHost), "download entries");
  hip_check(hipMemcpy(after_fp8, pool, bytes, hipMemcpyDeviceToHost), "download pool");

  /* 2. BF16 through the copy engine: blocks 2 and 5 -> host slots 1 and 0 -> blocks 4 and 1. */
  int64_t raw_logical = 0, raw_stride = 0;
  kvx_check(kvx_entry_layout(&layout, KVX_FORMAT_RAW, &raw_logical, NULL, &raw_stride), "kvx_entry_layout raw");
  kvx_cache* cache = NULL;
  kvx_check(kvx_cache_create(pool, &layout, KVX_FORMAT_RAW, save, restore, 0, &cache), "kvx_cache_create");
  void *save_staging = NULL, *restore_staging = NULL, *slab = NULL;
  hip_check(hipMalloc(&save_staging, (size_t)(4 * raw_stride)), "hipMalloc");
  hip_check(hipMalloc(&restore_staging, (size_t)(4 * raw_stride)), "hipMalloc");
  hip_check(hipHostMalloc(&slab, (size_t)(2 * raw_stride), 0), "hipHostMalloc");
  kvx_check(kvx_cache_set_staging(cache, save_staging, restore_staging, 4), "kvx_cache_set_staging");
  kvx_check(kvx_cache_add_slab(cache, slab, 2), "kvx_cache_add_slab");
  const int32_t raw_sources[2] = {2, 5}, slots[2] = {1, 0}, raw_dests[2] = {4, 1};
  kvx_check(kvx_cache_save(cache, raw_sources, slots, 2, compute), "kvx_cache_save");
  for (int i = 0; i < 2; ++i) kvx_check(kvx_cache_before_block_reuse(cache, raw_dests[i], compute), "reuse");
  kvx_check(kvx_cache_restore(cache, slots, raw_dests, 2, 1, compute), "kvx_cache_restore");
  hip_check(hipStreamSynchronize(compute), "sync");
  kvx_check(kvx_cache_synchronize(cache), "kvx_cache_synchronize");
  hip_check(hipMemcpy(after_raw, pool, bytes, hipMemcpyDeviceToHost), "download pool");
  int failures = 0;
  for (int i = 0; i < 2; ++i) {
    /* Each plane of a block is a contiguous run; the host slot holds the planes back to back. */
    for (int p = 0; p < 2 * L; ++p) {
      const size_t plane = (size_t)BS * H * HD;
      const uint16_t* want = after_fp8 + (size_t)p * NB * plane + (size_t)raw_sources[i] * plane;
      const uint16_t* got = after_raw + (size_t)p * NB * plane + (size_t)raw_dests[i] * plane;
      const uint16_t* slot = (const uint16_t*)((const uint8_t*)slab + (size_t)slots[i] * raw_stride) + p * plane;
      failures += memcmp(want, got, plane * 2) != 0;
      failures += memcmp(want, slot, plane * 2) != 0;
    }
  }
  int64_t saved = 0, restored = 0;
  kvx_check(kvx_cache_counters(cache, &saved, &restored, NULL), "kvx_cache_counters");
  failures += saved != 2 || restored != 2;

  /* 3. Bad arguments are error codes, with a message, and queue nothing. */
  const int32_t bad[1] = {NB};
  failures += kvx_save_blocks(pool, &layout, KVX_FORMAT_FP8, bad, entries, 1, scale_offset, compute) != KVX_E_RANGE;
  failures += strlen(kvx_last_error()) == 0;
  const int32_t twice[2] = {1, 1};
  failures += kvx_cache_save(cache, raw_sources, twice, 2, compute) != KVX_E_INVALID;
  kvx_check(kvx_cache_destroy(cache), "kvx_cache_destroy");

  FILE* out = fopen(argv[1], "wb");
  if (!out) return 6;
  fwrite(host, 1, bytes, out);
  fwrite(staged, 1, (size_t)(2 * stride), out);
  fwrite(after_fp8, 1, bytes, out);
  fwrite(after_raw, 1, bytes, out);
  fclose(out);
  hipHostFree(slab);
  hipFree(save_staging);
  hipFree(restore_staging);
  hipFree(staging);
  hipFree(pool);
  printf("c abi roundtrip: entry stride %lld, scale offset %lld, %d check failures\n", (long long)stride,
         (long long)scale_offset, failures);
  return failures ? 7 : 0;
}
