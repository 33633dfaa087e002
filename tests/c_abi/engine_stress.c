/*
 * A seeded random workload for libkvx's copy engine, from plain C: saves
 * (staged, kernel-written behind a busy caller stream, and through
 * kvx_cache_save_noalloc), restores (staged, prefetches, and waited ones the
 * kernel reads from the slots), caller writes after before_block_reuse,
 * before_block_use, delay kernels on every stream, staging re-cuts and slab
 * resets. BF16 entries: every block holds one repeated 16-bit value, so a
 * block or slot that mixes two writes, or holds a stale one, shows up at the
 * checkpoints, where everything is synchronised and compared with a
 * sequential shadow of the same calls.
 *
 * It is the host-side target for a sanitizer build as well (tests/c_abi/
 * Makefile, `make asan`): the engine's event pool, slot tables and batching
 * run here with every path taken.
 *
 * Usage: engine_stress SEED ITERATIONS [split:0|1] [debug flags]
 * Prints "N mismatches" and exits 0 only if N is 0 and every call succeeded.
 * The debug flags (KVX_DEBUG_*, kvx_cache_set_debug) drop ordering rules, for
 * negative controls.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kvx.h"

#define L 2
#define NB 12
#define BS 16
#define H 2
#define HD 64
#define SLOTS 10
#define STAGING 4

static uint64_t rng_state;

static uint32_t next_u32(void) {
  /* xorshift64* */
  rng_state ^= rng_state >> 12;
  rng_state ^= rng_state << 25;
  rng_state ^= rng_state >> 27;
  return (uint32_t)((rng_state * 2685821657736338717ULL) >> 32);
}

static int below(int n) { return (int)(next_u32() % (uint32_t)n); }

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

/* k distinct values below n into out; returns k. */
static int pick_distinct(int n, int k, int* out) {
  int all[64];
  for (int i = 0; i < n; ++i) all[i] = i;
  for (int i = 0; i < k; ++i) {
    const int j = i + below(n - i);
    const int t = all[i];
    all[i] = all[j];
    all[j] = t;
    out[i] = all[i];
  }
  return k;
}

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: %s SEED ITERATIONS [split]\n", argv[0]);
    return 1;
  }
  rng_state = 0x9E3779B97F4A7C15ULL ^ (uint64_t)strtoull(argv[1], NULL, 10);
  const int iterations = atoi(argv[2]);
  const int split = argc > 3 ? atoi(argv[3]) : 1;
  const int debug = argc > 4 ? atoi(argv[4]) : 0;

  const size_t plane_elems = (size_t)BS * H * HD;
  const size_t pool_elems = (size_t)2 * L * NB * plane_elems;
  const size_t block_bytes = (size_t)2 * L * plane_elems * 2;
  kvx_block_layout layout = {(int64_t)(NB * plane_elems), (int64_t)plane_elems, 2 * L, BS * H, HD, NB, 2,
                             KVX_SCALE_BF16};
  int64_t logical = 0, scale_offset = 0, stride = 0;
  kvx_check(kvx_entry_layout(&layout, KVX_FORMAT_RAW, &logical, &scale_offset, &stride), "entry layout");

  uint16_t* pool = NULL;
  uint8_t *save_staging = NULL, *restore_staging = NULL, *slab = NULL;
  hip_check(hipMalloc((void**)&pool, pool_elems * 2), "hipMalloc pool");
  hip_check(hipMalloc((void**)&save_staging, (size_t)STAGING * stride), "hipMalloc staging");
  hip_check(hipMalloc((void**)&restore_staging, (size_t)STAGING * stride), "hipMalloc staging");
  hip_check(hipHostMalloc((void**)&slab, (size_t)SLOTS * stride, 0), "hipHostMalloc slab");
  hipStream_t compute, save_s, restore_s;
  hip_check(hipStreamCreate(&compute), "stream");
  hip_check(hipStreamCreate(&save_s), "stream");
  hip_check(hipStreamCreate(&restore_s), "stream");
  if (!split) restore_s = save_s;
  uint8_t* restore_area = split ? restore_staging : save_staging;

  /* Shadow: the value every block and slot holds after all calls so far, in call order (-1: never written). */
  int block_val[NB], slot_val[SLOTS];
  int next_val = 1;
  uint16_t* host_pool = (uint16_t*)malloc(pool_elems * 2);
  for (int b = 0; b < NB; ++b) {
    block_val[b] = next_val++;
    for (int p = 0; p < 2 * L; ++p)
      for (size_t e = 0; e < plane_elems; ++e) host_pool[((size_t)p * NB + b) * plane_elems + e] = (uint16_t)block_val[b];
  }
  for (int s = 0; s < SLOTS; ++s) slot_val[s] = -1;
  hip_check(hipMemcpy(pool, host_pool, pool_elems * 2, hipMemcpyHostToDevice), "hipMemcpy pool");

  kvx_cache* cache = NULL;
  kvx_check(kvx_cache_create(pool, &layout, KVX_FORMAT_RAW, save_s, restore_s, 0, &cache), "create");
  kvx_check(kvx_cache_set_staging(cache, save_staging, restore_area, STAGING), "staging");
  kvx_check(kvx_cache_add_slab(cache, slab, SLOTS), "slab");
  kvx_check(kvx_cache_set_debug(cache, debug), "debug");

  long mismatches = 0, checkpoints = 0;
  const char* paths[] = {"save", "restore", "write", "use", "sleep", "noalloc", "restage", "checkpoint", "reset"};
  long counts[9] = {0};
  for (int it = 0; it < iterations; ++it) {
    const int r = below(100);
    int ids[8], slots[8];
    if (r < 28) { /* save 1-4 blocks into distinct slots */
      const int k = 1 + below(4);
      pick_distinct(NB, k, ids);
      pick_distinct(SLOTS, k, slots);
      if (below(3) == 0) kvx_check(kvx_sleep(compute, below(150)), "sleep");  /* a busy caller: kernel-written */
      kvx_check(kvx_cache_save(cache, ids, slots, k, compute), "save");
      for (int i = 0; i < k; ++i) slot_val[slots[i]] = block_val[ids[i]];
      counts[0]++;
    } else if (r < 52) { /* restore 1-3 written slots into distinct blocks */
      int written[SLOTS], nw = 0;
      for (int s = 0; s < SLOTS; ++s)
        if (slot_val[s] >= 0) written[nw++] = s;
      if (nw == 0) continue;
      const int k = 1 + below(nw < 3 ? nw : 3);
      int order[SLOTS];
      pick_distinct(nw, k, order);
      for (int i = 0; i < k; ++i) slots[i] = written[order[i]];
      pick_distinct(NB, k, ids);
      const int wait = below(2);
      kvx_check(kvx_cache_restore(cache, slots, ids, k, wait, compute), "restore");
      for (int i = 0; i < k; ++i) block_val[ids[i]] = slot_val[slots[i]];
      counts[1]++;
    } else if (r < 64) { /* the caller writes a block */
      const int b = below(NB);
      kvx_check(kvx_cache_before_block_reuse(cache, b, compute), "before_block_reuse");
      block_val[b] = next_val++;
      for (int p = 0; p < 2 * L; ++p)
        hip_check(hipMemsetD16Async((hipDeviceptr_t)(pool + ((size_t)p * NB + b) * plane_elems),
                                    (unsigned short)block_val[b], plane_elems, compute), "memset");
      counts[2]++;
    } else if (r < 72) {
      kvx_check(kvx_cache_before_block_use(cache, below(NB), compute), "before_block_use");
      counts[3]++;
    } else if (r < 84) {
      hipStream_t streams[3] = {compute, save_s, restore_s};
      kvx_check(kvx_sleep(streams[below(3)], below(300)), "sleep");
      counts[4]++;
    } else if (r < 90) { /* allocation-free save of 1-3 blocks */
      const int k = 1 + below(3);
      pick_distinct(NB, k, ids);
      pick_distinct(SLOTS, k, slots);
      kvx_check(kvx_cache_save_noalloc(cache, ids, slots, k, compute), "save_noalloc");
      for (int i = 0; i < k; ++i) slot_val[slots[i]] = block_val[ids[i]];
      counts[5]++;
    } else if (r < 94) { /* re-cut the staging: copies queued keep their areas, which stay allocated */
      kvx_check(kvx_cache_set_staging(cache, save_staging, restore_area, 1 + below(STAGING)), "staging");
      counts[6]++;
    } else if (r < 99) { /* checkpoint */
      kvx_check(kvx_cache_synchronize(cache), "synchronize");
      hip_check(hipStreamSynchronize(compute), "sync");
      hip_check(hipMemcpy(host_pool, pool, pool_elems * 2, hipMemcpyDeviceToHost), "read pool");
      for (int b = 0; b < NB; ++b)
        for (int p = 0; p < 2 * L; ++p)
          for (size_t e = 0; e < plane_elems; ++e)
            if (host_pool[((size_t)p * NB + b) * plane_elems + e] != (uint16_t)block_val[b]) {
              if (mismatches < 5) fprintf(stderr, "iteration %d: block %d plane %d\n", it, b, p);
              ++mismatches;
              p = 2 * L;
              break;
            }
      for (int s = 0; s < SLOTS; ++s) {
        if (slot_val[s] < 0) continue;
        const uint16_t* entry = (const uint16_t*)(slab + (size_t)s * stride);
        for (size_t e = 0; e < block_bytes / 2; ++e)
          if (entry[e] != (uint16_t)slot_val[s]) {
            if (mismatches < 5) fprintf(stderr, "iteration %d: slot %d\n", it, s);
            ++mismatches;
            break;
          }
      }
      ++checkpoints;
      counts[7]++;
    } else { /* drop the slabs and attach the same memory again: every slot forgets its entry */
      kvx_check(kvx_cache_reset_slabs(cache), "reset_slabs");
      kvx_check(kvx_cache_add_slab(cache, slab, SLOTS), "slab");
      for (int s = 0; s < SLOTS; ++s) slot_val[s] = -1;
      counts[8]++;
    }
  }
  /* Bad arguments come back as error codes and change nothing. */
  int dup[2] = {0, 0}, one[2] = {0, 1};
  if (kvx_cache_save(cache, one, dup, 2, compute) != KVX_E_INVALID) ++mismatches;
  if (kvx_cache_restore(cache, one, dup, 2, 1, compute) != KVX_E_INVALID) ++mismatches;
  int64_t saved = 0, restored = 0, waits = 0;
  kvx_check(kvx_cache_counters(cache, &saved, &restored, &waits), "counters");
  kvx_check(kvx_cache_destroy(cache), "destroy");
  hip_check(hipStreamSynchronize(compute), "sync");
  printf("%d iterations, %ld checkpoints; calls:", iterations, checkpoints);
  for (int i = 0; i < 9; ++i) printf(" %s %ld", paths[i], counts[i]);
  printf("; %lld blocks saved, %lld restored, %lld stream waits\n", (long long)saved, (long long)restored,
         (long long)waits);
  printf("%ld mismatches\n", mismatches);
  free(host_pool);
  hip_check(hipHostFree(slab), "hipHostFree");
  hip_check(hipFree(pool), "hipFree");
  hip_check(hipFree(save_staging), "hipFree");
  hip_check(hipFree(restore_staging), "hipFree");
  return mismatches == 0 ? 0 : 4;
}
