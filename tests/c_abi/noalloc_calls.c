/*
 * kvx_cache_save_noalloc from plain C, with the HIP runtime's allocation and
 * object-creation entry points interposed by this executable (linked with
 * -rdynamic, so libkvx's calls resolve here first; each wrapper forwards to
 * the runtime through dlsym(RTLD_NEXT)).
 *
 * Two copy engines over one BF16 pool, each with its own save stream and
 * pinned slab and no staging, alternate allocation-free saves of 1-3 blocks;
 * some calls follow a delay kernel on the caller's stream (the path where the
 * save kernel writes the slots itself). Every block holds one repeated 16-bit
 * value of its own, and both engines' saves pass through the device's one
 * static array, so a save whose array contents were overwritten by the other
 * engine's before its copy to the host leaves the wrong value in its slot.
 *
 * After a warm-up call per engine, the driver counts every call to the
 * interposed functions made during ITERATIONS further saves. It prints the
 * count and the number of slots whose bytes differ from a sequential shadow,
 * and exits 0 only if both are 0 and every call succeeded.
 *
 * Usage: noalloc_calls SEED ITERATIONS
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kvx.h"

#define L 2
#define NB 8
#define BS 256
#define H 2
#define HD 128
#define SLOTS 6

static int counting = 0;
static long counted = 0;
static char first_call[64] = "";

static void note(const char* name) {
  if (!counting) return;
  if (counted++ == 0) snprintf(first_call, sizeof first_call, "%s", name);
}

#define FORWARD(name, params, args)                                          \
  hipError_t name params {                                                   \
    static hipError_t(*real) params = NULL;                                  \
    if (!real) *(void**)(&real) = dlsym(RTLD_NEXT, #name);                   \
    note(#name);                                                             \
    return real ? real args : hipErrorUnknown;                               \
  }

FORWARD(hipMalloc, (void** p, size_t n), (p, n))
FORWARD(hipExtMallocWithFlags, (void** p, size_t n, unsigned int f), (p, n, f))
FORWARD(hipMallocManaged, (void** p, size_t n, unsigned int f), (p, n, f))
FORWARD(hipMallocAsync, (void** p, size_t n, hipStream_t s), (p, n, s))
FORWARD(hipHostMalloc, (void** p, size_t n, unsigned int f), (p, n, f))
FORWARD(hipHostAlloc, (void** p, size_t n, unsigned int f), (p, n, f))
FORWARD(hipMallocHost, (void** p, size_t n), (p, n))
FORWARD(hipFree, (void* p), (p))
FORWARD(hipFreeAsync, (void* p, hipStream_t s), (p, s))
FORWARD(hipHostFree, (void* p), (p))
FORWARD(hipEventCreate, (hipEvent_t* e), (e))
FORWARD(hipEventCreateWithFlags, (hipEvent_t* e, unsigned f), (e, f))
FORWARD(hipStreamCreate, (hipStream_t* s), (s))
FORWARD(hipStreamCreateWithFlags, (hipStream_t* s, unsigned int f), (s, f))

static uint64_t rng_state;

static uint32_t next_u32(void) {
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

static uint16_t block_value(int b) { return (uint16_t)(0x3C00u + 97u * (unsigned)b); }

/* k distinct values below n into out. */
static void pick_distinct(int n, int k, int* out) {
  int all[64];
  for (int i = 0; i < n; ++i) all[i] = i;
  for (int i = 0; i < k; ++i) {
    const int j = i + below(n - i);
    const int t = all[i];
    all[i] = all[j];
    all[j] = t;
    out[i] = all[i];
  }
}

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: %s SEED ITERATIONS\n", argv[0]);
    return 64;
  }
  rng_state = 0x9E3779B97F4A7C15ULL ^ (uint64_t)strtoull(argv[1], NULL, 10);
  const long iterations = strtol(argv[2], NULL, 10);

  kvx_block_layout layout;
  memset(&layout, 0, sizeof layout);
  layout.plane_stride = (int64_t)NB * BS * H * HD;
  layout.block_stride = (int64_t)BS * H * HD;
  layout.planes = 2 * L;
  layout.plane_rows = BS * H;
  layout.head_dim = HD;
  layout.num_blocks = NB;
  layout.elem_bytes = 2;
  layout.scale_dtype = KVX_SCALE_BF16;
  int64_t logical = 0, scale_offset = 0, stride = 0;
  kvx_check(kvx_entry_layout(&layout, KVX_FORMAT_RAW, &logical, &scale_offset, &stride), "kvx_entry_layout");
  const size_t plane_elems = (size_t)BS * H * HD;

  uint16_t* pool = NULL;
  hip_check(hipMalloc((void**)&pool, (size_t)2 * L * NB * plane_elems * 2), "hipMalloc pool");
  for (int p = 0; p < 2 * L; ++p)
    for (int b = 0; b < NB; ++b)
      hip_check(hipMemsetD16((hipDeviceptr_t)(pool + (size_t)p * layout.plane_stride + (size_t)b * plane_elems),
                             block_value(b), plane_elems),
                "hipMemsetD16");
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");

  hipStream_t compute;
  hip_check(hipStreamCreate(&compute), "hipStreamCreate");
  kvx_cache* cache[2];
  hipStream_t streams[2][2];
  uint8_t* slab[2];
  int shadow[2][SLOTS];
  for (int e = 0; e < 2; ++e) {
    hip_check(hipStreamCreate(&streams[e][0]), "hipStreamCreate");
    hip_check(hipStreamCreate(&streams[e][1]), "hipStreamCreate");
    kvx_check(kvx_cache_create(pool, &layout, KVX_FORMAT_RAW, streams[e][0], streams[e][1], 0, &cache[e]),
              "kvx_cache_create");
    hip_check(hipHostMalloc((void**)&slab[e], (size_t)SLOTS * stride, 0), "hipHostMalloc");
    memset(slab[e], 0xAB, (size_t)SLOTS * stride);
    kvx_check(kvx_cache_add_slab(cache[e], slab[e], SLOTS), "kvx_cache_add_slab");
    for (int s = 0; s < SLOTS; ++s) shadow[e][s] = -1;
  }

  long calls = 0;
  for (long it = -2; it < iterations; ++it) {
    if (it == 0) counting = 1;  /* after one warm-up call per engine */
    const int e = (int)((it + 2) % 2);
    const int n = 1 + below(3);
    int ids[3], slots[3];
    pick_distinct(NB, n, ids);
    pick_distinct(SLOTS, n, slots);
    if (below(3) == 0) kvx_check(kvx_sleep(compute, 20), "kvx_sleep");
    kvx_check(kvx_cache_save_noalloc(cache[e], ids, slots, n, compute), "kvx_cache_save_noalloc");
    for (int i = 0; i < n; ++i) shadow[e][slots[i]] = ids[i];
    ++calls;
  }
  counting = 0;

  long mismatches = 0;
  for (int e = 0; e < 2; ++e) {
    kvx_check(kvx_cache_synchronize(cache[e]), "kvx_cache_synchronize");
    for (int s = 0; s < SLOTS; ++s) {
      const uint16_t* entry = (const uint16_t*)(slab[e] + (size_t)s * stride);
      const size_t elems = (size_t)logical / 2;
      if (shadow[e][s] < 0) {
        if (((const uint8_t*)entry)[0] != 0xAB) ++mismatches;
        continue;
      }
      const uint16_t want = block_value(shadow[e][s]);
      for (size_t k = 0; k < elems; ++k)
        if (entry[k] != want) {
          ++mismatches;
          break;
        }
    }
  }
  printf("%ld noalloc calls over 2 engines; %ld allocation or creation calls during them%s%s; %ld mismatches\n",
         calls, counted, counted ? ", first: " : "", first_call, mismatches);
  for (int e = 0; e < 2; ++e) {
    kvx_check(kvx_cache_destroy(cache[e]), "kvx_cache_destroy");
    hip_check(hipHostFree(slab[e]), "hipHostFree");
  }
  hip_check(hipFree(pool), "hipFree");
  return counted == 0 && mismatches == 0 ? 0 : 1;
}
