// C ABI of libkvx: argument checking, batching, and the copy engine that
// orders saves and restores against the caller's compute stream.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <new>
#include <utility>
#include <vector>

#include "kvx_internal.h"

namespace kvx {

static thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return KVX_OK;
  return set_error((int)err, "%s: %s (hipError_t %d)", what, hipGetErrorString(err), (int)err);
}

// No layout, tensor, entry run or slab this library addresses may span more
// than this many bytes (1 TiB, above any MI355X pool or host slab). Every size
// the kernels and the entry sizing compute then fits int64 with room to spare.
constexpr int64_t kMaxSpan = int64_t{1} << 40;

// *out = the product of `factors`; false if a factor is negative or the
// product overflows or exceeds kMaxSpan.
static bool span_product(std::initializer_list<int64_t> factors, int64_t* out) {
  int64_t p = 1;
  for (int64_t f : factors)
    if (f < 0 || __builtin_mul_overflow(p, f, &p) || p > kMaxSpan) return false;
  *out = p;
  return true;
}

// Bytes from the first element of a strided run of `count` rows of `row`
// elements (rows `stride` elements apart) to the end of its last row, or -1 if
// that is more than kMaxSpan bytes.
static int64_t strided_span(int64_t count, int64_t stride, int64_t row, int64_t elem_bytes) {
  int64_t lead, elems, bytes;
  if (count <= 0) return 0;
  if (__builtin_mul_overflow(count - 1, stride, &lead) || __builtin_add_overflow(lead, row, &elems) ||
      !span_product({elems, elem_bytes}, &bytes))
    return -1;
  return bytes;
}

int check_layout(const kvx_block_layout* l, int32_t format) {
  if (!l) return set_error(KVX_E_INVALID, "layout is NULL");
  if (format != KVX_FORMAT_RAW && format != KVX_FORMAT_FP8)
    return set_error(KVX_E_INVALID, "unknown entry format %d", format);
  if (l->planes <= 0 || l->plane_rows <= 0 || l->head_dim <= 0 || l->num_blocks <= 0)
    return set_error(KVX_E_INVALID, "layout sizes must be positive (planes %d, rows %d, head_dim %d, blocks %d)",
                     l->planes, l->plane_rows, l->head_dim, l->num_blocks);
  if (l->plane_stride < 0 || l->block_stride < 0)
    return set_error(KVX_E_INVALID, "layout strides must be non-negative");
  const int64_t plane_elems = (int64_t)l->plane_rows * l->head_dim;
  if (l->num_blocks > 1 && l->block_stride < plane_elems)
    return set_error(KVX_E_INVALID, "block_stride %lld overlaps a %lld-element plane",
                     (long long)l->block_stride, (long long)plane_elems);
  if (format == KVX_FORMAT_FP8) {
    if (l->elem_bytes != 2) return set_error(KVX_E_UNSUPPORTED, "FP8 entries need bf16 (2-byte) pool elements");
    if (l->scale_dtype != KVX_SCALE_BF16 && l->scale_dtype != KVX_SCALE_FP32)
      return set_error(KVX_E_INVALID, "unknown scale dtype %d", l->scale_dtype);
  } else if (l->elem_bytes != 1 && l->elem_bytes != 2 && l->elem_bytes != 4 && l->elem_bytes != 8) {
    return set_error(KVX_E_INVALID, "elem_bytes must be 1, 2, 4 or 8");
  }
  int64_t block_bytes;
  if (!span_product({l->planes, l->plane_rows, l->head_dim, l->elem_bytes}, &block_bytes))
    return set_error(KVX_E_UNSUPPORTED, "a block of this layout spans more than 2^40 bytes");
  // The pool the layout describes ends with the last plane of the last block.
  int64_t blocks_lead, planes_lead, extent_elems, extent_bytes;
  if (__builtin_mul_overflow((int64_t)l->num_blocks - 1, l->block_stride, &blocks_lead) ||
      __builtin_mul_overflow((int64_t)l->planes - 1, l->plane_stride, &planes_lead) ||
      __builtin_add_overflow(blocks_lead, planes_lead, &extent_elems) ||
      __builtin_add_overflow(extent_elems, plane_elems, &extent_elems) ||
      !span_product({extent_elems, l->elem_bytes}, &extent_bytes))
    return set_error(KVX_E_UNSUPPORTED, "the layout spans more than 2^40 bytes");
  // Launch grids: blocks * planes * tiles must fit a 32-bit workgroup count.
  if ((int64_t)kMaxBatch * l->planes * ((plane_elems * l->elem_bytes) / 16 + 1) > (int64_t)INT32_MAX)
    return set_error(KVX_E_UNSUPPORTED, "block geometry too large for one launch");
  return KVX_OK;
}

static void entry_sizes(const kvx_block_layout& l, int32_t format, int64_t* logical, int64_t* scale_off,
                        int64_t* stride) {
  const int64_t rows = (int64_t)l.planes * l.plane_rows;
  int64_t payload, bytes;
  if (format == KVX_FORMAT_FP8) {
    payload = rows * l.head_dim;
    const int64_t sb = l.scale_dtype == KVX_SCALE_BF16 ? 2 : 4;
    // The reference budgets payload + scales (cpu_prefix_cache.py:98-100).
    *logical = payload + rows * sb;
    *scale_off = (payload + 255) / 256 * 256;
    bytes = *scale_off + rows * sb;
  } else {
    payload = rows * l.head_dim * l.elem_bytes;
    *logical = payload;
    *scale_off = 0;
    bytes = payload;
  }
  *stride = (bytes + 255) / 256 * 256;
}

// True if two of the n values are equal: two copies into one destination
// in one call would race, so calls reject it. Lists of up to kMaxBatch
// values are sorted on the stack (no heap allocation).
static bool any_repeat(const int32_t* v, int64_t n) {
  if (n < 2) return false;
  if (n <= kMaxBatch) {
    int32_t s[kMaxBatch];
    std::copy(v, v + n, s);
    std::sort(s, s + n);
    return std::adjacent_find(s, s + n) != s + n;
  }
  std::vector<int32_t> s(v, v + n);
  std::sort(s.begin(), s.end());
  return std::adjacent_find(s.begin(), s.end()) != s.end();
}

// True if two of the byte ranges [start, end) share a byte.
static bool any_overlap(std::vector<std::pair<uint64_t, uint64_t>>& ranges) {
  std::sort(ranges.begin(), ranges.end());
  for (size_t i = 1; i < ranges.size(); ++i)
    if (ranges[i].first < ranges[i - 1].second) return true;
  return false;
}

// Splits (ids, entries) into launches of at most kMaxBatch blocks.
static int run_batches(bool save, void* pool, const kvx_block_layout* layout, int32_t format,
                       const int32_t* ids, const uint64_t* entries, int32_t n, int64_t scale_offset,
                       hipStream_t stream) {
  int rc = check_layout(layout, format);
  if (rc) return rc;
  if (n < 0) return set_error(KVX_E_INVALID, "negative block count");
  if (n == 0) return KVX_OK;
  if (!pool || !ids || !entries) return set_error(KVX_E_INVALID, "NULL pool, block id or entry array");
  const int64_t sbytes = layout->scale_dtype == KVX_SCALE_BF16 ? 2 : 4;
  const bool vec_pool = layout->head_dim % 8 == 0;
  for (int32_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= layout->num_blocks)
      return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", ids[i], layout->num_blocks);
    if (!entries[i]) return set_error(KVX_E_INVALID, "entry %d is NULL", i);
    const uint64_t align = format == KVX_FORMAT_FP8 ? (vec_pool ? 8 : 1) : 2;
    if (entries[i] % align) return set_error(KVX_E_INVALID, "entry %d is not %llu-byte aligned", i,
                                             (unsigned long long)align);
    if (format == KVX_FORMAT_FP8 && (entries[i] + (uint64_t)scale_offset) % (uint64_t)sbytes)
      return set_error(KVX_E_INVALID, "scales of entry %d are misaligned", i);
  }
  if ((uintptr_t)pool % 2) return set_error(KVX_E_INVALID, "pool is not 2-byte aligned");
  if (save) {
    // Entries are written: no payload or scale range may share a byte with another.
    const int64_t rows = (int64_t)layout->planes * layout->plane_rows;
    const bool fp8 = format == KVX_FORMAT_FP8;
    const uint64_t payload = (uint64_t)(rows * layout->head_dim * (fp8 ? 1 : layout->elem_bytes));
    std::vector<std::pair<uint64_t, uint64_t>> ranges;
    ranges.reserve(fp8 ? 2 * (size_t)n : (size_t)n);
    for (int32_t i = 0; i < n; ++i) {
      ranges.emplace_back(entries[i], entries[i] + payload);
      if (fp8) {
        const uint64_t scales = entries[i] + (uint64_t)scale_offset;
        ranges.emplace_back(scales, scales + (uint64_t)(rows * sbytes));
      }
    }
    if (any_overlap(ranges)) return set_error(KVX_E_INVALID, "entries or their scales overlap in one save");
  } else if (any_repeat(ids, n)) {
    return set_error(KVX_E_INVALID, "a block appears twice in one restore");
  }
  BlockBatch b;
  for (int32_t base = 0; base < n; base += kMaxBatch) {
    b.n = std::min(kMaxBatch, n - base);
    for (int32_t i = 0; i < b.n; ++i) {
      b.ids[i] = ids[base + i];
      b.entries[i] = entries[base + i];
    }
    const bool vec = vector_access_ok(pool, *layout, b.entries, b.n);
    hipError_t err = save ? launch_save(pool, *layout, format, b, scale_offset, vec, 0, stream)
                          : launch_restore(pool, *layout, format, b, scale_offset, vec, 0, stream);
    if (err != hipSuccess) return hip_status(err, save ? "save kernel launch" : "restore kernel launch");
  }
  return KVX_OK;
}

// Token-granular copy between the blocks in `table` and a dense buffer.
static int token_copy(bool gather, void* pool, const kvx_block_layout* l, const int32_t* table, int32_t table_len,
                      int64_t num_rows, void* dense, hipStream_t stream) {
  int rc = check_layout(l, KVX_FORMAT_RAW);
  if (rc) return rc;
  if (num_rows < 0 || table_len < 0) return set_error(KVX_E_INVALID, "negative row or block count");
  if (num_rows == 0) return KVX_OK;
  if (!pool || !dense || !table) return set_error(KVX_E_INVALID, "NULL pool, buffer or block table");
  if ((uintptr_t)pool % 2 || (uintptr_t)dense % 2) return set_error(KVX_E_INVALID, "buffers must be 2-byte aligned");
  int64_t dense_bytes;
  if (!span_product({l->planes, num_rows, l->head_dim, l->elem_bytes}, &dense_bytes))
    return set_error(KVX_E_UNSUPPORTED, "%lld rows span more than 2^40 bytes", (long long)num_rows);
  const int64_t row_bytes = (int64_t)l->head_dim * l->elem_bytes;
  const int64_t plane_bytes = (int64_t)l->plane_rows * row_bytes;
  const int64_t nblocks = (num_rows + l->plane_rows - 1) / l->plane_rows;
  if (nblocks > table_len)
    return set_error(KVX_E_RANGE, "%lld rows need %lld blocks, the table has %d", (long long)num_rows,
                     (long long)nblocks, table_len);
  for (int64_t i = 0; i < nblocks; ++i)
    if (table[i] < 0 || table[i] >= l->num_blocks)
      return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", table[i], l->num_blocks);
  if (!gather && any_repeat(table, nblocks)) return set_error(KVX_E_INVALID, "a block appears twice in one scatter");
  const int64_t dense_plane_stride = num_rows * row_bytes;
  const int64_t tail_bytes = (num_rows - (nblocks - 1) * l->plane_rows) * row_bytes;
  BlockBatch b;
  for (int64_t base = 0; base < nblocks; base += kMaxBatch) {
    b.n = (int32_t)std::min<int64_t>(kMaxBatch, nblocks - base);
    for (int32_t i = 0; i < b.n; ++i) {
      b.ids[i] = table[base + i];
      b.entries[i] = (uint64_t)(uintptr_t)dense + (uint64_t)((base + i) * plane_bytes);
    }
    const int64_t last = base + b.n == nblocks ? tail_bytes : plane_bytes;
    const bool vec = vector_access_ok(pool, *l, b.entries, b.n);
    hipError_t err = launch_token_copy(gather, pool, *l, b, vec, dense_plane_stride, last, stream);
    if (err != hipSuccess) return hip_status(err, gather ? "token gather launch" : "token scatter launch");
  }
  return KVX_OK;
}

// Token-granular FP8 copy between the blocks in `table` and a dense
// [planes][num_rows][hd] e4m3 payload with one scale per row in a dense
// [planes][num_rows] array.
static int token_fp8(bool gather, void* pool, const kvx_block_layout* l, const int32_t* table, int32_t table_len,
                     int64_t num_rows, void* payload, void* scales, hipStream_t stream) {
  int rc = check_layout(l, KVX_FORMAT_FP8);
  if (rc) return rc;
  if (num_rows < 0 || table_len < 0) return set_error(KVX_E_INVALID, "negative row or block count");
  if (num_rows == 0) return KVX_OK;
  if (!pool || !payload || !scales || !table) return set_error(KVX_E_INVALID, "NULL pool, payload, scales or table");
  const int64_t sb = l->scale_dtype == KVX_SCALE_BF16 ? 2 : 4;
  if ((uintptr_t)pool % 2) return set_error(KVX_E_INVALID, "pool is not 2-byte aligned");
  if ((uintptr_t)scales % (uintptr_t)sb) return set_error(KVX_E_INVALID, "scales are not %lld-byte aligned", (long long)sb);
  int64_t payload_span, scale_span;
  if (!span_product({l->planes, num_rows, l->head_dim}, &payload_span) ||
      !span_product({l->planes, num_rows, sb}, &scale_span))
    return set_error(KVX_E_UNSUPPORTED, "%lld rows span more than 2^40 bytes", (long long)num_rows);
  const int64_t R = l->plane_rows, hd = l->head_dim;
  const int64_t nblocks = (num_rows + R - 1) / R;
  if (nblocks > table_len)
    return set_error(KVX_E_RANGE, "%lld rows need %lld blocks, the table has %d", (long long)num_rows,
                     (long long)nblocks, table_len);
  for (int64_t i = 0; i < nblocks; ++i)
    if (table[i] < 0 || table[i] >= l->num_blocks)
      return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", table[i], l->num_blocks);
  if (!gather && any_repeat(table, nblocks)) return set_error(KVX_E_INVALID, "a block appears twice in one scatter");
  const uintptr_t p0 = (uintptr_t)payload, s0 = (uintptr_t)scales;
  const uintptr_t payload_bytes = (uintptr_t)(l->planes * num_rows * hd), scale_bytes = (uintptr_t)(l->planes * num_rows * sb);
  if (gather && p0 < s0 + scale_bytes && s0 < p0 + payload_bytes)
    return set_error(KVX_E_INVALID, "payload and scales overlap");
  // Vector kernels store scales 16 bytes at a time from tile-aligned rows.
  const bool aligned = p0 % 16 == 0 && s0 % 16 == 0 && (num_rows * hd) % 16 == 0 && (num_rows * sb) % 16 == 0 &&
                       (R * sb) % 16 == 0;
  TokenSpan span{num_rows * hd, num_rows * sb, R * (sb - hd), (int32_t)R};
  BlockBatch b;
  for (int64_t base = 0; base < nblocks; base += kMaxBatch) {
    b.n = (int32_t)std::min<int64_t>(kMaxBatch, nblocks - base);
    for (int32_t i = 0; i < b.n; ++i) {
      b.ids[i] = table[base + i];
      b.entries[i] = (uint64_t)(p0 + (uintptr_t)((base + i) * R * hd));
    }
    span.last_rows = (int32_t)(base + b.n == nblocks ? num_rows - (nblocks - 1) * R : R);
    // Entry i's scales: scales + (base + i) * R * sb = entries[i] + scale_offset + i * scale_entry_step.
    const int64_t scale_offset = (int64_t)(s0 + (uintptr_t)(base * R * sb)) - (int64_t)(p0 + (uintptr_t)(base * R * hd));
    const bool vec = aligned && vector_access_ok(pool, *l, b.entries, b.n);
    hipError_t err = launch_token_fp8(gather, pool, *l, b, scale_offset, span, vec, stream);
    if (err != hipSuccess) return hip_status(err, gather ? "FP8 token gather launch" : "FP8 token scatter launch");
  }
  return KVX_OK;
}

}  // namespace kvx

using namespace kvx;

// ---------------------------------------------------------------------------
// Copy engine

namespace {

struct Event {
  hipEvent_t ev = nullptr;
  int refs = 0;
  hipStream_t stream = nullptr;  // where it was last recorded
};

struct Slab {
  uint8_t* base;
  int32_t first;
  int32_t count;
};

// Makes the cache's device current for one call and restores the caller's
// current device afterwards (torch and other callers keep their own notion of
// the current device; the engine must not change it behind their backs).
class DeviceScope {
 public:
  int enter(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ == device) return KVX_OK;
    const int rc = hip_status(hipSetDevice(device), "hipSetDevice");
    changed_ = rc == KVX_OK;
    return rc;
  }
  ~DeviceScope() {
    if (changed_ && prev_ >= 0) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1;
  bool changed_ = false;
};

}  // namespace

// Staging of kvx_cache_save_noalloc, for callers that cannot allocate device
// memory. Every device that runs the library holds its own copy of this
// array, at its own address, until the process ends. In host code the name
// `scratch` is only a host-side stand-in: kernels and copies get the device
// address that scratch_setup() looks up per device.
static __device__ __align__(256) uint8_t scratch[KVX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;

struct ScratchTable {
  std::mutex mu;
  bool looked_up[kMaxScratchDevices] = {};
  int status[kMaxScratchDevices] = {};        // KVX_OK, or the code of a failed lookup
  uint8_t* address[kMaxScratchDevices] = {};  // device address of `scratch` on each device
  // Per device: the latest allocation-free save's copies out of the array
  // (recorded on that save's stream), and a mutex held while a call queues
  // its wait, its work and the new record, so calls of different caches
  // follow each other in the order they are made.
  std::mutex use_mu[kMaxScratchDevices];
  hipEvent_t last_use[kMaxScratchDevices] = {};
  hipStream_t last_stream[kMaxScratchDevices] = {};
};

ScratchTable g_scratch;

// Looks up `scratch` on `device`, which must be current; once per device.
// Writes the device's address (nullptr if the lookup failed) and status.
void scratch_setup(int device, uint8_t** address, int* status) {
  *address = nullptr;
  if (device < 0 || device >= kMaxScratchDevices) {
    *status = set_error(KVX_E_UNSUPPORTED, "static staging supports devices 0..%d", kMaxScratchDevices - 1);
    return;
  }
  std::lock_guard<std::mutex> lock(g_scratch.mu);
  if (!g_scratch.looked_up[device]) {
    void* p = nullptr;
    hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err == hipSuccess) err = hipEventCreateWithFlags(&g_scratch.last_use[device], hipEventDisableTiming);
    if (err != hipSuccess) {
      (void)hipGetLastError();  // leave no error behind for the caller's next HIP call
      g_scratch.status[device] = (int)err;
    } else {
      g_scratch.address[device] = (uint8_t*)p;
    }
    g_scratch.looked_up[device] = true;
  }
  *address = g_scratch.address[device];
  *status = g_scratch.status[device];
}

}  // namespace

struct kvx_cache {
  int device = 0;
  uint8_t* pool = nullptr;
  kvx_block_layout layout{};
  int32_t format = KVX_FORMAT_RAW;
  int64_t logical_bytes = 0, scale_offset = 0, entry_stride = 0;
  bool split = false;
  hipStream_t save_stream = nullptr, restore_stream = nullptr;
  hipEvent_t marker = nullptr;  // makes one stream wait for everything queued on another
  uint8_t* save_staging = nullptr;
  uint8_t* restore_staging = nullptr;
  int32_t staging_entries = 0;
  std::vector<Slab> slabs;
  int32_t num_slots = 0;
  std::vector<Event*> pending_save, pending_restore;  // per GPU block
  std::vector<Event*> slot_read, slot_saved;          // per host slot
  std::vector<Event*> free_events, all_events;
  Event* last_save = nullptr;  // the latest save's completion
  // Per caller stream, the completion of the latest restore queued on it
  // (waited direct restores), until seen complete. Work on one stream
  // completes in order, so the latest covers the earlier ones. synchronize
  // and destroy wait for them as for the engine's own streams: such a
  // restore still reads its host slot, and the slot's memory may be released
  // once those calls return.
  std::vector<std::pair<hipStream_t, Event*>> caller_reads;
  bool host_reads_ok = false;  // restores may read host slots with the striding kernel
  int64_t saved = 0, restored = 0, waits = 0;
  int64_t d2h_copies = 0, d2h_bytes = 0, h2d_copies = 0, h2d_bytes = 0;  // DMA transfers queued
  int32_t debug = 0;  // KVX_DEBUG_* negative-control flags
  // kvx_cache_save_noalloc: the device's static staging and the status of its
  // lookup, and the one event every such save records (created with the
  // cache and never returned to the pool). Saves run in order on the save
  // stream, so a later record of this event completes after every earlier
  // one: waiting for its latest record orders at least as strongly.
  uint8_t* static_staging = nullptr;
  int static_staging_status = KVX_E_STATE;
  Event* static_done = nullptr;

  uint8_t* host_entry(int32_t slot) const {
    for (const Slab& s : slabs)
      if (slot >= s.first && slot < s.first + s.count) return s.base + (int64_t)(slot - s.first) * entry_stride;
    return nullptr;
  }

  int new_event(Event** out) {
    Event* e;
    if (!free_events.empty()) {
      e = free_events.back();
      free_events.pop_back();
    } else {
      e = new (std::nothrow) Event();
      if (!e) return set_error(KVX_E_STATE, "out of host memory for events");
      hipError_t err = hipEventCreateWithFlags(&e->ev, hipEventDisableTiming);
      if (err != hipSuccess) {
        delete e;
        return hip_status(err, "hipEventCreateWithFlags");
      }
      all_events.push_back(e);
      // unref() returns events with push_back: with this capacity it never
      // reallocates, so calls that create no event allocate nothing.
      free_events.reserve(all_events.size());
    }
    e->refs = 0;
    *out = e;
    return KVX_OK;
  }

  void unref(Event*& e) {
    if (!e) return;
    if (--e->refs == 0) free_events.push_back(e);
    e = nullptr;
  }

  void assign(Event*& slot, Event* e) {
    unref(slot);
    ++e->refs;
    slot = e;
  }

  void release_if_unused(Event* e) {
    if (e->refs == 0) free_events.push_back(e);
  }

  // Tracks `e`, just recorded on caller stream `s`, in place of the stream's
  // previous one; drops other streams' events that have completed.
  void track_caller_read(hipStream_t s, Event* e) {
    ++e->refs;
    size_t kept = 0;
    bool placed = false;
    for (auto& [stream, t] : caller_reads) {
      if (stream == s) {
        unref(t);
        t = e;
        placed = true;
      } else if (hipEventQuery(t->ev) == hipSuccess) {
        unref(t);
        continue;
      }
      caller_reads[kept++] = {stream, t};
    }
    caller_reads.resize(kept);
    if (!placed) caller_reads.emplace_back(s, e);
  }

  // Blocks until every tracked caller-stream restore has completed.
  int sync_caller_reads() {
    int rc = KVX_OK;
    for (auto& [stream, t] : caller_reads) {
      const int r = hip_status(hipEventSynchronize(t->ev), "hipEventSynchronize");
      if (!rc) rc = r;
      unref(t);
    }
    caller_reads.clear();
    return rc;
  }

  int record(Event* e, hipStream_t s) {
    e->stream = s;
    return hip_status(hipEventRecord(e->ev, s), "hipEventRecord");
  }

  // The save kernel just queued on `s` is the last reader of these pool
  // blocks: their pending_save becomes an event recorded now.
  int release_blocks_after(const int32_t* ids, int32_t n, hipStream_t s) {
    Event* read = nullptr;
    int rc = new_event(&read);
    if (!rc) rc = record(read, s);
    if (!rc)
      for (int32_t i = 0; i < n; ++i) assign(pending_save[ids[i]], read);
    if (read) release_if_unused(read);
    return rc;
  }

  // `s` waits for `e`. An event recorded on `s` itself, or one that has
  // already completed, orders nothing queued from now on, so it costs no
  // wait: a one-block restore used to queue one on its slot's long-finished
  // save.
  int wait_event(hipStream_t s, Event* e) {
    if (e->stream == s) return KVX_OK;
    const hipError_t q = hipEventQuery(e->ev);
    if (q == hipSuccess) return KVX_OK;
    if (q != hipErrorNotReady) return hip_status(q, "hipEventQuery");
    return queue_wait(s, e);
  }

  int queue_wait(hipStream_t s, Event* e) {
    ++waits;
    return hip_status(hipStreamWaitEvent(s, e->ev, 0), "hipStreamWaitEvent");
  }

  // `dst` waits for all work queued so far on `src`. An idle `src` needs no
  // wait: between engine steps the caller's stream has usually drained (the
  // step's sampled tokens were read back), and skipping the marker event and
  // cross-stream wait there raised 128 queued one-block FP8 restores from
  // 46.5-48.1 to 52.8 GB/s and one-block saves beside restores from 85-86 to
  // 87-94 GB/s on MI355X.
  // *needed (optional) tells whether a wait was queued.
  int wait_stream(hipStream_t dst, hipStream_t src, bool* needed = nullptr) {
    const bool wait = dst != src && hipStreamQuery(src) != hipSuccess;
    if (needed) *needed = wait;
    if (!wait) return KVX_OK;
    int rc = hip_status(hipEventRecord(marker, src), "hipEventRecord");
    if (rc) return rc;
    ++waits;
    return hip_status(hipStreamWaitEvent(dst, marker, 0), "hipStreamWaitEvent");
  }

  // `save`: the slots are destinations and must be distinct; otherwise the blocks are.
  // `staged`: the call uses the attached staging.
  int check_lists(bool save, const int32_t* ids, const int32_t* slots, int32_t n, bool staged = true) const {
    if (n < 0) return set_error(KVX_E_INVALID, "negative block count");
    if (n > 0 && (!ids || !slots)) return set_error(KVX_E_INVALID, "NULL block id or slot array");
    for (int32_t i = 0; i < n; ++i) {
      if (ids[i] < 0 || ids[i] >= layout.num_blocks)
        return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", ids[i], layout.num_blocks);
      if (slots[i] < 0 || slots[i] >= num_slots)
        return set_error(KVX_E_RANGE, "host slot %d outside [0, %d)", slots[i], num_slots);
    }
    if (any_repeat(save ? slots : ids, n))
      return set_error(KVX_E_INVALID, save ? "a slot appears twice in one save" : "a block appears twice in one restore");
    if (n > 0 && staged && !save_staging) return set_error(KVX_E_STATE, "no staging attached");
    return KVX_OK;
  }

  // Saves of one or two blocks issued while the caller's stream still has
  // work queued have the save kernel write the pinned slots itself; other
  // saves gather into staging and copy to the host. Measured on MI355X with
  // Qwen3-8B FP8 blocks and a restore stream running beside the save stream
  // (save alone / both directions, GB/s):
  //  - staged, 1-2 blocks per call behind a busy caller stream: the D2H copy
  //    of the entries, queued behind the save kernel whose stream waited for
  //    the caller's, started ~0.65 ms late: 29.6 / 32 (one block), 53 / 42.5
  //    (two blocks). Three or more blocks never showed it: 53.8-54.9 /
  //    92.7-94.5. With the caller's stream idle (no wait) one-block saves run
  //    at 51.5 / 90-92;
  //  - written by the kernel (direct_save_grid workgroups, system-scope
  //    stores): 48.7-49.3 / 93-93.5 for one block, 49.5 / 93.5-93.8 for two.
  // Kernel-written saves hold CUs for the whole transfer: 64 one-block FP8
  // saves queued before 200 bf16 4096^2 matmuls left the matmuls 29.5 ms
  // against 23.8 ms beside staged saves (19.8 ms alone), so they are used
  // only where the staged copy would start late.
  static bool direct_save(int32_t n, bool caller_busy) { return n <= 2 && caller_busy; }

  // Workgroups of a save that writes host slots directly. The launch lasts as
  // long as its writes take to cross the host link (~0.4 ms per Qwen3-8B FP8
  // block). Too many workgroups hold CUs the restore stream's kernels need
  // and crowd the link's upstream direction, which also carries the restore
  // DMA's read requests; too few cannot keep the link busy. Measured for
  // one-block saves beside one-block restores (save alone / both, GB/s):
  //   FP8 (2 KiB tiles): 16 -> 25 / 49, 24 -> 37 / 72, 32 -> 48.6 / 92.8,
  //                      48 -> 53.8 / 86, 64 -> 52.9 / 76, 128 -> 53.4 / 77;
  //   BF16 (16 KiB tiles): 16 -> 55.4 / 90.3, 24 -> 55.9 / 87.8,
  //                        32 -> 54.5 / 85, 64 -> 56 / 82.4.
  int32_t direct_save_grid() const { return format == KVX_FORMAT_FP8 ? 32 : 16; }

  // Restores of one or two blocks whose caller waits for them (wait != 0),
  // issued while no save is in flight, have the restore kernel read the host
  // slots itself: a capped grid strides over the tiles with system-scope
  // loads, queued on the caller's stream (kvx_cache_restore). Everything else
  // goes through device staging and an H2D copy on the restore stream.
  // Measured on MI355X with one engine call per block (the reference
  // BlockManager's pattern): waited restores 47.8 -> 48.3 GB/s (FP8) and
  // 51.1 -> 54.1 (BF16); the agent-pressure workload 3.34 -> 3.09 s. Not for
  // prefetches (wait == 0), which overlap compute: a kernel-read restore
  // holds its workgroups for the whole transfer, as kernel-written saves do.
  // Not beside a running save either: kernel reads and kernel writes of host
  // memory together ran at ~63 GB/s both ways, against ~93 for staged
  // restores beside kernel-written saves.
  bool direct_restore(int32_t n, bool wait) const {
    if (n > 2 || !wait || !host_reads_ok) return false;
    return !last_save || hipEventQuery(last_save->ev) == hipSuccess;
  }
  int32_t direct_restore_grid() const { return format == KVX_FORMAT_FP8 ? 64 : 32; }

  // Copies `count` entries between consecutive staging entries and host
  // slots. Runs of consecutive slots in one slab are merged, then cut into
  // pieces of at most kDmaPiece bytes: two multi-gigabyte copies queued at the
  // same moment on the save and restore streams were measured to serialize
  // (57 GB/s in total), while the same bytes in pieces ran full duplex
  // (~95 GB/s over PCIe 5.0 for 32-128 MiB pieces; 8 MiB pieces lose 3-4%,
  // and 16 MiB was best on one host but 1% behind on another).
  static constexpr size_t kDmaPiece = 64u << 20;
  int dma(bool to_host, uint8_t* staging, const int32_t* slots, int32_t count, hipStream_t s) {
    int32_t i = 0;
    while (i < count) {
      int32_t j = i + 1;
      uint8_t* h0 = host_entry(slots[i]);
      while (j < count && slots[j] == slots[j - 1] + 1 && host_entry(slots[j]) == h0 + (int64_t)(j - i) * entry_stride)
        ++j;
      const size_t bytes = (size_t)(j - i - 1) * entry_stride + (size_t)logical_bytes_with_scales();
      uint8_t* d = staging + (int64_t)i * entry_stride;
      for (size_t off = 0; off < bytes; off += kDmaPiece) {
        const size_t n = std::min(kDmaPiece, bytes - off);
        hipError_t err = to_host ? hipMemcpyAsync(h0 + off, d + off, n, hipMemcpyDeviceToHost, s)
                                 : hipMemcpyAsync(d + off, h0 + off, n, hipMemcpyHostToDevice, s);
        if (err != hipSuccess) return hip_status(err, to_host ? "D2H hipMemcpyAsync" : "H2D hipMemcpyAsync");
        ++(to_host ? d2h_copies : h2d_copies);
        (to_host ? d2h_bytes : h2d_bytes) += (int64_t)n;
      }
      i = j;
    }
    return KVX_OK;
  }

  // Bytes of one entry that carry data (payload, and scales at scale_offset).
  int64_t logical_bytes_with_scales() const {
    if (format == KVX_FORMAT_RAW) return logical_bytes;
    const int64_t rows = (int64_t)layout.planes * layout.plane_rows;
    return scale_offset + rows * (layout.scale_dtype == KVX_SCALE_BF16 ? 2 : 4);
  }

  // Launches the save or restore kernel for `count` (<= kMaxBatch) blocks whose
  // entries start at staging (consecutive entries) or, with staging == nullptr,
  // at the host slots `slots` (the kernel then moves the bytes over the host link).
  int launch(bool save, const int32_t* ids, uint8_t* staging, const int32_t* slots, int32_t count,
             hipStream_t s) {
    BlockBatch b;
    b.n = count;
    for (int32_t i = 0; i < count; ++i) {
      b.ids[i] = ids[i];
      b.entries[i] = (uint64_t)(uintptr_t)(staging ? staging + (int64_t)i * entry_stride : host_entry(slots[i]));
    }
    const bool vec = vector_access_ok(pool, layout, b.entries, b.n);
    hipError_t err = save ? launch_save(pool, layout, format, b, scale_offset, vec, staging ? 0 : direct_save_grid(), s)
                          : launch_restore(pool, layout, format, b, scale_offset, vec,
                                           staging ? 0 : direct_restore_grid(), s);
    return hip_status(err, save ? "save kernel launch" : "restore kernel launch");
  }

  int chunk() const { return std::min(staging_entries, kMaxBatch); }

  // Entries the static staging holds (at most kMaxBatch: one launch).
  int32_t static_entries() const {
    return (int32_t)std::min<int64_t>(kMaxBatch, (int64_t)KVX_NOALLOC_SCRATCH_BYTES / entry_stride);
  }
};

// The body of kvx_cache_save and kvx_cache_save_noalloc. `staging` holds
// `staging_entries` entries; `fixed_done` (if set) is recorded instead of a
// pooled event. Allocates nothing when fixed_done is set.
static int save_blocks_to_slots(kvx_cache* c, const int32_t* ids, const int32_t* slots, int32_t n,
                                hipStream_t compute, uint8_t* staging, int32_t staging_entries,
                                Event* fixed_done) {
  DeviceScope scope;
  int rc = scope.enter(c->device);
  if (rc) return rc;
  hipStream_t s = c->save_stream;
  // Start after the kernels that wrote these blocks (cpu_prefix_cache.py:310-311).
  bool caller_busy = false;
  rc = c->wait_stream(s, compute, &caller_busy);
  if (rc) return rc;
  // After the last restore that read each target slot (:312-314). With one
  // copy stream only a kernel-read restore, queued on a caller's stream, is
  // not already ahead of the save; the wait for `compute` covers it only if
  // it was queued there.
  if (!(c->debug & KVX_DEBUG_SKIP_SLOT_READ_WAIT)) {
    for (int32_t i = 0; i < n; ++i) {
      Event*& r = c->slot_read[slots[i]];
      if (r) {
        rc = c->wait_event(s, r);
        if (rc) return rc;
        c->unref(r);
      }
    }
  }
  // After a background restore still writing a source block (a prefetched
  // block whose CPU entry was dropped can be saved again before first use).
  {
    for (int32_t i = 0; i < n; ++i) {
      if (Event* pr = c->pending_restore[ids[i]]) {
        rc = c->wait_event(s, pr);
        if (rc) return rc;
      }
    }
  }
  // A staged save reads its pool blocks in the kernel; the copies to the
  // host read only the staging. Each chunk's blocks are therefore released
  // (pending_save) by an event right after its kernel, so a restore into a
  // recycled victim, or the caller's writes into it, wait for the kernel and
  // not for the transfer: the restore's host-to-device copies then overlap
  // the save's device-to-host ones. The host slots are released (slot_saved)
  // after the copies. A kernel-written save, and one with a fixed event (the
  // allocation-free save, which creates none), release both after the copies.
  const bool direct = kvx_cache::direct_save(n, caller_busy);
  if (direct) {
    rc = c->launch(true, ids, nullptr, slots, n, s);
    if (rc) return rc;
  } else {
    const int32_t step = std::min(staging_entries, kMaxBatch);
    for (int32_t base = 0; base < n; base += step) {
      const int32_t cnt = std::min(step, n - base);
      rc = c->launch(true, ids + base, staging, nullptr, cnt, s);
      if (!rc && !fixed_done) rc = c->release_blocks_after(ids + base, cnt, s);
      if (!rc) rc = c->dma(true, staging, slots + base, cnt, s);
      if (rc) return rc;
    }
  }
  Event* done = fixed_done;
  if (!done) rc = c->new_event(&done);
  if (!rc) rc = c->record(done, s);
  if (rc) {
    if (done && !fixed_done) c->release_if_unused(done);
    return rc;
  }
  for (int32_t i = 0; i < n; ++i) {
    if (direct || fixed_done) c->assign(c->pending_save[ids[i]], done);
    c->assign(c->slot_saved[slots[i]], done);
  }
  c->assign(c->last_save, done);
  c->saved += n;
  return KVX_OK;
}

extern "C" {

const char* kvx_last_error(void) { return g_error; }

int kvx_abi_version(void) { return KVX_ABI_VERSION; }

int kvx_entry_layout(const kvx_block_layout* layout, int32_t format, int64_t* logical_bytes,
                     int64_t* scale_offset, int64_t* entry_stride) {
  int rc = check_layout(layout, format);
  if (rc) return rc;
  int64_t a, b, c;
  entry_sizes(*layout, format, &a, &b, &c);
  if (logical_bytes) *logical_bytes = a;
  if (scale_offset) *scale_offset = b;
  if (entry_stride) *entry_stride = c;
  return KVX_OK;
}

int kvx_store_kvcache(const void* key, int64_t key_stride, const void* value, int64_t value_stride, void* k_cache,
                      void* v_cache, const int32_t* slot_mapping, int64_t num_tokens, int32_t num_heads,
                      int32_t head_dim, int32_t elem_bytes, int64_t cache_slots, void* stream) {
  if (num_tokens < 0) return set_error(KVX_E_INVALID, "negative token count");
  if (num_heads <= 0 || head_dim <= 0) return set_error(KVX_E_INVALID, "num_heads and head_dim must be positive");
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return set_error(KVX_E_INVALID, "elem_bytes must be 1, 2, 4 or 8");
  if (key_stride < 0 || value_stride < 0 || cache_slots < 0)
    return set_error(KVX_E_INVALID, "strides and cache_slots must be non-negative");
  if (num_tokens == 0 || cache_slots == 0) return KVX_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return set_error(KVX_E_INVALID, "NULL tensor pointer");
  if (num_tokens > (int64_t)INT32_MAX) return set_error(KVX_E_UNSUPPORTED, "too many tokens for one launch");
  const int64_t row = (int64_t)num_heads * head_dim;
  int64_t cache_bytes;
  if (strided_span(num_tokens, key_stride, row, elem_bytes) < 0 ||
      strided_span(num_tokens, value_stride, row, elem_bytes) < 0 ||
      !span_product({cache_slots, row, elem_bytes}, &cache_bytes))
    return set_error(KVX_E_UNSUPPORTED, "key, value or cache spans more than 2^40 bytes");
  hipError_t err = launch_store_kvcache(key, key_stride, value, value_stride, k_cache, v_cache, slot_mapping,
                                        num_tokens, row, elem_bytes, cache_slots, (hipStream_t)stream);
  return hip_status(err, "store_kvcache launch");
}

int kvx_save_blocks(const void* pool, const kvx_block_layout* layout, int32_t format, const int32_t* block_ids_host,
                    const uint64_t* entries_host, int32_t n, int64_t scale_offset, void* stream) {
  return run_batches(true, const_cast<void*>(pool), layout, format, block_ids_host, entries_host, n, scale_offset,
                     (hipStream_t)stream);
}

int kvx_restore_blocks(void* pool, const kvx_block_layout* layout, int32_t format, const int32_t* block_ids_host,
                       const uint64_t* entries_host, int32_t n, int64_t scale_offset, void* stream) {
  return run_batches(false, pool, layout, format, block_ids_host, entries_host, n, scale_offset,
                     (hipStream_t)stream);
}

int kvx_gather_tokens(const void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                      int32_t table_len, int64_t num_rows, void* dst, void* stream) {
  return token_copy(true, const_cast<void*>(pool), layout, block_table_host, table_len, num_rows, dst,
                    (hipStream_t)stream);
}

int kvx_scatter_tokens(void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                       int32_t table_len, int64_t num_rows, const void* src, void* stream) {
  return token_copy(false, pool, layout, block_table_host, table_len, num_rows, const_cast<void*>(src),
                    (hipStream_t)stream);
}

int kvx_gather_tokens_fp8(const void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                          int32_t table_len, int64_t num_rows, void* payload, void* scales, void* stream) {
  return token_fp8(true, const_cast<void*>(pool), layout, block_table_host, table_len, num_rows, payload, scales,
                   (hipStream_t)stream);
}

int kvx_scatter_tokens_fp8(void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                           int32_t table_len, int64_t num_rows, const void* payload, const void* scales,
                           void* stream) {
  return token_fp8(false, pool, layout, block_table_host, table_len, num_rows, const_cast<void*>(payload),
                   const_cast<void*>(scales), (hipStream_t)stream);
}

int kvx_upload(void* dst, const void* src_pinned, int64_t nbytes, void* stream) {
  if (nbytes < 0) return set_error(KVX_E_INVALID, "negative byte count");
  if (nbytes > KVX_UPLOAD_MAX_BYTES)
    return set_error(KVX_E_RANGE, "%lld bytes exceed the largest upload (%lld)", (long long)nbytes,
                     (long long)KVX_UPLOAD_MAX_BYTES);
  if (nbytes == 0) return KVX_OK;
  if (!dst || !src_pinned) return set_error(KVX_E_INVALID, "NULL destination or source");
  // The kernel reads the source through the device's mapping of it. Two
  // independent checks that every byte read lies in one pinned allocation:
  // the first and last bytes are both pinned host memory, mapped nbytes - 1
  // apart, and the allocation holding the first byte extends past the last.
  hipPointerAttribute_t head, tail;
  const uint8_t* last = (const uint8_t*)src_pinned + (nbytes - 1);
  if (hipPointerGetAttributes(&head, src_pinned) != hipSuccess || hipPointerGetAttributes(&tail, last) != hipSuccess ||
      head.type != hipMemoryTypeHost || tail.type != hipMemoryTypeHost || !head.devicePointer ||
      (uintptr_t)tail.devicePointer - (uintptr_t)head.devicePointer != (uintptr_t)(nbytes - 1)) {
    (void)hipGetLastError();
    return set_error(KVX_E_INVALID, "the upload source is not %lld bytes of pinned, device-accessible host memory",
                     (long long)nbytes);
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, head.devicePointer) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(KVX_E_INVALID, "the upload source's allocation could not be looked up");
  }
  const uintptr_t start = (uintptr_t)head.devicePointer, first = (uintptr_t)base;
  if (start < first || start - first + (uint64_t)nbytes > (uint64_t)size)
    return set_error(KVX_E_INVALID, "the upload source runs past its pinned allocation (%lld of %llu bytes left)",
                     (long long)(first + size - start), (unsigned long long)size);
  return hip_status(launch_upload(dst, head.devicePointer, nbytes, (hipStream_t)stream), "upload kernel launch");
}

int kvx_sleep(void* stream, int64_t microseconds) {
  if (microseconds < 0 || microseconds > 60LL * 1000 * 1000)
    return set_error(KVX_E_RANGE, "sleep must be within [0, 60 s]");
  return hip_status(launch_sleep((hipStream_t)stream, microseconds), "sleep kernel launch");
}

int kvx_selftest(uint64_t* counters, void* stream) {
  if (!counters) return set_error(KVX_E_INVALID, "NULL counter array");
  return hip_status(launch_selftest(counters, (hipStream_t)stream), "selftest launch");
}

int kvx_cache_create(void* pool, const kvx_block_layout* layout, int32_t format, void* save_stream,
                     void* restore_stream, int32_t device, kvx_cache** out) {
  if (!out) return set_error(KVX_E_INVALID, "NULL output handle");
  *out = nullptr;
  int rc = check_layout(layout, format);
  if (rc) return rc;
  if (!pool || (uintptr_t)pool % 16) return set_error(KVX_E_INVALID, "pool must be a 16-byte aligned pointer");
  if (!save_stream || !restore_stream)
    return set_error(KVX_E_INVALID, "the copy engine needs two non-null streams (pass one twice to share it)");
  kvx_cache* c = new (std::nothrow) kvx_cache();
  if (!c) return set_error(KVX_E_STATE, "out of host memory");
  c->device = device;
  c->pool = (uint8_t*)pool;
  c->layout = *layout;
  c->format = format;
  entry_sizes(*layout, format, &c->logical_bytes, &c->scale_offset, &c->entry_stride);
  c->save_stream = (hipStream_t)save_stream;
  c->restore_stream = (hipStream_t)restore_stream;
  c->split = save_stream != restore_stream;
  // Host slots are 256-byte aligned and entry_stride apart (a multiple of 256),
  // so the pool alone decides whether the vector kernels can address them.
  c->host_reads_ok = striding_restore_supported(*layout, format, vector_access_ok(pool, *layout, nullptr, 0));
  c->pending_save.assign(layout->num_blocks, nullptr);
  c->pending_restore.assign(layout->num_blocks, nullptr);
  DeviceScope scope;
  rc = scope.enter(device);
  // The marker only orders device work behind device work: saves behind the
  // caller's writes of their pool blocks, restores behind the caller's reads
  // of their destinations, and each copy stream behind the other's use of a
  // re-cut staging area. Hand-offs through host slots wait on the pooled
  // events, which keep the system-scope release. A device-scope release cut
  // the host cost of the wait behind a busy stream from 12.6 to 6.6 us on
  // MI355X.
  if (!rc)
    rc = hip_status(hipEventCreateWithFlags(&c->marker, hipEventDisableTiming | hipEventReleaseToDevice),
                    "hipEventCreate");
  if (!rc) rc = c->new_event(&c->static_done);
  if (rc) {
    kvx_cache_destroy(c);
    return rc;
  }
  c->static_done->refs = 1;  // held by the cache: never returns to the event pool
  // Set-up for kvx_cache_save_noalloc, with the device current. A failed
  // lookup fails only that entry point, which reports it.
  scratch_setup(device, &c->static_staging, &c->static_staging_status);
  *out = c;
  return KVX_OK;
}

int kvx_cache_destroy(kvx_cache* c) {
  if (!c) return KVX_OK;
  int rc = KVX_OK;
  DeviceScope scope;
  (void)scope.enter(c->device);
  if (c->save_stream) rc = hip_status(hipStreamSynchronize(c->save_stream), "hipStreamSynchronize");
  if (c->split && c->restore_stream) {
    int rc2 = hip_status(hipStreamSynchronize(c->restore_stream), "hipStreamSynchronize");
    if (!rc) rc = rc2;
  }
  const int rc3 = c->sync_caller_reads();
  if (!rc) rc = rc3;
  for (Event* e : c->all_events) {
    (void)hipEventDestroy(e->ev);
    delete e;
  }
  if (c->marker) (void)hipEventDestroy(c->marker);
  delete c;  // the streams belong to the caller
  return rc;
}

int kvx_cache_set_staging(kvx_cache* c, void* save_staging, void* restore_staging, int32_t entries) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (entries <= 0 || !save_staging || !restore_staging)
    return set_error(KVX_E_INVALID, "staging needs two buffers and a positive entry count");
  if ((uintptr_t)save_staging % 256 || (uintptr_t)restore_staging % 256)
    return set_error(KVX_E_INVALID, "staging buffers must be 256-byte aligned");
  if (!c->split && save_staging != restore_staging)
    return set_error(KVX_E_INVALID, "one stream shares one staging buffer");
  int64_t staging_bytes;
  if (!span_product({entries, c->entry_stride}, &staging_bytes))
    return set_error(KVX_E_UNSUPPORTED, "staging of %d entries spans more than 2^40 bytes", entries);
  // With split streams a save's chunks and a restore's chunks use their
  // buffers at the same time.
  const uintptr_t save_at = (uintptr_t)save_staging, restore_at = (uintptr_t)restore_staging;
  if (c->split && save_at < restore_at + (uintptr_t)staging_bytes && restore_at < save_at + (uintptr_t)staging_bytes)
    return set_error(KVX_E_INVALID, "split streams need save and restore staging buffers that do not overlap");
  // Copies queued on one stream may still use an area that becomes the other
  // stream's: each stream's later copies wait for the other's queued work.
  if (c->split && c->save_staging &&
      ((uint8_t*)save_staging != c->save_staging || (uint8_t*)restore_staging != c->restore_staging)) {
    DeviceScope scope;
    int rc = scope.enter(c->device);
    if (!rc) rc = c->wait_stream(c->restore_stream, c->save_stream);
    if (!rc) rc = c->wait_stream(c->save_stream, c->restore_stream);
    if (rc) return rc;
  }
  c->save_staging = (uint8_t*)save_staging;
  c->restore_staging = (uint8_t*)restore_staging;
  c->staging_entries = entries;
  return KVX_OK;
}

int kvx_cache_add_slab(kvx_cache* c, void* host_base, int32_t count) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (!host_base || count <= 0) return set_error(KVX_E_INVALID, "slab needs memory and a positive slot count");
  if ((uintptr_t)host_base % 256) return set_error(KVX_E_INVALID, "slab must be 256-byte aligned");
  if ((int64_t)c->num_slots + count > (int64_t)INT32_MAX) return set_error(KVX_E_RANGE, "too many slots");
  int64_t slab_bytes;
  if (!span_product({count, c->entry_stride}, &slab_bytes))
    return set_error(KVX_E_UNSUPPORTED, "a slab of %d entries spans more than 2^40 bytes", count);
  c->slabs.push_back(Slab{(uint8_t*)host_base, c->num_slots, count});
  c->num_slots += count;
  c->slot_read.resize(c->num_slots, nullptr);
  c->slot_saved.resize(c->num_slots, nullptr);
  return KVX_OK;
}

int kvx_cache_reset_slabs(kvx_cache* c) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  int rc = kvx_cache_synchronize(c);
  if (rc) return rc;
  for (Event*& e : c->slot_read) c->unref(e);
  for (Event*& e : c->slot_saved) c->unref(e);
  c->slot_read.clear();
  c->slot_saved.clear();
  c->slabs.clear();
  c->num_slots = 0;
  return KVX_OK;
}

int kvx_cache_streams(kvx_cache* c, void** save_stream, void** restore_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (save_stream) *save_stream = (void*)c->save_stream;
  if (restore_stream) *restore_stream = (void*)c->restore_stream;
  return KVX_OK;
}

int kvx_cache_save(kvx_cache* c, const int32_t* ids, const int32_t* slots, int32_t n, void* compute_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  int rc = c->check_lists(true, ids, slots, n);
  if (rc || n == 0) return rc;
  return save_blocks_to_slots(c, ids, slots, n, (hipStream_t)compute_stream, c->save_staging, c->staging_entries,
                              nullptr);
}

int kvx_cache_save_noalloc(kvx_cache* c, const int32_t* ids, const int32_t* slots, int32_t n,
                           void* compute_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  int rc = c->check_lists(true, ids, slots, n, false);
  if (rc || n == 0) return rc;
  if (c->static_staging_status != KVX_OK || !c->static_staging || !c->static_done)
    return set_error(c->static_staging_status != KVX_OK ? c->static_staging_status : KVX_E_STATE,
                     "no static staging on device %d", c->device);
  const int32_t max_n = c->static_entries();
  if (n > max_n)
    return set_error(KVX_E_RANGE, "%d blocks exceed the static staging: at most %d entries of %lld bytes fit in %lld "
                     "bytes", n, max_n, (long long)c->entry_stride, (long long)KVX_NOALLOC_SCRATCH_BYTES);
  // The array is the device's, not the cache's: wait for the previous call's
  // copies out of it unless stream order already gives that.
  std::lock_guard<std::mutex> lock(g_scratch.use_mu[c->device]);
  hipEvent_t last_use = g_scratch.last_use[c->device];
  hipStream_t& last_stream = g_scratch.last_stream[c->device];
  DeviceScope scope;
  rc = scope.enter(c->device);
  if (rc) return rc;
  if (last_stream && last_stream != c->save_stream) {
    rc = hip_status(hipStreamWaitEvent(c->save_stream, last_use, 0), "hipStreamWaitEvent");
    if (rc) return rc;
    ++c->waits;
  }
  rc = save_blocks_to_slots(c, ids, slots, n, (hipStream_t)compute_stream, c->static_staging, max_n,
                            c->static_done);
  // Recorded even after a failure: work already queued may still use the array.
  const int rc2 = hip_status(hipEventRecord(last_use, c->save_stream), "hipEventRecord");
  if (rc2 == KVX_OK) last_stream = c->save_stream;
  return rc ? rc : rc2;
}

int kvx_cache_restore(kvx_cache* c, const int32_t* slots, const int32_t* ids, int32_t n, int32_t wait,
                      void* compute_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  int rc = c->check_lists(false, ids, slots, n);
  if (rc || n == 0) return rc;
  DeviceScope scope;
  rc = scope.enter(c->device);
  if (rc) return rc;
  hipStream_t compute = (hipStream_t)compute_stream;
  // A restore the caller waits for at once, read by the kernel straight from
  // the host slots, runs on the caller's stream: there it follows the
  // caller's queued work and precedes the caller's later work with no
  // cross-stream wait. The two waits and the query of the busy caller stream
  // a one-block call made on the restore stream cost 60-80 us of host time
  // per call on MI355X, against ~5 us for the launch.
  const bool direct = c->direct_restore(n, wait != 0);
  hipStream_t s = direct ? compute : c->restore_stream;
  // What the work of blocks [base, base + cnt) waits for on `s`. With the
  // restore on the save stream (one copy stream), stream order covers saves.
  const bool order_saves = c->split || s != c->save_stream;
  // Before a copy reads the slots: their payload may still be arriving from
  // its save (:380-381).
  auto wait_slots = [&](int32_t base, int32_t cnt) -> int {
    if (!order_saves || (c->debug & KVX_DEBUG_SKIP_SAVE_WAIT)) return KVX_OK;
    for (int32_t i = base; i < base + cnt; ++i)
      if (Event* sv = c->slot_saved[slots[i]]) {
        const int r = c->wait_event(s, sv);
        if (r) return r;
      }
    return KVX_OK;
  };
  // Before a kernel writes the destinations: a save of a recycled victim may
  // still be reading one (the save releases its blocks once its kernel has
  // read them, so this does not wait for the save's transfer).
  auto wait_victims = [&](int32_t base, int32_t cnt) -> int {
    if (!order_saves || (c->debug & KVX_DEBUG_SKIP_VICTIM_WAIT)) return KVX_OK;
    for (int32_t i = base; i < base + cnt; ++i) {
      Event* ps = c->pending_save[ids[i]];
      if (ps && ps != c->slot_saved[slots[i]]) {
        const int r = c->wait_event(s, ps);
        if (r) return r;
      }
    }
    return KVX_OK;
  };
  // A restore on the caller's stream is not behind the restore stream's
  // queue: it also waits for a background restore (a prefetch) still writing
  // one of its blocks, as when a prefetched block is recycled before its
  // first use without before_block_reuse (block_manager.py:168).
  auto wait_overwrites = [&]() -> int {
    if (s == c->restore_stream || (c->debug & KVX_DEBUG_SKIP_OVERWRITE_WAIT)) return KVX_OK;
    for (int32_t i = 0; i < n; ++i)
      if (Event* pr = c->pending_restore[ids[i]]) {
        const int r = c->wait_event(s, pr);
        if (r) return r;
      }
    return KVX_OK;
  };
  // Before the first kernel: the destinations may still be read by kernels
  // queued on the caller's stream (:375-379). The copies into staging before
  // it touch no destination, so they start without these waits, beside the
  // transfers of saves still in flight.
  if (direct) {
    rc = c->wait_stream(s, compute);
    if (!rc) rc = wait_slots(0, n);
    if (!rc) rc = wait_victims(0, n);
    if (!rc) rc = wait_overwrites();
    if (!rc) rc = c->launch(false, ids, nullptr, slots, n, s);
    if (rc) return rc;
  } else {
    const int32_t step = c->chunk();
    for (int32_t base = 0; base < n; base += step) {
      const int32_t cnt = std::min(step, n - base);
      rc = wait_slots(base, cnt);
      if (!rc) rc = c->dma(false, c->restore_staging, slots + base, cnt, s);
      if (!rc && base == 0) rc = c->wait_stream(s, compute);
      if (!rc) rc = wait_victims(base, cnt);
      if (!rc) rc = c->launch(false, ids + base, c->restore_staging, nullptr, cnt, s);
      if (rc) {
        // Earlier chunks are queued with no event the caller could order on,
        // and the caller frees these blocks on an error: let them land first.
        if (base > 0) (void)hipStreamSynchronize(s);
        return rc;
      }
    }
  }
  Event* done = nullptr;
  rc = c->new_event(&done);
  if (!rc) rc = c->record(done, s);
  if (!rc && s == compute) c->track_caller_read(s, done);
  if (!rc && wait && s != compute) rc = c->queue_wait(compute, done);
  if (rc) {
    if (done) c->release_if_unused(done);
    (void)hipStreamSynchronize(s);  // the restore is queued; the caller frees its blocks on an error
    return rc;
  }
  for (int32_t i = 0; i < n; ++i) {
    c->assign(c->slot_read[slots[i]], done);
    if (!wait) c->assign(c->pending_restore[ids[i]], done);
  }
  c->release_if_unused(done);
  c->restored += n;
  return KVX_OK;
}

int kvx_cache_before_block_reuse(kvx_cache* c, int32_t block_id, void* compute_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (block_id < 0 || block_id >= c->layout.num_blocks)
    return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", block_id, c->layout.num_blocks);
  for (std::vector<Event*>* pending : {&c->pending_save, &c->pending_restore}) {
    Event*& e = (*pending)[block_id];
    if (e && pending == &c->pending_save && (c->debug & KVX_DEBUG_SKIP_REUSE_WAIT)) {
      c->unref(e);
      continue;
    }
    if (e) {
      int rc = c->wait_event((hipStream_t)compute_stream, e);
      if (rc) return rc;
      c->unref(e);
    }
  }
  return KVX_OK;
}

int kvx_cache_before_block_use(kvx_cache* c, int32_t block_id, void* compute_stream) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (block_id < 0 || block_id >= c->layout.num_blocks)
    return set_error(KVX_E_RANGE, "block id %d outside [0, %d)", block_id, c->layout.num_blocks);
  Event*& e = c->pending_restore[block_id];
  if (e) {
    int rc = c->wait_event((hipStream_t)compute_stream, e);
    if (rc) return rc;
    c->unref(e);
  }
  return KVX_OK;
}

int kvx_cache_set_debug(kvx_cache* c, int32_t flags) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (flags & ~(KVX_DEBUG_SKIP_SAVE_WAIT | KVX_DEBUG_SKIP_SLOT_READ_WAIT | KVX_DEBUG_SKIP_REUSE_WAIT |
                KVX_DEBUG_SKIP_VICTIM_WAIT | KVX_DEBUG_SKIP_OVERWRITE_WAIT))
    return set_error(KVX_E_INVALID, "unknown debug flags %d", flags);
  c->debug = flags;
  return KVX_OK;
}

int kvx_cache_synchronize(kvx_cache* c) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  DeviceScope scope;
  int rc = scope.enter(c->device);
  if (!rc) rc = hip_status(hipStreamSynchronize(c->save_stream), "hipStreamSynchronize");
  if (!rc && c->split) rc = hip_status(hipStreamSynchronize(c->restore_stream), "hipStreamSynchronize");
  if (!rc) rc = c->sync_caller_reads();
  return rc;
}

int kvx_cache_counters(kvx_cache* c, int64_t* saved_blocks, int64_t* restored_blocks, int64_t* stream_waits) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (saved_blocks) *saved_blocks = c->saved;
  if (restored_blocks) *restored_blocks = c->restored;
  if (stream_waits) *stream_waits = c->waits;
  return KVX_OK;
}

int kvx_cache_dma_counters(kvx_cache* c, int64_t* d2h_copies, int64_t* d2h_bytes, int64_t* h2d_copies,
                           int64_t* h2d_bytes) {
  if (!c) return set_error(KVX_E_INVALID, "NULL cache");
  if (d2h_copies) *d2h_copies = c->d2h_copies;
  if (d2h_bytes) *d2h_bytes = c->d2h_bytes;
  if (h2d_copies) *h2d_copies = c->h2d_copies;
  if (h2d_bytes) *h2d_bytes = c->h2d_bytes;
  return KVX_OK;
}

}  // extern "C"
