// Internal declarations shared by the kernel launchers and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvx.h"

namespace kvx {

// Blocks handled by one save/restore launch. The list travels in the kernel
// argument segment (ids + entry addresses: 12 bytes per block), so a launch
// needs no device-side index buffer and stays capturable in a HIP graph.
constexpr int kMaxBatch = 128;

struct BlockBatch {
  int32_t n;
  int32_t ids[kMaxBatch];
  uint64_t entries[kMaxBatch];
};

// Launch-time geometry derived from kvx_block_layout. For FP8 entries, the
// payload of (entry e, plane p, row r) is at
//   entries[e] + p * payload_plane_stride + r * head_dim
// and its scale at
//   entries[e] + scale_offset + e * scale_entry_step + p * scale_plane_stride + r * scale_bytes.
// Block entries are dense per block (payload_plane_stride = plane_rows *
// head_dim, scale_plane_stride = plane_rows * scale_bytes, no entry step);
// token entries (KV handoff) are one block's rows of a [planes][rows][hd]
// payload and a [planes][rows] scale array. The batch's last entry has
// last_rows valid rows per plane (a sequence's partial final block), the
// others plane_rows.
struct PlaneGeom {
  int64_t plane_stride;  // elements
  int64_t block_stride;  // elements
  int64_t scale_offset;  // bytes from an entry's payload to its scales
  int64_t payload_plane_stride;  // bytes (FP8)
  int64_t scale_plane_stride;    // bytes (FP8)
  int64_t scale_entry_step;      // bytes (FP8)
  int32_t planes;
  int32_t plane_rows;
  int32_t last_rows;
  int32_t head_dim;
  int32_t chunks;        // tiles per plane
};

// FP8 token entries of one launch (see PlaneGeom).
struct TokenSpan {
  int64_t payload_plane_stride;
  int64_t scale_plane_stride;
  int64_t scale_entry_step;
  int32_t last_rows;
};

// Records a message for kvx_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
// Converts a HIP status into the ABI convention, recording a message.
int hip_status(hipError_t err, const char* what);

int check_layout(const kvx_block_layout* layout, int32_t format);

// Kernel launchers: arguments are validated by the caller.
// `vector_ok`: the pool base, both strides and every entry allow 16-byte
// vector access; otherwise the element-granular kernels run.
// `max_grid` > 0 caps a vector kernel's workgroups (they then stride over
// the tiles): for saves written to and restores read from host memory, which
// hold their workgroups while the bytes cross the host link.
hipError_t launch_save(const void* pool, const kvx_block_layout& layout, int32_t format,
                       const BlockBatch& batch, int64_t scale_offset, bool vector_ok, int32_t max_grid,
                       hipStream_t stream);
hipError_t launch_restore(void* pool, const kvx_block_layout& layout, int32_t format,
                          const BlockBatch& batch, int64_t scale_offset, bool vector_ok, int32_t max_grid,
                          hipStream_t stream);
// True when a restore launched with max_grid > 0 runs the striding kernel,
// whose reads of host entries are system-scope loads (the element-granular
// kernels read with plain loads and must not read host memory).
bool striding_restore_supported(const kvx_block_layout& layout, int32_t format, bool vector_ok);
// Token gather/scatter between a sequence's blocks and a dense
// [planes][rows][head_dim] buffer: entries are the dense buffer at
// block_index * plane_bytes, dense_plane_stride apart per plane, and the
// batch's last block copies last_bytes per plane.
hipError_t launch_token_copy(bool gather, void* pool, const kvx_block_layout& layout, const BlockBatch& batch,
                             bool vector_ok, int64_t dense_plane_stride, int64_t last_bytes, hipStream_t stream);
// The same with FP8 quantisation (gather) or dequantisation (scatter):
// entries are the payload rows of each block, scales per `span`.
hipError_t launch_token_fp8(bool gather, void* pool, const kvx_block_layout& layout, const BlockBatch& batch,
                            int64_t scale_offset, const TokenSpan& span, bool vector_ok, hipStream_t stream);
// True when 16-byte vector kernels may address this pool/entry combination.
bool vector_access_ok(const void* pool, const kvx_block_layout& layout, const uint64_t* entries, int32_t n);
hipError_t launch_store_kvcache(const void* key, int64_t key_stride, const void* value,
                                int64_t value_stride, void* k_cache, void* v_cache,
                                const int32_t* slot_mapping, int64_t num_tokens, int64_t row_elems,
                                int32_t elem_bytes, int64_t cache_slots, hipStream_t stream);
// Copies n bytes of pinned host memory at `src` (a device-accessible address)
// to device memory at `dst` with a kernel on `stream`; n < 2^31.
hipError_t launch_upload(void* dst, const void* src, int64_t n, hipStream_t stream);
hipError_t launch_sleep(hipStream_t stream, int64_t microseconds);
hipError_t launch_selftest(uint64_t* counters, hipStream_t stream);

}  // namespace kvx
