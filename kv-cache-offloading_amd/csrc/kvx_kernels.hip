// Device kernels of the KV-block copy path for CDNA4 (gfx950).
//
// All kernels stream: every byte of the pool, the staging buffers and the
// host entries is read or written once per pass, so they are bound by HBM
// (or host-link) bandwidth, not by MFMA or VALU throughput.
//
// Arithmetic contract of the FP8 codec (nanovllm/engine/cpu_prefix_cache.py:20-28):
//   scale = max(fp32(amax|x|) / 448, 1e-30f), stored as the scale dtype
//   code  = e4m3fn_rne(clamp(fp32(x) / fp32(scale), -448, 448))
//   back  = bf16_rne(fp32(code) * fp32(scale))
// The per-element division is evaluated as q0 = |x|*y, r = fma(-q0, s, |x|),
// q = fma(r, y, q0) with y = 1/s correctly rounded. For s in [2^-90, 2^120]
// this equals the IEEE quotient for every bf16 |x| (checked exhaustively over
// all bf16 x fp32 significand pairs by kvx_selftest); rows whose scale falls
// outside that range (non-finite or extreme amax) use IEEE division.
#include <stdarg.h>

#include "kvx_internal.h"

namespace kvx {
namespace {

constexpr int kThreads = 256;
constexpr float kFp8Max = 448.0f;
constexpr float kScaleFloor = 1e-30f;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Streaming memory access

// Nontemporal accesses: every byte is touched once per pass, so the data
// should not displace anything in the caches.
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt16(void* p, uint4 v) {
  u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// A 16-byte vector store with system scope (sc0 sc1: written through to
// memory, as host memory must be), for kernels that write pinned host slots.
// Measured on MI355X with one-block FP8 saves from 128 workgroups running
// beside a restore stream: 77 GB/s both ways against 71 with nontemporal
// stores, and concurrent bf16 matmuls took 1.4x their time alone instead of
// 1.7x.
__device__ __forceinline__ void store_host16(void* p, uint4 v) {
  u32x4 w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" : : "v"(p), "v"(w) : "memory");
}

template <bool kHost>
__device__ __forceinline__ void store16(void* p, uint4 v) {
  if (kHost) store_host16(p, v);
  else store_nt16(p, v);
}

// Reads of host memory at system scope (sc0 sc1): never served from a GPU
// cache line older than the host's or a DMA engine's last write there. Buffer
// loads through a resource over [base, base + bytes): the compiler tracks them
// like any other load, and a read past `bytes` returns zeros.
constexpr int kSystemScope = 1 | 16;  // cache-policy bits sc0 | sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t host_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 load_host16(__amdgpu_buffer_rsrc_t r, int offset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kSystemScope);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t load_host32(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, kSystemScope);
}

// Workgroups are dispatched round-robin over the chip's 8 XCDs, each with its
// own L2. xcd_tile<kChunk> maps workgroup IDs to tiles so that each XCD
// streams through runs of kChunk consecutive tiles, the XCDs taking runs in
// turn; kChunk < 0 gives each XCD one contiguous eighth of the grid. Measured
// on the Qwen3-8B block workload: one eighth per XCD (instead of every 8th
// tile) raised the FP8 kernels from ~5.5 to ~6.2-6.5 TB/s, and no run length
// beats it for the restore and store_kvcache kernels. The save kernel alone
// gains ~1% with runs of 1024 tiles, but a restore launched after such a save
// ran 0.4-0.5% slower, so the save keeps one eighth per XCD too. The BF16
// copies, with 1 KiB tiles, are fastest in the dispatcher's own order (0).
constexpr int kXcds = 8;
constexpr int kSaveXcdRun = -1;
constexpr int kCopyXcdRun = 0;
template <int kChunk = -1>
__device__ __forceinline__ int xcd_tile(int bid, int grid) {
  if (kChunk == 0) return bid;  // the dispatcher's own round-robin order
  if (kChunk < 0) {
    const int per = grid / kXcds;
    if (bid >= per * kXcds) return bid;  // the ragged tail keeps its place
    return (bid % kXcds) * per + bid / kXcds;
  }
  const int span = kXcds * kChunk;  // one run for each XCD
  if (bid >= grid / span * span) return bid;  // likewise
  const int nth = bid / kXcds;  // this workgroup's place in its XCD's sequence
  return nth / kChunk * span + (bid % kXcds) * kChunk + nth % kChunk;
}

// ---------------------------------------------------------------------------
// Scalar conversions

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16 in integer arithmetic; NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_sw(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 -> two bf16 (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

// Round-to-nearest-even fp32 -> e4m3fn (bias 7, no infinities, 0x7F/0xFF NaN,
// |f| >= 480 -> NaN), built from the format definition: normal codes keep
// 3 mantissa bits, values below 2^-6 are multiples of 2^-9.
__device__ __host__ __forceinline__ uint32_t f32_to_e4m3_sw(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u || a >= 0x43F00000u) return sign | 0x7Fu;  // NaN, or >= 480
  if (a < 0x3C800000u) {                                        // below 2^-6
    // |f| * 2^9 is exact; round it to an integer, ties to even.
    float t = __builtin_bit_cast(float, a) * 512.0f;
    uint32_t k = (uint32_t)t;
    float frac = t - (float)k;
    if (frac > 0.5f || (frac == 0.5f && (k & 1u))) ++k;
    return sign | k;  // k == 8 is the smallest normal, code 0x08
  }
  uint32_t exp = (a >> 23) - 127u + 7u;
  uint32_t keep = (a >> 20) & 7u;
  uint32_t rest = a & 0xFFFFFu;
  uint32_t code = (exp << 3) + keep;
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) ++code;  // carry may bump exp
  return sign | code;
}

// e4m3fn code -> fp32 from the format definition.
__device__ __forceinline__ float e4m3_to_f32_sw(uint32_t c) {
  uint32_t sign = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 15u, m = c & 7u;
  if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7FC00000u);
  float mag = e == 0 ? (float)m * 0x1p-9f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(mag) | sign);
}

// Four non-negative finite fp32 in [0, 448] -> four e4m3fn codes (v_cvt_pk_fp8_f32, RNE).
__device__ __forceinline__ uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
  uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}

// ---------------------------------------------------------------------------
// Row scale (cpu_prefix_cache.py:23) and the division it feeds (:24).

struct RowScale {
  float s;       // the stored scale, read back as fp32 (what :24 divides by)
  float y;       // correctly rounded 1/s
  uint32_t bits; // stored scale bits (bf16 in the low half, or fp32)
  bool fast;     // s in [2^-90, 2^120]: the reciprocal-FMA quotient is exact
};

template <bool kScaleBf16>
__device__ __forceinline__ RowScale row_scale(uint32_t amax_bits) {
  RowScale r;
  float s = bf16_bits_to_f32(amax_bits) / kFp8Max;
  s = s < kScaleFloor ? kScaleFloor : s;  // a NaN amax stays NaN, as clamp_min does
  if (kScaleBf16) {
    r.bits = f32x2_to_bf16x2(s, 0.0f) & 0xFFFFu;
    r.s = bf16_bits_to_f32(r.bits);
  } else {
    r.bits = __float_as_uint(s);
    r.s = s;
  }
  r.fast = r.s >= 0x1p-90f && r.s <= 0x1p120f;  // false for NaN and infinity
  r.y = 1.0f / r.s;
  return r;
}

// |q| for one bf16 element's magnitude bits (sign cleared), clamped to [0, 448].
__device__ __forceinline__ float quotient_fast(uint32_t mag_bits_hi, const RowScale& r) {
  float a = __uint_as_float(mag_bits_hi);
  float q0 = a * r.y;
  float rem = __builtin_fmaf(-q0, r.s, a);
  float q = __builtin_fmaf(rem, r.y, q0);
  return __builtin_amdgcn_fmed3f(q, 0.0f, kFp8Max);
}

// Slow path for rows with an out-of-range or non-finite scale: IEEE division;
// a NaN quotient encodes as 0x7F (the caller ORs the sign in).
__device__ __forceinline__ uint32_t code_slow(uint32_t mag_bits_hi, const RowScale& r) {
  float q = __uint_as_float(mag_bits_hi) / r.s;
  if (q != q) return 0x7Fu;
  return __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(q, 0.0f, kFp8Max), 0.0f, 0, false) & 0xFFu;
}

// Sign bits of four bf16 values (two packed words) placed at bit 7 of four bytes.
__device__ __forceinline__ uint32_t signs4(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x07050301u) & 0x80808080u;
}

// Quantises 8 bf16 (one uint4) to 8 e4m3 codes (one uint2).
__device__ __forceinline__ uint2 quantize8(uint4 x, const RowScale& r) {
  uint2 out;
  if (r.fast) {
    float q[8];
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q[2 * i] = quotient_fast((w[i] << 16) & 0x7FFF0000u, r);
      q[2 * i + 1] = quotient_fast(w[i] & 0x7FFF0000u, r);
    }
    out.x = f32x4_to_e4m3x4(q[0], q[1], q[2], q[3]);
    out.y = f32x4_to_e4m3x4(q[4], q[5], q[6], q[7]);
  } else {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[2 * i] = code_slow((w[i] << 16) & 0x7FFF0000u, r);
      c[2 * i + 1] = code_slow(w[i] & 0x7FFF0000u, r);
    }
    out.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    out.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  }
  out.x |= signs4(x.x, x.y);
  out.y |= signs4(x.z, x.w);
  return out;
}

// max |x| over 8 bf16 as bf16 bits. Comparing magnitudes as integers orders
// finite values and infinity correctly and ranks every NaN above infinity,
// so a NaN anywhere in the row propagates, as torch's amax does.
__device__ __forceinline__ uint32_t amax8(uint4 x) {
  const uint32_t m = 0x7FFF7FFFu;
  u16x2 a = __builtin_bit_cast(u16x2, x.x & m), b = __builtin_bit_cast(u16x2, x.y & m);
  u16x2 c = __builtin_bit_cast(u16x2, x.z & m), d = __builtin_bit_cast(u16x2, x.w & m);
  u16x2 t = __builtin_elementwise_max(__builtin_elementwise_max(a, b), __builtin_elementwise_max(c, d));
  return t.x > t.y ? t.x : t.y;
}

// Dequantises 8 codes (one uint2) with scale s to 8 bf16 (one uint4).
__device__ __forceinline__ uint4 dequantize8(uint2 c, float s) {
  f32x2 v0 = __builtin_amdgcn_cvt_pk_f32_fp8(c.x, false);
  f32x2 v1 = __builtin_amdgcn_cvt_pk_f32_fp8(c.x, true);
  f32x2 v2 = __builtin_amdgcn_cvt_pk_f32_fp8(c.y, false);
  f32x2 v3 = __builtin_amdgcn_cvt_pk_f32_fp8(c.y, true);
  uint4 o;
  o.x = f32x2_to_bf16x2(v0.x * s, v0.y * s);
  o.y = f32x2_to_bf16x2(v1.x * s, v1.y * s);
  o.z = f32x2_to_bf16x2(v2.x * s, v2.y * s);
  o.w = f32x2_to_bf16x2(v3.x * s, v3.y * s);
  return o;
}

template <int kLanes>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
#pragma unroll
  for (int off = kLanes / 2; off > 0; off /= 2) {
    uint32_t o = (uint32_t)__shfl_xor((int)v, off, kLanes);
    v = v > o ? v : o;
  }
  return v;
}

__device__ __forceinline__ float scale_value(const uint8_t* scales, int64_t row, bool bf16) {
  return bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(scales)[row])
              : reinterpret_cast<const float*>(scales)[row];
}

// The same from host memory (`r` covers one plane's scales): the scale's
// aligned 4-byte word, read at system scope.
__device__ __forceinline__ float scale_value_host(__amdgpu_buffer_rsrc_t r, int row, bool bf16) {
  if (!bf16) return __uint_as_float(load_host32(r, row * 4));
  const uint32_t w = load_host32(r, (row & ~1) * 2);
  return bf16_bits_to_f32((row & 1) ? w >> 16 : w & 0xFFFFu);
}

// ---------------------------------------------------------------------------
// FP8 save / restore, vector path: head_dim = kHd, kVec uint4 (8 bf16) per lane
// per row, so kHd / (8 * kVec) lanes share one row. A workgroup owns a tile of
// (threads / lanes) rows of one plane of one block.

template <int kHd, int kVec>
struct RowMap {
  static constexpr int kLanes = kHd / (8 * kVec);
  static_assert(kLanes >= 1 && kLanes <= 64 && (kLanes & (kLanes - 1)) == 0, "lanes per row");
};

struct TileCoord {
  int entry, plane, row0;
};

__device__ __forceinline__ TileCoord tile_coord_at(const PlaneGeom& g, int tile_rows, int tile) {
  const int per_entry = g.planes * g.chunks;
  TileCoord t;
  t.entry = tile / per_entry;
  const int rem = tile - t.entry * per_entry;
  t.plane = rem / g.chunks;
  t.row0 = (rem - t.plane * g.chunks) * tile_rows;
  return t;
}

template <int kChunk>
__device__ __forceinline__ TileCoord tile_coord(const PlaneGeom& g, int tile_rows) {
  return tile_coord_at(g, tile_rows, xcd_tile<kChunk>(blockIdx.x, gridDim.x));
}

// Save: one (token, head) row per kLanes lanes, one row per lane group; the
// tile's codes and scales are staged in LDS so that the stores write whole
// 128-byte lines (computing straight from the load layout leaves each store
// instruction with half lines, which cost ~11% extra HBM write traffic).
// kStride: saves written straight to host memory, by a capped grid whose
// workgroups stride over the tiles, with system-scope stores. Such a launch
// lasts as long as its writes take to cross the host link; a few workgroups
// keep the link busy and leave the CUs to other streams' kernels.
template <int kHd, int kVec, int kBlock, bool kScaleBf16, bool kStride>
__global__ __launch_bounds__(kBlock) void fp8_save_kernel(const uint16_t* __restrict__ pool, PlaneGeom g,
                                                         BlockBatch b) {
  using M = RowMap<kHd, kVec>;
  constexpr int kRows = kBlock / M::kLanes;       // rows per tile
  constexpr int kScaleBytes = kScaleBf16 ? 2 : 4;
  static_assert((kRows * kHd) % 16 == 0 && (kRows * kScaleBytes) % 16 == 0, "tile must store in 16-byte units");
  __shared__ uint4 codes[kRows * kHd / 16];
  __shared__ uint4 scale_tile[kRows * kScaleBytes / 16];
  const int tiles = kStride ? b.n * g.planes * g.chunks : 1;
  for (int tile = kStride ? (int)blockIdx.x : 0; tile < tiles; tile += kStride ? (int)gridDim.x : 1) {
  if (kStride) __syncthreads();  // the previous tile's stores have read the LDS tile
  const TileCoord tc = kStride ? tile_coord_at(g, kRows, tile) : tile_coord<kSaveXcdRun>(g, kRows);
  const int lane = threadIdx.x % M::kLanes;
  const int rsub = threadIdx.x / M::kLanes;
  const int row = tc.row0 + rsub;
  const int rows = tc.entry == b.n - 1 ? g.last_rows : g.plane_rows;  // valid rows of this plane
  const bool full = tc.row0 + kRows <= rows;
  const uint16_t* src = pool + (int64_t)b.ids[tc.entry] * g.block_stride + (int64_t)tc.plane * g.plane_stride;
  uint8_t* payload = reinterpret_cast<uint8_t*>(b.entries[tc.entry]) + (int64_t)tc.plane * g.payload_plane_stride;
  uint8_t* scales = reinterpret_cast<uint8_t*>(b.entries[tc.entry]) + g.scale_offset +
                    (int64_t)tc.entry * g.scale_entry_step + (int64_t)tc.plane * g.scale_plane_stride;

  uint4 x[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v)
    x[v] = row < rows ? load_nt16(src + (int64_t)row * kHd + v * (kHd / kVec) + lane * 8) : make_uint4(0, 0, 0, 0);
  uint32_t m = amax8(x[0]);
#pragma unroll
  for (int v = 1; v < kVec; ++v) {
    const uint32_t mv = amax8(x[v]);
    m = m > mv ? m : mv;
  }
  m = group_max<M::kLanes>(m);
  const RowScale r = row_scale<kScaleBf16>(m);
  uint2* code_words = reinterpret_cast<uint2*>(codes);
#pragma unroll
  for (int v = 0; v < kVec; ++v) code_words[(rsub * kHd + v * (kHd / kVec) + lane * 8) / 8] = quantize8(x[v], r);
  if (lane == 0) {
    if (kScaleBf16) reinterpret_cast<uint16_t*>(scale_tile)[rsub] = (uint16_t)r.bits;
    else reinterpret_cast<uint32_t*>(scale_tile)[rsub] = r.bits;
  }
  __syncthreads();
  uint8_t* tile_payload = payload + (int64_t)tc.row0 * kHd;
  for (int i = threadIdx.x; i < kRows * kHd / 16; i += kBlock)
    if (full || tc.row0 + i * 16 / kHd < rows) store16<kStride>(tile_payload + i * 16, codes[i]);
  if (full) {
    for (int i = threadIdx.x; i < kRows * kScaleBytes / 16; i += kBlock)
      store16<kStride>(scales + (int64_t)tc.row0 * kScaleBytes + i * 16, scale_tile[i]);
  } else if (lane == 0 && row < rows) {  // ragged last tile of a plane
    if (kScaleBf16) reinterpret_cast<uint16_t*>(scales)[row] = (uint16_t)r.bits;
    else reinterpret_cast<uint32_t*>(scales)[row] = r.bits;
  }
  }
}

// Restore: the tile's codes are loaded as whole 16-byte pieces with
// nontemporal loads into LDS, then each lane group reads back the codes of
// its row in the store layout. With head_dim 128 the store layout's own
// 8-byte code loads cover only half of each 128-byte line per instruction;
// loading through LDS raised the Qwen3-8B restore from ~6.23 to ~6.49 TB/s
// (one-wave workgroups; 128 and 256 threads gave ~6.48 and ~6.43).
// kStride: restores read straight from host slots, by a capped grid whose
// workgroups stride over the tiles (as the striding save instance).
template <int kHd, int kVec, int kBlock, bool kScaleBf16, bool kStride>
__global__ __launch_bounds__(kBlock) void fp8_restore_kernel(uint16_t* __restrict__ pool, PlaneGeom g,
                                                            BlockBatch b) {
  using M = RowMap<kHd, kVec>;
  constexpr int kRows = kBlock / M::kLanes;  // rows per tile
  constexpr int kPieces = kRows * kHd / 16;  // 16-byte pieces of the tile's codes
  __shared__ uint4 codes[kPieces];
  const int tiles = kStride ? b.n * g.planes * g.chunks : 1;
  for (int tile = kStride ? (int)blockIdx.x : 0; tile < tiles; tile += kStride ? (int)gridDim.x : 1) {
  if (kStride) __syncthreads();  // the previous tile's codes have been read back
  const TileCoord tc = kStride ? tile_coord_at(g, kRows, tile) : tile_coord<-1>(g, kRows);
  const int lane = threadIdx.x % M::kLanes;
  const int rsub = threadIdx.x / M::kLanes;
  const int row = tc.row0 + rsub;
  const int rows = tc.entry == b.n - 1 ? g.last_rows : g.plane_rows;  // valid rows of this plane
  uint16_t* dst = pool + (int64_t)b.ids[tc.entry] * g.block_stride + (int64_t)tc.plane * g.plane_stride;
  const uint8_t* payload =
      reinterpret_cast<const uint8_t*>(b.entries[tc.entry]) + (int64_t)tc.plane * g.payload_plane_stride;
  const uint8_t* scales = reinterpret_cast<const uint8_t*>(b.entries[tc.entry]) + g.scale_offset +
                          (int64_t)tc.entry * g.scale_entry_step + (int64_t)tc.plane * g.scale_plane_stride;

  const uint8_t* tile_codes = payload + (int64_t)tc.row0 * kHd;
  float s = 0.0f;
  if (kStride) {  // entries in host memory
    const int left = rows - tc.row0;
    const int tile_bytes = (left < 0 ? 0 : left < kRows ? left : kRows) * kHd;
    const __amdgpu_buffer_rsrc_t rc = host_rsrc(tile_codes, tile_bytes);
    for (int i = threadIdx.x; i < kPieces; i += kBlock) codes[i] = load_host16(rc, i * 16);
    if (row < rows) s = scale_value_host(host_rsrc(scales, (int64_t)rows * (kScaleBf16 ? 2 : 4)), row, kScaleBf16);
  } else {
    for (int i = threadIdx.x; i < kPieces; i += kBlock)
      codes[i] = tc.row0 + i * 16 / kHd < rows ? load_nt16(tile_codes + i * 16) : make_uint4(0, 0, 0, 0);
    if (row < rows) s = scale_value(scales, row, kScaleBf16);
  }
  __syncthreads();
  if (row < rows) {
    const uint2* code_words = reinterpret_cast<const uint2*>(codes);
#pragma unroll
    for (int v = 0; v < kVec; ++v) {
      const int col = v * (kHd / kVec) + lane * 8;
      store_nt16(dst + (int64_t)row * kHd + col, dequantize8(code_words[(rsub * kHd + col) / 8], s));
    }
  }
  }
}

// ---------------------------------------------------------------------------
// FP8 save / restore, generic path (any head_dim): one thread per row.

__device__ __forceinline__ bool generic_row(const PlaneGeom& g, int n, int64_t& entry, int64_t& plane,
                                            int64_t& row) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t per_entry = (int64_t)g.planes * g.plane_rows;
  entry = idx / per_entry;
  if (entry >= n) return false;
  const int64_t rem = idx - entry * per_entry;
  plane = rem / g.plane_rows;
  row = rem - plane * g.plane_rows;
  return row < (entry == n - 1 ? g.last_rows : g.plane_rows);
}

template <bool kScaleBf16>
__global__ __launch_bounds__(kThreads) void fp8_save_generic(const uint16_t* __restrict__ pool, PlaneGeom g,
                                                            BlockBatch b) {
  int64_t e, p, row;
  if (!generic_row(g, b.n, e, p, row)) return;
  const int hd = g.head_dim;
  const uint16_t* src = pool + (int64_t)b.ids[e] * g.block_stride + p * g.plane_stride + row * hd;
  uint8_t* payload = reinterpret_cast<uint8_t*>(b.entries[e]) + p * g.payload_plane_stride + row * hd;
  uint8_t* scales = reinterpret_cast<uint8_t*>(b.entries[e]) + g.scale_offset + e * g.scale_entry_step +
                    p * g.scale_plane_stride;
  uint32_t m = 0;
  for (int i = 0; i < hd; ++i) {
    uint32_t a = src[i] & 0x7FFFu;
    m = m > a ? m : a;
  }
  const RowScale r = row_scale<kScaleBf16>(m);
  for (int i = 0; i < hd; ++i) {
    const uint32_t h = src[i];
    const uint32_t mag = (h & 0x7FFFu) << 16;
    uint32_t code = r.fast ? (__builtin_amdgcn_cvt_pk_fp8_f32(quotient_fast(mag, r), 0.0f, 0, false) & 0xFFu)
                           : code_slow(mag, r);
    payload[i] = (uint8_t)(code | ((h >> 8) & 0x80u));
  }
  if (kScaleBf16) reinterpret_cast<uint16_t*>(scales)[row] = (uint16_t)r.bits;
  else reinterpret_cast<uint32_t*>(scales)[row] = r.bits;
}

template <bool kScaleBf16>
__global__ __launch_bounds__(kThreads) void fp8_restore_generic(uint16_t* __restrict__ pool, PlaneGeom g,
                                                               BlockBatch b) {
  int64_t e, p, row;
  if (!generic_row(g, b.n, e, p, row)) return;
  const int hd = g.head_dim;
  uint16_t* dst = pool + (int64_t)b.ids[e] * g.block_stride + p * g.plane_stride + row * hd;
  const uint8_t* payload = reinterpret_cast<const uint8_t*>(b.entries[e]) + p * g.payload_plane_stride + row * hd;
  const uint8_t* scales = reinterpret_cast<const uint8_t*>(b.entries[e]) + g.scale_offset + e * g.scale_entry_step +
                          p * g.scale_plane_stride;
  const float s = scale_value(scales, row, kScaleBf16);
  for (int i = 0; i < hd; ++i) {
    const float v = __builtin_amdgcn_cvt_f32_fp8((uint32_t)payload[i], 0);
    dst[i] = (uint16_t)(f32x2_to_bf16x2(v * s, 0.0f) & 0xFFFFu);
  }
}

// ---------------------------------------------------------------------------
// RAW (BF16 mode) gather / scatter: byte copies of each block plane.

// Tile shape of the device-side copies: one nontemporal 16-byte piece per
// thread in 64-thread workgroups (1 KiB tiles), taken in the dispatcher's
// order. Measured on 128 Qwen3-8B blocks (TB/s, gather / scatter, median of
// two passes): 6.71 / 6.62, against 6.28 / 6.31 for 8 KiB tiles of 256
// threads in 64-tile runs per XCD, 6.59 / 6.58 for 1 KiB tiles in one
// contiguous eighth per XCD, 6.34 / 6.33 for 2 KiB tiles of 128 threads and
// 5.45 / 5.53 for 2 KiB tiles of 64 threads. A plain 1:1 streaming copy of
// the same bytes reaches 6.63-6.73 (hipMemcpyAsync device to device: 4.25).
// Striding copies to or from host memory keep 16 KiB tiles of 256 threads:
// their few workgroups need the larger tiles in flight to keep the host link
// busy.
constexpr int kCopyThreads = 64;
constexpr int kCopyVecs = 1;
constexpr int kStrideCopyVecs = 4;

// Entry e receives plane p of its block at entries[e] + p * entry_plane_stride;
// every entry copies plane_bytes per plane except the batch's last, which
// copies last_bytes (a sequence's partial final block in a token gather).
// kStride: copies to or from host memory by a capped striding grid, as the
// FP8 kernels' striding instances; writes to host memory use system-scope stores.
template <bool kToEntry, bool kStride, int kBlock = kStride ? kThreads : kCopyThreads>
__global__ __launch_bounds__(kBlock) void raw_copy_kernel(uint8_t* __restrict__ pool, PlaneGeom g,
                                                         BlockBatch b, int64_t plane_bytes,
                                                         int64_t elem_bytes, int64_t entry_plane_stride,
                                                         int64_t last_bytes) {
  constexpr int kVecs = kStride ? kStrideCopyVecs : kCopyVecs;
  constexpr int kTileBytes = kBlock * kVecs * 16;
  const int per_entry = g.planes * g.chunks;
  const int tiles = kStride ? b.n * per_entry : 1;
  for (int t = kStride ? (int)blockIdx.x : 0; t < tiles; t += kStride ? (int)gridDim.x : 1) {
  const int tile = kStride ? t : xcd_tile<kCopyXcdRun>(blockIdx.x, gridDim.x);
  const int e = tile / per_entry;
  const int rem = tile - e * per_entry;
  const int p = rem / g.chunks;
  const int64_t off0 = (int64_t)(rem - p * g.chunks) * kTileBytes;
  const int64_t valid = e == b.n - 1 ? last_bytes : plane_bytes;
  uint8_t* pl = pool + ((int64_t)b.ids[e] * g.block_stride + (int64_t)p * g.plane_stride) * elem_bytes;
  uint8_t* en = reinterpret_cast<uint8_t*>(b.entries[e]) + (int64_t)p * entry_plane_stride;
  const uint8_t* src = kToEntry ? pl : en;
  uint8_t* dst = kToEntry ? en : pl;
  uint4 v[kVecs];
#pragma unroll
  for (int k = 0; k < kVecs; ++k) {
    const int64_t off = off0 + ((int64_t)k * kBlock + threadIdx.x) * 16;
    if (kStride && !kToEntry)  // from host memory; past `valid` the resource reads zeros
      v[k] = load_host16(host_rsrc(src + off0, valid - off0), (int)(off - off0));
    else
      v[k] = off < valid ? load_nt16(src + off) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int k = 0; k < kVecs; ++k) {
    const int64_t off = off0 + ((int64_t)k * kBlock + threadIdx.x) * 16;
    if (off < valid) store16<kStride && kToEntry>(dst + off, v[k]);
  }
  }
}

// Sizes or strides that are not multiples of 16 bytes: 2-byte granules.
template <bool kToEntry>
__global__ __launch_bounds__(kThreads) void raw_copy_generic(uint8_t* __restrict__ pool, PlaneGeom g,
                                                            BlockBatch b, int64_t plane_bytes,
                                                            int64_t elem_bytes, int64_t entry_plane_stride,
                                                            int64_t last_bytes) {
  const int64_t granules = plane_bytes / 2;
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t per_entry = granules * g.planes;
  const int64_t e = idx / per_entry;
  if (e >= b.n) return;
  const int64_t rem = idx - e * per_entry;
  const int64_t p = rem / granules;
  const int64_t k = rem - p * granules;
  if (e == b.n - 1 && k >= last_bytes / 2) return;
  uint16_t* pl = reinterpret_cast<uint16_t*>(pool + ((int64_t)b.ids[e] * g.block_stride + p * g.plane_stride) * elem_bytes);
  uint16_t* en = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(b.entries[e]) + p * entry_plane_stride);
  if (kToEntry) en[k] = pl[k];
  else pl[k] = en[k];
}

// ---------------------------------------------------------------------------
// store_kvcache (nanovllm/layers/attention.py:10-30)

// Rows of kRow16 uint4: each thread moves one 16-byte piece of a token's K
// row or V row, kStoreThreads consecutive pieces per workgroup. One access
// per thread, nontemporal accesses and XCD-contiguous token ranges were the
// fastest shape on the 16-sequence Qwen3-8B batch (random slots: 4.77 -> 5.29
// TB/s; contiguous slots: 4.85 -> 5.89 TB/s); several passes per workgroup
// were slower. Workgroup size and order, as fractions of 8 TB/s (random /
// paged-block / contiguous slots, two passes agreeing within 0.1 point):
// 128 threads in eighths 67.2 / 75.1 / 76.4; 256 in eighths 66.6 / 74.3 /
// 75.4; 64 in eighths 66.9 / 75.0 / 76.2; 64 in dispatch order 66.7 / 75.5 /
// 77.6; 64 in 64-workgroup runs 65.0 / 71.2 / 75.0.
constexpr int kStoreThreads = 128;
constexpr int kStoreXcdRun = -1;
template <int kRow16>
__global__ __launch_bounds__(kStoreThreads) void store_kv_vec(const uint4* __restrict__ key, int64_t key_stride16,
                                                             const uint4* __restrict__ value, int64_t value_stride16,
                                                             uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
                                                             const int32_t* __restrict__ slots, int64_t n,
                                                             int64_t cache_slots) {
  // 16-byte piece p of the batch: token p / (2 kRow16), then its K row and its V row.
  const int64_t p = (int64_t)xcd_tile<kStoreXcdRun>(blockIdx.x, gridDim.x) * kStoreThreads + threadIdx.x;
  const int64_t t = p / (2 * kRow16);
  const int within = (int)(p - t * (2 * kRow16));
  const bool is_v = within >= kRow16;
  const int col = is_v ? within - kRow16 : within;
  if (t >= n) return;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= cache_slots) return;
  const uint4 v = load_nt16((is_v ? value : key) + t * (is_v ? value_stride16 : key_stride16) + col);
  store_nt16((is_v ? v_cache : k_cache) + slot * kRow16 + col, v);
}

// Any row size / alignment: one workgroup per token, copying granules of T
// (row, strides in units of T).
template <typename T>
__global__ __launch_bounds__(kThreads) void store_kv_generic(const T* __restrict__ key, int64_t key_stride,
                                                            const T* __restrict__ value, int64_t value_stride,
                                                            T* __restrict__ k_cache, T* __restrict__ v_cache,
                                                            const int32_t* __restrict__ slots, int64_t row,
                                                            int64_t cache_slots) {
  const int64_t t = blockIdx.x;
  const int64_t s = slots[t];
  if (s < 0 || s >= cache_slots) return;
  for (int64_t i = threadIdx.x; i < 2 * row; i += kThreads) {
    if (i < row) k_cache[s * row + i] = key[t * key_stride + i];
    else v_cache[s * row + i - row] = value[t * value_stride + i - row];
  }
}

// ---------------------------------------------------------------------------
// Test delay (bench/test_automatic_cpu_cache.py:47-48): one wave polls the
// device wall clock until `ticks` have passed.

// ---------------------------------------------------------------------------
// Host-to-device uploads read by a kernel

// A host-to-device copy queued on the caller's stream waits behind every
// host-to-device DMA already queued on the device, whichever stream queued
// it: on MI355X a 128 KiB pinned upload beside 2 GB of restore DMA on another
// stream finished only when the DMA did (33.4 ms, against 0.04 ms alone). A
// kernel on the caller's stream that reads the pinned source over the host
// link leaves the DMA queue out. 16-byte system-scope loads when source and
// destination allow them, else bytes; the buffer resource bounds every read
// to [src, src + n).
constexpr int kUploadThreads = 256;
constexpr int kUploadMaxGrid = 64;

template <bool kVec>
__global__ __launch_bounds__(kUploadThreads) void upload_kernel(uint8_t* __restrict__ dst, const uint8_t* src,
                                                               int64_t n) {
  const __amdgpu_buffer_rsrc_t r = host_rsrc(src, n);
  const int64_t first = (int64_t)blockIdx.x * kUploadThreads + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kUploadThreads;
  int64_t done = 0;
  if (kVec) {
    const int64_t pieces = n / 16;
    for (int64_t i = first; i < pieces; i += step)
      *reinterpret_cast<uint4*>(dst + i * 16) = load_host16(r, (int)(i * 16));
    done = pieces * 16;
  }
  for (int64_t i = done + first; i < n; i += step)
    dst[i] = __builtin_amdgcn_raw_buffer_load_b8(r, (int)i, 0, kSystemScope);
}

__global__ void sleep_kernel(uint64_t ticks) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(32);
}

// ---------------------------------------------------------------------------
// Self-test sweeps (see kvx_selftest in kvx.h).

__device__ __forceinline__ void count(uint64_t* c, int i, uint32_t n) {
  // Wave-level sum, then one atomic per wave.
  uint64_t v = n;
#pragma unroll
  for (int off = 32; off > 0; off /= 2) v += __shfl_xor(v, off);
  if ((threadIdx.x & 63) == 0 && v) atomicAdd((unsigned long long*)&c[i], (unsigned long long)v);
}

__global__ __launch_bounds__(kThreads) void selftest_conversions(uint64_t* c) {
  // Sweep every fp32 bit pattern: 2^32 = gridDim * 256 * 64 inputs.
  const uint64_t base = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * 64;
  uint32_t bad_e4m3 = 0, bad_bf16 = 0, bad_nan = 0;
  for (int k = 0; k < 64; k += 2) {
    const uint32_t u0 = (uint32_t)(base + k), u1 = (uint32_t)(base + k + 1);
    const float f0 = __uint_as_float(u0), f1 = __uint_as_float(u1);
    // e4m3: the kernels convert fmed3(q, 0, 448) of finite q.
    const float q0 = __builtin_amdgcn_fmed3f(f0, 0.0f, kFp8Max);
    const float q1 = __builtin_amdgcn_fmed3f(f1, 0.0f, kFp8Max);
    const uint32_t hw = __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false);
    if (f0 == f0) bad_e4m3 += (hw & 0xFFu) != f32_to_e4m3_sw(q0);
    if (f1 == f1) bad_e4m3 += ((hw >> 8) & 0xFFu) != f32_to_e4m3_sw(q1);
    // bf16 RNE.
    const uint32_t hb = f32x2_to_bf16x2(f0, f1);
    if (f0 == f0) bad_bf16 += (hb & 0xFFFFu) != f32_to_bf16_sw(f0);
    else bad_nan += ((hb & 0x7FFFu) <= 0x7F80u);
    if (f1 == f1) bad_bf16 += (hb >> 16) != f32_to_bf16_sw(f1);
    else bad_nan += (((hb >> 16) & 0x7FFFu) <= 0x7F80u);
  }
  count(c, 0, bad_e4m3);
  count(c, 1, bad_bf16);
  count(c, 2, bad_nan);
  if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd((unsigned long long*)&c[5], 4096ull);
}

__global__ __launch_bounds__(kThreads) void selftest_division(uint64_t* c) {
  // Every (bf16 significand a, fp32 significand b) pair in [1, 2): the
  // reciprocal-FMA quotient must equal IEEE division. blockIdx/thread pick b;
  // each thread loops over the 128 a.
  const uint32_t mb = (uint32_t)blockIdx.x * kThreads + threadIdx.x;  // < 2^23
  const float b = __uint_as_float(0x3F800000u | mb);
  RowScale r;
  r.s = b;
  r.y = 1.0f / b;
  r.fast = true;
  uint32_t bad = 0;
  for (uint32_t ma = 0; ma < 128; ++ma) {
    const float a = __uint_as_float(0x3F800000u | (ma << 16));
    const float q0 = a * r.y;
    const float rem = __builtin_fmaf(-q0, r.s, a);
    const float q = __builtin_fmaf(rem, r.y, q0);
    bad += __float_as_uint(q) != __float_as_uint(a / b);
  }
  count(c, 3, bad);
  if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd((unsigned long long*)&c[6], 1024ull);
}

__global__ void selftest_decode(uint64_t* c) {
  const uint32_t code = threadIdx.x;  // 256 threads
  const float hw = __builtin_amdgcn_cvt_f32_fp8(code, 0);
  const float sw = e4m3_to_f32_sw(code);
  uint32_t bad = (hw != hw) ? (sw == sw) : (__float_as_uint(hw) != __float_as_uint(sw));
  count(c, 4, bad);
  if (threadIdx.x == 0) atomicAdd((unsigned long long*)&c[7], 1ull);
}

__global__ void zero_counters(uint64_t* c) {
  if (threadIdx.x < 8) c[threadIdx.x] = 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers

// Geometry of block entries (dense per block); `span` switches FP8 entries to token entries.
static PlaneGeom make_geom(const kvx_block_layout& l, int tile_rows, int64_t scale_offset,
                           const TokenSpan* span = nullptr) {
  PlaneGeom g;
  g.plane_stride = l.plane_stride;
  g.block_stride = l.block_stride;
  g.scale_offset = scale_offset;
  const int64_t scale_bytes = l.scale_dtype == KVX_SCALE_BF16 ? 2 : 4;
  g.payload_plane_stride = span ? span->payload_plane_stride : (int64_t)l.plane_rows * l.head_dim;
  g.scale_plane_stride = span ? span->scale_plane_stride : (int64_t)l.plane_rows * scale_bytes;
  g.scale_entry_step = span ? span->scale_entry_step : 0;
  g.planes = l.planes;
  g.plane_rows = l.plane_rows;
  g.last_rows = span ? span->last_rows : l.plane_rows;
  g.head_dim = l.head_dim;
  g.chunks = tile_rows > 0 ? (l.plane_rows + tile_rows - 1) / tile_rows : 0;
  return g;
}

static unsigned generic_grid(int64_t items) { return (unsigned)((items + kThreads - 1) / kThreads); }

template <bool kScaleBf16>
static hipError_t launch_fp8(bool save, void* pool, const kvx_block_layout& l, const BlockBatch& b,
                             int64_t scale_offset, bool vector_ok, int32_t max_grid, hipStream_t stream,
                             const TokenSpan* span = nullptr) {
  // Workgroup sizes chosen by sweeps on the Qwen3-8B block workload: save
  // 128 threads (16 rows for hd=128), restore 64 threads (8 rows). A capped
  // (striding) restore reads host slots and needs more bytes in flight per
  // workgroup: 256 threads (32 rows).
  constexpr int kSaveBlock = 128;
  constexpr int kRestoreBlock = 64;
  constexpr int kRestoreStrideBlock = 256;
  auto run = [&](auto save_k, auto save_stride_k, auto restore_k, auto restore_stride_k, int lanes) -> hipError_t {
    const int block = save ? kSaveBlock : kRestoreBlock;
    PlaneGeom g = make_geom(l, block / lanes, scale_offset, span);
    const unsigned grid = (unsigned)(b.n * g.planes * g.chunks);
    if (save && max_grid > 0 && (unsigned)max_grid < grid) {
      hipLaunchKernelGGL(save_stride_k, dim3((unsigned)max_grid), dim3(kSaveBlock), 0, stream, (const uint16_t*)pool,
                         g, b);
    } else if (save) {
      hipLaunchKernelGGL(save_k, dim3(grid), dim3(kSaveBlock), 0, stream, (const uint16_t*)pool, g, b);
    } else if (max_grid > 0) {
      PlaneGeom gs = make_geom(l, kRestoreStrideBlock / lanes, scale_offset, span);
      const unsigned tiles = (unsigned)(b.n * gs.planes * gs.chunks);
      hipLaunchKernelGGL(restore_stride_k, dim3((unsigned)max_grid < tiles ? (unsigned)max_grid : tiles), dim3(kRestoreStrideBlock), 0,
                         stream, (uint16_t*)pool, gs, b);
    } else {
      hipLaunchKernelGGL(restore_k, dim3(grid), dim3(kRestoreBlock), 0, stream, (uint16_t*)pool, g, b);
    }
    return hipGetLastError();
  };
  switch (vector_ok ? l.head_dim : 0) {
    case 64:
      return run(fp8_save_kernel<64, 1, kSaveBlock, kScaleBf16, false>,
                 fp8_save_kernel<64, 1, kSaveBlock, kScaleBf16, true>,
                 fp8_restore_kernel<64, 1, kRestoreBlock, kScaleBf16, false>,
                 fp8_restore_kernel<64, 1, kRestoreStrideBlock, kScaleBf16, true>, RowMap<64, 1>::kLanes);
    case 128:
      return run(fp8_save_kernel<128, 2, kSaveBlock, kScaleBf16, false>,
                 fp8_save_kernel<128, 2, kSaveBlock, kScaleBf16, true>,
                 fp8_restore_kernel<128, 2, kRestoreBlock, kScaleBf16, false>,
                 fp8_restore_kernel<128, 2, kRestoreStrideBlock, kScaleBf16, true>, RowMap<128, 2>::kLanes);
    case 256:
      return run(fp8_save_kernel<256, 2, kSaveBlock, kScaleBf16, false>,
                 fp8_save_kernel<256, 2, kSaveBlock, kScaleBf16, true>,
                 fp8_restore_kernel<256, 2, kRestoreBlock, kScaleBf16, false>,
                 fp8_restore_kernel<256, 2, kRestoreStrideBlock, kScaleBf16, true>, RowMap<256, 2>::kLanes);
    default: {
      PlaneGeom g = make_geom(l, 0, scale_offset, span);
      const unsigned grid = generic_grid((int64_t)b.n * l.planes * l.plane_rows);
      if (save)
        hipLaunchKernelGGL(fp8_save_generic<kScaleBf16>, dim3(grid), dim3(kThreads), 0, stream,
                           (const uint16_t*)pool, g, b);
      else
        hipLaunchKernelGGL(fp8_restore_generic<kScaleBf16>, dim3(grid), dim3(kThreads), 0, stream,
                           (uint16_t*)pool, g, b);
      return hipGetLastError();
    }
  }
}

static hipError_t launch_raw(bool to_entry, void* pool, const kvx_block_layout& l, const BlockBatch& b,
                             bool vector_ok, int64_t entry_plane_stride, int64_t last_bytes, int32_t max_grid,
                             hipStream_t stream) {
  const int64_t plane_bytes = (int64_t)l.plane_rows * l.head_dim * l.elem_bytes;
  if (entry_plane_stride < 0) entry_plane_stride = plane_bytes;
  if (last_bytes < 0) last_bytes = plane_bytes;
  const bool vec = vector_ok && plane_bytes % 16 == 0 && entry_plane_stride % 16 == 0 && last_bytes % 16 == 0;
  const int64_t es = l.elem_bytes;
  if (vec) {
    auto tiled = [&](int threads, int vecs) {
      const int64_t tile_bytes = (int64_t)threads * vecs * 16;
      PlaneGeom g = make_geom(l, 0, 0);
      g.chunks = (int32_t)((plane_bytes + tile_bytes - 1) / tile_bytes);
      return g;
    };
    if (max_grid > 0) {
      const PlaneGeom g = tiled(kThreads, kStrideCopyVecs);
      if ((unsigned)max_grid < (unsigned)(b.n * g.planes * g.chunks)) {
        if (to_entry)
          hipLaunchKernelGGL((raw_copy_kernel<true, true>), dim3((unsigned)max_grid), dim3(kThreads), 0, stream,
                             (uint8_t*)pool, g, b, plane_bytes, es, entry_plane_stride, last_bytes);
        else
          hipLaunchKernelGGL((raw_copy_kernel<false, true>), dim3((unsigned)max_grid), dim3(kThreads), 0, stream,
                             (uint8_t*)pool, g, b, plane_bytes, es, entry_plane_stride, last_bytes);
        return hipGetLastError();
      }
    }
    const PlaneGeom g = tiled(kCopyThreads, kCopyVecs);
    const unsigned grid = (unsigned)(b.n * g.planes * g.chunks);
    if (to_entry)
      hipLaunchKernelGGL((raw_copy_kernel<true, false>), dim3(grid), dim3(kCopyThreads), 0, stream, (uint8_t*)pool, g,
                         b, plane_bytes, es, entry_plane_stride, last_bytes);
    else
      hipLaunchKernelGGL((raw_copy_kernel<false, false>), dim3(grid), dim3(kCopyThreads), 0, stream, (uint8_t*)pool,
                         g, b, plane_bytes, es, entry_plane_stride, last_bytes);
  } else {
    PlaneGeom g = make_geom(l, 0, 0);
    const unsigned grid = generic_grid((int64_t)b.n * l.planes * (plane_bytes / 2));
    if (to_entry)
      hipLaunchKernelGGL(raw_copy_generic<true>, dim3(grid), dim3(kThreads), 0, stream, (uint8_t*)pool, g, b,
                         plane_bytes, es, entry_plane_stride, last_bytes);
    else
      hipLaunchKernelGGL(raw_copy_generic<false>, dim3(grid), dim3(kThreads), 0, stream, (uint8_t*)pool, g, b,
                         plane_bytes, es, entry_plane_stride, last_bytes);
  }
  return hipGetLastError();
}

hipError_t launch_token_copy(bool gather, void* pool, const kvx_block_layout& l, const BlockBatch& b,
                             bool vector_ok, int64_t dense_plane_stride, int64_t last_bytes, hipStream_t stream) {
  if (b.n <= 0) return hipSuccess;
  return launch_raw(gather, pool, l, b, vector_ok, dense_plane_stride, last_bytes, 0, stream);
}

hipError_t launch_token_fp8(bool gather, void* pool, const kvx_block_layout& l, const BlockBatch& b,
                            int64_t scale_offset, const TokenSpan& span, bool vector_ok, hipStream_t stream) {
  if (b.n <= 0) return hipSuccess;
  return l.scale_dtype == KVX_SCALE_BF16
             ? launch_fp8<true>(gather, pool, l, b, scale_offset, vector_ok, 0, stream, &span)
             : launch_fp8<false>(gather, pool, l, b, scale_offset, vector_ok, 0, stream, &span);
}

bool vector_access_ok(const void* pool, const kvx_block_layout& l, const uint64_t* entries, int32_t n) {
  const int64_t es = l.elem_bytes;
  if ((uintptr_t)pool % 16 || (l.plane_stride * es) % 16 || (l.block_stride * es) % 16) return false;
  for (int32_t i = 0; i < n; ++i)
    if (entries[i] % 16) return false;
  return true;
}

hipError_t launch_save(const void* pool, const kvx_block_layout& l, int32_t format, const BlockBatch& b,
                       int64_t scale_offset, bool vector_ok, int32_t max_grid, hipStream_t stream) {
  if (b.n <= 0) return hipSuccess;
  void* p = const_cast<void*>(pool);
  if (format == KVX_FORMAT_RAW) return launch_raw(true, p, l, b, vector_ok, -1, -1, max_grid, stream);
  return l.scale_dtype == KVX_SCALE_BF16
             ? launch_fp8<true>(true, p, l, b, scale_offset, vector_ok, max_grid, stream)
             : launch_fp8<false>(true, p, l, b, scale_offset, vector_ok, max_grid, stream);
}

bool striding_restore_supported(const kvx_block_layout& l, int32_t format, bool vector_ok) {
  if (!vector_ok) return false;
  if (format == KVX_FORMAT_RAW) return ((int64_t)l.plane_rows * l.head_dim * l.elem_bytes) % 16 == 0;
  return l.head_dim == 64 || l.head_dim == 128 || l.head_dim == 256;  // launch_fp8's vector kernels
}

hipError_t launch_restore(void* pool, const kvx_block_layout& l, int32_t format, const BlockBatch& b,
                          int64_t scale_offset, bool vector_ok, int32_t max_grid, hipStream_t stream) {
  if (b.n <= 0) return hipSuccess;
  if (format == KVX_FORMAT_RAW) return launch_raw(false, pool, l, b, vector_ok, -1, -1, max_grid, stream);
  return l.scale_dtype == KVX_SCALE_BF16
             ? launch_fp8<true>(false, pool, l, b, scale_offset, vector_ok, max_grid, stream)
             : launch_fp8<false>(false, pool, l, b, scale_offset, vector_ok, max_grid, stream);
}

hipError_t launch_store_kvcache(const void* key, int64_t key_stride, const void* value, int64_t value_stride,
                                void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t n,
                                int64_t row_elems, int32_t elem_bytes, int64_t cache_slots, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t row_bytes = row_elems * elem_bytes;
  const int64_t ks = key_stride * elem_bytes, vs = value_stride * elem_bytes;
  const bool aligned = ((uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0 &&
                       ks % 16 == 0 && vs % 16 == 0 && row_bytes % 16 == 0;
  auto vec = [&](auto kernel, int row16) {
    const int64_t grid = (n * 2 * row16 + kStoreThreads - 1) / kStoreThreads;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kStoreThreads), 0, stream, (const uint4*)key, ks / 16,
                       (const uint4*)value, vs / 16, (uint4*)k_cache, (uint4*)v_cache, slot_mapping, n,
                       cache_slots);
    return hipGetLastError();
  };
  if (aligned) {
    switch (row_bytes / 16) {
      case 8: return vec(store_kv_vec<8>, 8);
      case 16: return vec(store_kv_vec<16>, 16);
      case 32: return vec(store_kv_vec<32>, 32);
      case 64: return vec(store_kv_vec<64>, 64);
      case 128: return vec(store_kv_vec<128>, 128);
      default: break;
    }
  }
  // Generic path: granules of the element size when it is 2 or 4 bytes, else bytes.
  const unsigned grid = (unsigned)n;
  if (elem_bytes == 2) {
    hipLaunchKernelGGL(store_kv_generic<uint16_t>, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)key,
                       key_stride, (const uint16_t*)value, value_stride, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       slot_mapping, row_elems, cache_slots);
  } else if (elem_bytes == 4) {
    hipLaunchKernelGGL(store_kv_generic<uint32_t>, dim3(grid), dim3(kThreads), 0, stream, (const uint32_t*)key,
                       key_stride, (const uint32_t*)value, value_stride, (uint32_t*)k_cache, (uint32_t*)v_cache,
                       slot_mapping, row_elems, cache_slots);
  } else {
    hipLaunchKernelGGL(store_kv_generic<uint8_t>, dim3(grid), dim3(kThreads), 0, stream, (const uint8_t*)key, ks,
                       (const uint8_t*)value, vs, (uint8_t*)k_cache, (uint8_t*)v_cache, slot_mapping, row_bytes,
                       cache_slots);
  }
  return hipGetLastError();
}

hipError_t launch_upload(void* dst, const void* src, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const bool vec = ((uintptr_t)dst | (uintptr_t)src) % 16 == 0;
  const int64_t units = vec ? (n + 15) / 16 : n;
  const unsigned grid = (unsigned)std::min<int64_t>(kUploadMaxGrid, (units + kUploadThreads - 1) / kUploadThreads);
  if (vec)
    hipLaunchKernelGGL(upload_kernel<true>, dim3(grid), dim3(kUploadThreads), 0, stream, (uint8_t*)dst,
                       (const uint8_t*)src, n);
  else
    hipLaunchKernelGGL(upload_kernel<false>, dim3(grid), dim3(kUploadThreads), 0, stream, (uint8_t*)dst,
                       (const uint8_t*)src, n);
  return hipGetLastError();
}

hipError_t launch_sleep(hipStream_t stream, int64_t microseconds) {
  int device = 0, khz = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  err = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device);
  if (err != hipSuccess) return err;
  if (khz <= 0) khz = 100000;  // 100 MHz, the MI300-series constant clock
  const uint64_t ticks = (uint64_t)microseconds * (uint64_t)khz / 1000u;
  hipLaunchKernelGGL(sleep_kernel, dim3(1), dim3(64), 0, stream, ticks);
  return hipGetLastError();
}

hipError_t launch_selftest(uint64_t* counters, hipStream_t stream) {
  hipLaunchKernelGGL(zero_counters, dim3(1), dim3(64), 0, stream, counters);
  // 2^32 inputs / (256 threads * 64 per thread) = 2^18 workgroups.
  hipLaunchKernelGGL(selftest_conversions, dim3(1u << 18), dim3(kThreads), 0, stream, counters);
  // 2^23 fp32 significands / 256 threads = 2^15 workgroups.
  hipLaunchKernelGGL(selftest_division, dim3(1u << 15), dim3(kThreads), 0, stream, counters);
  hipLaunchKernelGGL(selftest_decode, dim3(1), dim3(256), 0, stream, counters);
  return hipGetLastError();
}

}  // namespace kvx
