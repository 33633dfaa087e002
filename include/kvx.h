/*
 * kvx.h — C ABI of libkvx, the MI355X (gfx950) KV-block copy path.
 *
 * The library replaces the data movement of an offloaded paged KV cache:
 *   - the slot-mapped paged KV write (store_kvcache),
 *   - block save: gather of a pool block plus per-(token, KV-head) e4m3 FP8
 *     quantisation (or a byte copy in BF16 mode) into a host slab entry,
 *   - block restore: FP8 dequantisation (or byte copy) and scatter into a
 *     freed pool block,
 *   - a copy engine owning one save and one restore HIP stream whose events
 *     order save -> restore -> slot reuse against the caller's compute stream.
 *
 * Conventions
 *   - Every function returns 0 on success, a negative KVX_E_* code for a bad
 *     argument or state, or a positive hipError_t value for a HIP failure.
 *     kvx_last_error() returns the message of the calling thread's last error.
 *   - `stream` arguments are hipStream_t values passed as void*; NULL is the
 *     device's null stream. Queueing functions never synchronise the host.
 *   - Pointers named *_host are host memory read during the call only.
 *     Device pointers are borrowed for the lifetime of the queued work.
 *   - No torch types cross this boundary; PyTorch (or any other owner)
 *     allocates the pool, the staging buffers and the pinned host slabs.
 *
 * Citations name the reference interface each entry point replaces, in
 * xxdydx/KV-Cache-Offloading (paths relative to its repository root).
 */
#ifndef KVX_H
#define KVX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Version 2: kvx_upload and kvx_cache_dma_counters; allocation-free saves of
 * different caches on one device ordered by a per-device event; staging areas
 * replaced on a split-stream cache order both copy streams; waited one- and
 * two-block restores may run on the caller's stream; synchronize/destroy wait
 * for those; set_staging rejects overlapping split areas; KVX_DEBUG_* flags.
 */
#define KVX_ABI_VERSION 2

/* Error codes (negative); positive values are hipError_t. */
#define KVX_OK 0
#define KVX_E_INVALID (-1)  /* malformed argument (null pointer, bad size, bad layout) */
#define KVX_E_RANGE (-2)    /* block id / slot / size outside its valid range */
#define KVX_E_STATE (-3)    /* object in the wrong state (e.g. no staging attached) */
#define KVX_E_UNSUPPORTED (-4) /* valid request this build does not implement */

/* Scale element types of an FP8 entry. */
#define KVX_SCALE_BF16 0 /* nanovllm/engine/cpu_prefix_cache.py:205-206 (scale in the pool dtype) */
#define KVX_SCALE_FP32 1 /* one fp32 scale per (token, head) row */

/* Payload formats of a host entry. */
#define KVX_FORMAT_RAW 0 /* byte copy of the pool block (BF16 mode) */
#define KVX_FORMAT_FP8 1 /* e4m3fn payload + one scale per row */

/*
 * Geometry of a paged KV pool laid out [2, L, NB, BS, H, hd]
 * (nanovllm/engine/model_runner.py:120). A block is 2*L "planes" of BS*H rows
 * of hd elements; each plane of a block is contiguous in the pool.
 * The same descriptor also describes any tensor viewed as
 * [planes][plane_rows][head_dim] with a plane stride (use num_blocks = 1,
 * block_stride = 0 for a single view).
 */
typedef struct kvx_block_layout {
  int64_t plane_stride; /* elements between consecutive planes of one block (NB*BS*H*hd) */
  int64_t block_stride; /* elements between consecutive blocks in one plane (BS*H*hd) */
  int32_t planes;       /* planes per block (2*L) */
  int32_t plane_rows;   /* (token, head) rows per plane (BS*H) */
  int32_t head_dim;     /* elements per row (hd) */
  int32_t num_blocks;   /* blocks addressable through block_stride (NB) */
  int32_t elem_bytes;   /* pool element size in bytes (2 for bf16) */
  int32_t scale_dtype;  /* KVX_SCALE_* for FP8 entries */
} kvx_block_layout;

/*
 * Host/staging entry layout for one block: the payload (planes*plane_rows*hd
 * bytes for FP8, *elem_bytes for RAW) followed, for FP8, by the scales at
 * *scale_offset, one per row in plane-major order. *logical_bytes is the
 * payload+scale size the reference budgets per entry
 * (nanovllm/engine/cpu_prefix_cache.py:98-100); *entry_stride rounds it up to
 * 256 bytes so entries packed in a slab stay aligned.
 */
int kvx_entry_layout(const kvx_block_layout* layout, int32_t format, int64_t* logical_bytes,
                     int64_t* scale_offset, int64_t* entry_stride);

/* Message of the calling thread's last error ("" if none). */
const char* kvx_last_error(void);
/* KVX_ABI_VERSION of the loaded library. */
int kvx_abi_version(void);

/*
 * Slot-mapped paged KV write. Replaces store_kvcache + store_kvcache_kernel
 * (nanovllm/layers/attention.py:10-40). For each token i with
 * s = slot_mapping[i] in [0, cache_slots): copies num_heads*head_dim elements
 * of key row i (key + i*key_stride elements) to k_cache + s*D, and the same
 * for value/v_cache. s == -1 (CUDA-graph padding, model_runner.py:211) and
 * any other out-of-range slot write nothing. slot_mapping is a device array
 * of num_tokens int32. Strides are in elements. Graph-capturable.
 */
int kvx_store_kvcache(const void* key, int64_t key_stride, const void* value, int64_t value_stride,
                      void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t num_tokens,
                      int32_t num_heads, int32_t head_dim, int32_t elem_bytes, int64_t cache_slots,
                      void* stream);

/*
 * Save n pool blocks into entries. Replaces save_block's copy
 * (nanovllm/engine/cpu_prefix_cache.py:315-319): FP8 format runs
 * fp8_quantize (:20-24) on pool[:, :, block] via _quantize (:225-234);
 * RAW format is payload.copy_(pool[:, :, block]) (:319).
 * block_ids_host[i] selects the pool block; entries_host[i] is the
 * device-accessible byte address of entry i (device staging or mapped
 * pinned host memory). For FP8 the scales of entry i are at
 * entries_host[i] + scale_offset (may be negative). n may exceed the
 * per-launch batch; the call splits it. No two payload or scale ranges may
 * overlap (KVX_E_INVALID).
 */
int kvx_save_blocks(const void* pool, const kvx_block_layout* layout, int32_t format,
                    const int32_t* block_ids_host, const uint64_t* entries_host, int32_t n,
                    int64_t scale_offset, void* stream);

/*
 * Restore n entries into pool blocks. Replaces _copy_entry's copy
 * (nanovllm/engine/cpu_prefix_cache.py:383-386): FP8 format runs
 * fp8_dequantize (:27-28) via _dequantize (:236-243) into pool[:, :, block];
 * RAW format is target.copy_(entry.kv) (:386). Arguments as kvx_save_blocks;
 * a block may appear only once per call (KVX_E_INVALID).
 */
int kvx_restore_blocks(void* pool, const kvx_block_layout* layout, int32_t format,
                       const int32_t* block_ids_host, const uint64_t* entries_host, int32_t n,
                       int64_t scale_offset, void* stream);

/*
 * Token-granular KV handoff copies (nanovllm/engine/kv_handoff.py). A
 * sequence's first num_rows (token, head) rows live in the pool blocks
 * block_table_host[0..]; the dense buffer holds them as
 * [planes][num_rows][head_dim] (the reference's [2, L, tokens, H, hd] payload,
 * num_rows = tokens * H). Byte copies; any element size in `layout`.
 * kvx_gather_tokens replaces export_kv's index_select + contiguous
 * (:46-55); kvx_scatter_tokens replaces import_kv's per-block copy_
 * (:112-118). The buffer may be device memory or mapped pinned host memory.
 * A scatter's table may not name a block twice (KVX_E_INVALID). To copy only
 * planes [first, end), pass pool + first * plane_stride * elem_bytes and a
 * layout with planes = end - first; the buffer then holds those planes.
 */
int kvx_gather_tokens(const void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                      int32_t table_len, int64_t num_rows, void* dst, void* stream);
int kvx_scatter_tokens(void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                       int32_t table_len, int64_t num_rows, const void* src, void* stream);

/*
 * FP8 KV handoff: the token copies above with the FP8 codec. A sequence's
 * first num_rows rows of the blocks block_table_host[0..] correspond to a
 * dense e4m3 payload [planes][num_rows][head_dim] and a dense scale array
 * [planes][num_rows] of layout->scale_dtype. kvx_gather_tokens_fp8 writes
 * them with fp8_quantize's arithmetic (nanovllm/engine/cpu_prefix_cache.py:
 * 20-24), i.e. what fp8_quantize gives for export_kv's BF16 payload
 * (nanovllm/engine/kv_handoff.py:46-55), at half its bytes on the wire;
 * kvx_scatter_tokens_fp8 dequantises them into the blocks (:27-28), in place
 * of import_kv's per-block copy (kv_handoff.py:112-118). Payload and scales
 * may be device memory or, for the gather, pinned host memory; they may not
 * overlap; a scatter's table may not name a block twice (KVX_E_INVALID).
 */
int kvx_gather_tokens_fp8(const void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                          int32_t table_len, int64_t num_rows, void* payload, void* scales, void* stream);
int kvx_scatter_tokens_fp8(void* pool, const kvx_block_layout* layout, const int32_t* block_table_host,
                           int32_t table_len, int64_t num_rows, const void* payload, const void* scales,
                           void* stream);

/*
 * Copy engine: the stream/event half of CPUBlockCache
 * (nanovllm/engine/cpu_prefix_cache.py:72-131, 270-273, 306-322, 352-363,
 * 370-398). It queues copies on a save stream and a restore stream that the
 * caller creates and keeps alive (the reference uses torch.cuda.Stream,
 * :110-113; pass the same stream twice for split_streams=False) and keeps
 * per GPU block / host slot events. Host slabs and device staging are
 * owned by the caller too; the engine never frees or destroys them.
 */
typedef struct kvx_cache kvx_cache;

/* Creates an engine for `pool` on `device` using the caller's two streams (non-NULL). */
int kvx_cache_create(void* pool, const kvx_block_layout* layout, int32_t format, void* save_stream,
                     void* restore_stream, int32_t device, kvx_cache** out);
/* Synchronises both streams and the restores queued on callers' streams, then frees the engine's events
 * (:431-448). */
int kvx_cache_destroy(kvx_cache* cache);
/*
 * Attaches one device staging area per stream, each holding `entries`
 * entries of kvx_entry_layout's entry_stride (per-stream staging, :217-223).
 * Pass the same pointer twice when split_streams == 0; with split streams the
 * two areas may not overlap (KVX_E_INVALID). Copies already queued keep
 * using the previous areas, which must stay allocated until they complete.
 * When a split-stream cache's areas change, each copy stream first waits for
 * the work already queued on the other, so a previous area may become the
 * other stream's new one without a race.
 */
int kvx_cache_set_staging(kvx_cache* cache, void* save_staging, void* restore_staging,
                          int32_t entries);
/*
 * Appends `count` host slots at host_base (pinned, device-accessible),
 * entry_stride apart, as slots [num_slots, num_slots + count) (_grow, :199-208).
 */
int kvx_cache_add_slab(kvx_cache* cache, void* host_base, int32_t count);
/* Drops all slabs and per-slot events after synchronising (close, :431-448). */
int kvx_cache_reset_slabs(kvx_cache* cache);
/* The save and restore streams the engine was created with (equal without split streams). */
int kvx_cache_streams(kvx_cache* cache, void** save_stream, void** restore_stream);

/*
 * Saves pool blocks block_ids_host[i] into host slots slots_host[i]
 * (save_block, :306-322). The save stream first waits for all work queued
 * on compute_stream, for the last restore that read each slot and for any
 * background restore still writing each block; a "save done" event then
 * marks each block (for before_block_reuse) and each slot (for a later
 * restore of it). Calls of one or two blocks issued while compute_stream
 * still has work queued have the save kernel write the slots itself; other
 * calls go through device staging and a copy.
 * Slabs must be pinned, device-accessible host memory (hipHostMalloc).
 * A slot may appear only once per call (KVX_E_INVALID).
 */
int kvx_cache_save(kvx_cache* cache, const int32_t* block_ids_host, const int32_t* slots_host,
                   int32_t n, void* compute_stream);

/* Bytes of the static device staging behind kvx_cache_save_noalloc, one array per device. */
#define KVX_NOALLOC_SCRATCH_BYTES (64LL << 20)

/*
 * kvx_cache_save without attached staging and without allocation. It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * (serving loops and harnesses that forbid hipMalloc, or processes whose
 * device memory all belongs to the KV pool). Results and errors are those
 * of kvx_cache_save, and so are its ordering rules, except that it records a
 * single event after its copies to host memory: a restore into a block it
 * saved waits for those copies, not only for the save kernel. Entries are
 * staged in a static array of KVX_NOALLOC_SCRATCH_BYTES that the library
 * holds on each device until the process ends, and the call creates no
 * events and allocates no host or device memory. n may not exceed the entries that array holds,
 * min(128, KVX_NOALLOC_SCRATCH_BYTES / entry_stride) (three Qwen3-8B FP8
 * entries); a larger n fails with KVX_E_RANGE before any work is queued.
 * Every such call on one device shares its array. Calls are ordered by one
 * event per device, created with the device's first cache: each call's save
 * stream waits for the previous call's copies out of the array, whichever
 * cache made it, and the calls are issued one at a time (a per-device
 * mutex). Calls of different caches therefore follow each other on the
 * device in the order they were made.
 */
int kvx_cache_save_noalloc(kvx_cache* cache, const int32_t* block_ids_host, const int32_t* slots_host,
                           int32_t n, void* compute_stream);
/*
 * Restores host slots slots_host[i] into pool blocks block_ids_host[i]
 * (_copy_entry, :370-398). The restore stream waits for compute_stream, for
 * each slot's save, and for any pending save of each destination block (the
 * write-after-read order the reference leaves to its callers). With
 * wait != 0 compute_stream waits for the restore; otherwise the block is
 * marked pending until before_block_use/before_block_reuse. A block may
 * appear only once per call (KVX_E_INVALID). Calls of one or two blocks with
 * wait != 0, issued while no save is in flight, have the restore kernel read
 * the slots itself (a capped grid, system-scope loads), queued on
 * compute_stream, which waits for them anyway; such a restore also waits
 * for a pending restore (wait == 0) still writing one of its blocks, which
 * the restore stream's order gives the others (a prefetched block recycled
 * before its first use). Others are staged in device memory by an H2D copy
 * first, on the restore stream.
 */
int kvx_cache_restore(kvx_cache* cache, const int32_t* slots_host, const int32_t* block_ids_host,
                      int32_t n, int32_t wait, void* compute_stream);
/* Orders later writes of block_id on compute_stream after its pending save and restore (:352-357). */
int kvx_cache_before_block_reuse(kvx_cache* cache, int32_t block_id, void* compute_stream);
/* Orders later reads of block_id on compute_stream after its pending restore (:359-363). */
int kvx_cache_before_block_use(kvx_cache* cache, int32_t block_id, void* compute_stream);
/* Blocks the host until both streams are idle and every restore queued on a caller's stream has completed
 * (synchronize, :270-273). */
int kvx_cache_synchronize(kvx_cache* cache);
/* Counts of engine activity: saves, restores, waits inserted; for tests and stats. */
int kvx_cache_counters(kvx_cache* cache, int64_t* saved_blocks, int64_t* restored_blocks,
                       int64_t* stream_waits);
/*
 * DMA transfers the engine has queued (hipMemcpyAsync calls, each at most
 * 64 MiB) and their bytes, per direction. Saves and restores that the kernels
 * move over the host link themselves queue none. A memory-copy trace of the
 * engine's work holds exactly these copies; comparing the counts shows
 * whether the tracer lost records. No reference counterpart (the reference's
 * copies are torch copy_ calls).
 */
int kvx_cache_dma_counters(kvx_cache* cache, int64_t* d2h_copies, int64_t* d2h_bytes, int64_t* h2d_copies,
                           int64_t* h2d_bytes);

/*
 * Negative controls (tests only): each flag drops one ordering rule so a test
 * can show that its check fails without it (the reference claims such controls,
 * README.md:114-117, but commits none). Flags:
 *   KVX_DEBUG_SKIP_SAVE_WAIT       a restore does not wait for its slot's save
 *   KVX_DEBUG_SKIP_SLOT_READ_WAIT  a save does not wait for restores reading its slot
 *   KVX_DEBUG_SKIP_REUSE_WAIT      before_block_reuse does not wait for the block's save
 *   KVX_DEBUG_SKIP_VICTIM_WAIT     a restore does not wait for a pending save of its destination
 *   KVX_DEBUG_SKIP_OVERWRITE_WAIT  a restore on compute_stream does not wait for a pending restore
 *                                  of its destination
 * Results are wrong (never a fault) while a flag is set; 0 restores normal operation.
 */
#define KVX_DEBUG_SKIP_SAVE_WAIT 1
#define KVX_DEBUG_SKIP_SLOT_READ_WAIT 2
#define KVX_DEBUG_SKIP_REUSE_WAIT 4
#define KVX_DEBUG_SKIP_VICTIM_WAIT 8
#define KVX_DEBUG_SKIP_OVERWRITE_WAIT 16
int kvx_cache_set_debug(kvx_cache* cache, int32_t flags);

/* Largest kvx_upload. */
#define KVX_UPLOAD_MAX_BYTES (1LL << 30)

/*
 * Copies nbytes from pinned, device-accessible host memory (hipHostMalloc;
 * torch's pin_memory) to device memory by a kernel queued on `stream`, in
 * place of the pinned non-blocking host-to-device copies of a step's inputs
 * (token ids, positions, slot_mapping: nanovllm/engine/model_runner.py:
 * 169-173, 187-190). A DMA copy queued there waits behind every
 * host-to-device DMA already queued on the device, a restore stream's bulk
 * copies included; the kernel does not. The source is read when the kernel
 * runs: it must stay allocated and unchanged until then. Both ends of
 * [src_pinned, src_pinned + nbytes) must lie in one pinned host allocation
 * (KVX_E_INVALID otherwise) and nbytes may not exceed KVX_UPLOAD_MAX_BYTES
 * (KVX_E_RANGE). Graph-capturable.
 */
int kvx_upload(void* dst, const void* src_pinned, int64_t nbytes, void* stream);

/*
 * Queues a kernel that keeps one wave busy for `microseconds` on `stream`
 * (the injected delay of bench/test_automatic_cpu_cache.py:47-48, which
 * uses torch.cuda._sleep). The wait is bounded by the device wall clock.
 */
int kvx_sleep(void* stream, int64_t microseconds);

/*
 * Exhaustive device self-test of the arithmetic the FP8 kernels rely on.
 * Writes 8 uint64 counters to the device array `counters` (zeroed by the
 * call): [0] e4m3 hardware vs software encode mismatches over every fp32
 * bit pattern (after the kernels' clamp), [1] bf16 hardware vs software RNE
 * mismatches over every non-NaN fp32, [2] NaN inputs not encoded as NaN,
 * [3] reciprocal-FMA vs IEEE division mismatches over every (bf16
 * significand, fp32 significand) pair, [4] e4m3 decode mismatches over the
 * 256 codes, [5..7] inputs checked by the three sweeps / 2^20.
 */
int kvx_selftest(uint64_t* counters, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVX_H */
