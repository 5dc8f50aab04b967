/*
 * vapi_kv.h — C ABI of the MI355X (gfx950) paged KV-cache library.
 *
 * This is the drop-in boundary for vapi's paged KV hot path: the KV append
 * (slot_mapping scatter), the block-table gather, paged attention (decode and
 * chunked prefill in one varlen call), the copy-on-write block copy and the
 * spill-tier export/import/swap. Every entry point:
 *   - is `extern "C"` with plain pointers, sizes and a hipStream_t;
 *   - returns 0 on success and a negative VAPI_KV_E* code on error, with a
 *     thread-local message in vapi_kv_last_error();
 *   - never allocates device or host memory (the "vapi_cache_*" host object
 *     at the bottom of this file is the exception: it owns the pool, like the
 *     reference's PagedKvCache);
 *   - takes every device argument by value/pointer, so a call can be recorded
 *     into a HIP graph.
 *
 * Reference interfaces replaced (paths relative to the vapi repository):
 *   crates/vapi-backend-candle/src/cache.rs:12-118   PagedKvCache
 *   crates/vapi-backend-candle/src/cache.rs:136-278  write_kv_to_cache/write_rows
 *   crates/vapi-backend-candle/src/rows.rs:22-33     rows::scatter (CUDA append)
 *   crates/vapi-backend-candle/src/cache.rs:283-290  gather_kv
 *   crates/vapi-backend-candle/src/attention.rs:42-71,170-288 paged attention
 *   crates/vapi-backend-candle/src/backend.rs:695-797 block_bytes/export/import/copy
 *   crates/vapi-engine/src/backend.rs:96-204          ForwardBatch::validate
 */
#ifndef VAPI_KV_H
#define VAPI_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* vapi_stream_t;

/* ---- status codes ------------------------------------------------------ */
#define VAPI_KV_OK 0
#define VAPI_KV_EINVAL (-1)   /* bad argument, shape, dtype or range */
#define VAPI_KV_EUNSUP (-2)   /* valid but unsupported configuration */
#define VAPI_KV_EHIP (-3)     /* a HIP runtime call failed */
#define VAPI_KV_ESPACE (-4)   /* a caller-provided buffer is too small */

/* ---- pool description -------------------------------------------------- */
typedef enum {
  VAPI_KV_F32 = 0,
  VAPI_KV_F16 = 1,
  VAPI_KV_BF16 = 2
} vapi_kv_dtype;

typedef enum {
  /* [num_blocks, num_kv_heads, block_size, head_dim]: each (block, head) is
   * one contiguous block_size*head_dim tile. The default on MI355X. */
  VAPI_KV_LAYOUT_HND = 0,
  /* [num_blocks, block_size, num_kv_heads, head_dim]: the reference's own
   * layout (cache.rs:7-11), for byte-for-byte interchange. */
  VAPI_KV_LAYOUT_NHD = 1
} vapi_kv_layout;

/* A padded token in slot_mapping: written nowhere (vLLM's -1 as u32). */
#define VAPI_KV_SLOT_SKIP 0xFFFFFFFFu

/*
 * One paged K/V pool for `num_layers` layers. Layer l's K buffer starts at
 * (char*)k + l*layer_stride_bytes and its V buffer at (char*)v +
 * l*layer_stride_bytes; each is num_blocks blocks in `layout`. A slot is
 * block*block_size + offset, the addressing of ForwardBatch::slot_mapping
 * (crates/vapi-engine/src/backend.rs:62-64).
 *
 * k and v must be 16-byte aligned and layer_stride_bytes a multiple of 16
 * (the kernels move 16-byte chunks; vapi_cache_new and the Python cache pad
 * layers to 256 bytes); anything else is VAPI_KV_EINVAL.
 *
 * v == NULL makes a K-only pool: LayerLayout::Rows layers (cache.rs:24-33,
 * 89-96), one (1, width) row per token, num_kv_heads 1 and head_dim width.
 * Appends and gathers then move K only; attention rejects the pool.
 *
 * block_stride_bytes: 0 packs a layer buffer's blocks densely (block b at
 * b * block_size * num_kv_heads * head_dim elements, as above). Nonzero
 * places block b of every layer buffer at b * block_stride_bytes from that
 * buffer's base instead: a block-major pool, where one allocation holds,
 * per block, every layer's K and V block side by side (layer_stride_bytes
 * then the distance between two layers' blocks within it, at least one
 * block's bytes, and block_stride_bytes at least (num_layers - 1) *
 * layer_stride_bytes plus one block's bytes; both multiples of 16). A
 * copy-on-write pair and an exported blob are then one contiguous run;
 * every call accepts either form.
 *
 * next chains further pools of the same cache (same num_blocks and
 * block_size; any geometry, dtype, layout, with or without V), in layer
 * order: a cache whose layers differ (PagedKvCache::with_layouts,
 * cache.rs:71-105) is one pool per run of alike layers. Block-level calls
 * (block_bytes, copy_blocks, export/import, swap, the spill tier) walk the
 * chain; per-layer calls (append, gather, attention) use the pool they are
 * given and ignore next. NULL ends the chain.
 */
typedef struct vapi_kv_pool {
  void* k;
  void* v;
  uint64_t layer_stride_bytes;
  uint32_t num_layers;
  uint32_t num_blocks;
  uint32_t block_size;
  uint32_t num_kv_heads;
  uint32_t head_dim;
  uint32_t dtype;  /* vapi_kv_dtype */
  uint32_t layout; /* vapi_kv_layout */
  const struct vapi_kv_pool* next; /* the next pool of the same cache, or NULL */
  uint64_t block_stride_bytes;       /* 0: dense blocks; else the block stride */
} vapi_kv_pool;

/* Thread-local message for the last failing call on this thread ("" if none). */
const char* vapi_kv_last_error(void);

/* Library version string. */
const char* vapi_kv_version(void);

/* Bytes of one block across every layer, K then V (backend.rs:695-708):
 * num_layers * 2 * block_size * num_kv_heads * head_dim * sizeof(dtype)
 * (1 instead of 2 for a K-only pool), summed over the pool chain. */
size_t vapi_kv_block_bytes(const vapi_kv_pool* pool);

/* Bytes of one layer's K (or V) buffer: num_blocks * block elements. */
size_t vapi_kv_layer_bytes(const vapi_kv_pool* pool);

/*
 * KV append (reshape_and_cache). Replaces write_kv_to_cache/write_rows
 * (cache.rs:136-148, 217-273) and the CUDA rows::scatter kernel
 * (rows.rs:22-33, 60-72; call site models/qwen.rs:372-382).
 *
 * k_src, v_src: device [n_tokens, num_kv_heads, head_dim] in pool dtype.
 * slot_mapping: device u32[n_tokens]; token i lands in flat slot
 * slot_mapping[i]. VAPI_KV_SLOT_SKIP skips the token. A slot past the end of
 * the pool is never written (the device guard drops it); the host-side
 * vapi_cache_write_kv() reports it as an error as the reference does.
 * Duplicate slots are undefined (ForwardBatch::validate rejects them).
 * K and V are written in one launch.
 */
int vapi_kv_append(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                   const void* v_src, const uint32_t* slot_mapping,
                   uint32_t n_tokens, vapi_stream_t stream);

/*
 * vapi_kv_append with flags. VAPI_APPEND_COLD_SOURCE: the source rows are
 * not expected in the GPU's caches (rows read back from host memory or
 * written long before, not just produced by a projection kernel), so they
 * are read with streaming (non-temporal) loads that do not allocate in the
 * last-level cache; a warm source is read slower that way. Same result
 * either way. No counterpart flag in the reference (write_kv_to_cache,
 * cache.rs:136-148, has one path).
 */
#define VAPI_APPEND_COLD_SOURCE 1u
int vapi_kv_append_ex(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                      const void* v_src, const uint32_t* slot_mapping, uint32_t n_tokens,
                      uint32_t flags, vapi_stream_t stream);

/*
 * The same append over layers layer0 .. layer0 + n_layers - 1 in one launch
 * (one slot_mapping for all of them): layer l's rows are at k_src/v_src +
 * (l - layer0) * src_layer_stride bytes, each [n_tokens, num_kv_heads,
 * head_dim]. Equals n_layers vapi_kv_append calls. No counterpart call in
 * the reference, which writes each layer inside its forward
 * (models/qwen.rs:371-387); it is the multi-layer write of a step whose K/V
 * are all at hand, e.g. a restored prefix.
 */
int vapi_kv_append_layers(const vapi_kv_pool* pool, uint32_t layer0, uint32_t n_layers,
                          const void* k_src, const void* v_src, uint64_t src_layer_stride,
                          const uint32_t* slot_mapping, uint32_t n_tokens,
                          vapi_stream_t stream);

/*
 * Block-table gather into logical order. Replaces gather_kv (cache.rs:283-290).
 * block_table: device u32[n_table]; out: device [len_k, num_kv_heads,
 * head_dim] for K and for V (either may be NULL; V must be NULL for a
 * K-only pool). len_k <= n_table*block_size. Rows of a table entry past the
 * pool are gathered as zeros.
 */
int vapi_kv_gather(const vapi_kv_pool* pool, uint32_t layer,
                   const uint32_t* block_table, uint32_t n_table,
                   uint32_t len_k, void* k_out, void* v_out,
                   vapi_stream_t stream);

/*
 * Paged attention over a varlen batch: decode rows (len_q == 1) and prefill
 * chunks (len_q > 1) in one call, dispatched inside. Replaces
 * paged_attention_cuda/_windowed/_prepared (attention.rs:170-288) with
 * paged_attention_cpu (attention.rs:90-163) as the numerical contract.
 *
 * q:   device [cu_seqlens_q[batch], num_heads, head_dim], pool dtype.
 * out: device, same shape and dtype as q. q and out must be 16-byte aligned
 *   (the kernels move 16-byte chunks of their rows); VAPI_KV_EINVAL otherwise.
 * cu_seqlens_q, cu_seqlens_k: device u32[batch+1]; len_k includes the cached
 *   prefix and len_q <= len_k. Query j of a sequence sits at absolute
 *   position p = len_k - len_q + j (bottom-right aligned).
 * block_table: device u32[batch, max_blocks] (pack_block_tables layout,
 *   attention.rs:42-62). Entries past the pool are clamped to its last block,
 *   and keys past a row's max_blocks * block_size read the row's last entry
 *   (no fault); ForwardBatch::validate is where bad batches are refused.
 * max_seqlen_q, max_seqlen_k: upper bounds of len_q and len_k.
 * window_left: keys k < p - window_left are hidden; -1 = unlimited. A sliding
 *   window of w (HF q - k < w) is window_left = w - 1 (attention.rs:179-194).
 * window_right: keys k > p + window_right are hidden; 0 = causal, -1 =
 *   unlimited (bidirectional).
 * workspace: device scratch of at least vapi_paged_attention_workspace_size()
 *   bytes (the decode's per-XCD work shares, per-segment ranges and
 *   split-context partials); may be NULL when that size is 0. Zero-fill it once before its
 *   first use. Keep one workspace per stream across calls and layers: each
 *   call measures how fast each XCD streamed and moves the shares the next
 *   call on that workspace uses (a fresh workspace starts from equal
 *   shares). Results do not depend on the shares beyond f32 rounding of the
 *   split merge. Calls sharing one workspace must not overlap (same stream,
 *   or ordered streams).
 * max_seqlen_q/k must bound every sequence's len_q/len_k (as in
 *   flash-attention); max_seqlen_q sizes the prefill grid. On the MFMA path
 *   (bf16/f16, head_dim 64, 128 or 256, or any other multiple of 8 below 256,
 *   run at the next of them with the extra elements read as zeros) the decode's part depends on the batch,
 *   the heads and the GPU's CU count, not on the lengths; a prefill batch
 *   with fewer query tiles than the GPU has CUs asks for more (up to 256
 *   MiB) to split its keys over more workgroups. That part is optional: a
 *   workspace holding only the decode's part (or none, for a call with
 *   VAPI_ATTN_NO_DECODE_ROWS) runs the prefill unsplit, and a
 *   VAPI_ATTN_DETERMINISTIC call never splits. An f32 pool with head_dim
 *   64 or 128, or another multiple of 4 below 128 run at the next of them,
 *   runs the decode stream and an f32 prefill kernel, sized the
 *   same way (the f32 prefill's key split is the optional part; a
 *   pure-decode f32 call over at
 *   most 512 keys per sequence and 8,192 in all runs the VALU kernel). On
 *   the VALU path (those small calls, other head dims, groups of more than 256
 *   query heads per kv head, block sizes below 16) it holds the split-context partials and
 *   grows with the batch, max_seqlen_q and max_seqlen_k (0 while
 *   max_seqlen_k <= 64; small batches split their keys into chunks of 64
 *   to 512 keys to fill the GPU).
 */
size_t vapi_paged_attention_workspace_size(const vapi_kv_pool* pool,
                                           uint32_t batch, uint32_t num_heads,
                                           uint32_t max_seqlen_q,
                                           uint32_t max_seqlen_k);

int vapi_paged_attention(const vapi_kv_pool* pool, uint32_t layer,
                         const void* q, void* out,
                         const uint32_t* cu_seqlens_q,
                         const uint32_t* cu_seqlens_k,
                         const uint32_t* block_table, uint32_t batch,
                         uint32_t max_blocks, uint32_t max_seqlen_q,
                         uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                         int32_t window_left, int32_t window_right,
                         void* workspace, size_t workspace_bytes,
                         vapi_stream_t stream);

/*
 * vapi_paged_attention with flags (0 = vapi_paged_attention itself). No
 * counterpart in the reference, whose flash call takes no such options
 * (attention.rs:272-287); they are host knowledge a caller can pass on:
 *
 * VAPI_ATTN_NO_DECODE_ROWS: the caller knows no row has len_q == 1 (a
 *   prefill-only step; PreparedAttention knows it from its host
 *   cu_seqlens). The call then launches the prefill kernel alone, which
 *   takes every row, so a wrong hint costs time, never correctness. Such a
 *   call needs no workspace (workspace may be NULL, workspace_bytes 0).
 * VAPI_ATTN_DETERMINISTIC: the decode splits its work with fixed equal
 *   per-XCD shares instead of the shares the previous call measured, and
 *   does not update them: two calls on identical inputs give bit-identical
 *   outputs, whatever ran on the workspace before. Costs the XCD balancing
 *   (a few percent of decode time).
 * Unknown flag bits are VAPI_KV_EINVAL.
 */
#define VAPI_ATTN_DETERMINISTIC 0x1u
#define VAPI_ATTN_NO_DECODE_ROWS 0x2u
int vapi_paged_attention_ex(const vapi_kv_pool* pool, uint32_t layer, const void* q, void* out,
                            const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                            const uint32_t* block_table, uint32_t batch, uint32_t max_blocks,
                            uint32_t max_seqlen_q, uint32_t max_seqlen_k, uint32_t num_heads,
                            float scale, int32_t window_left, int32_t window_right,
                            uint32_t flags, void* workspace, size_t workspace_bytes,
                            vapi_stream_t stream);

/*
 * vapi_paged_attention_ex with the step's prefill sequences named by the
 * host: prefill_seqs = device u32[n_prefill], the indices of every sequence
 * with len_q > 1, in ascending order. It mirrors paged_attention_cuda_prepared
 * (attention.rs:262-288), whose PreparedAttention the host builds once per
 * step from the batch (attention.rs:234-256); the list is one more array of
 * that kind. The prefill grid then covers those sequences only, and its key
 * split is chosen for them: a chunked-prefill step of many decode rows and
 * one prefill chunk runs that chunk over the whole GPU instead of one
 * workgroup per query tile and kv head. A sequence with len_q > 1 missing
 * from the list gets no output rows; the list is trusted like the block
 * table. With VAPI_ATTN_NO_DECODE_ROWS the call covers every sequence and
 * ignores the list. Same workspace contract as vapi_paged_attention, sized
 * by vapi_paged_attention_prepared_workspace_size (the prefill's optional
 * key-split part is sized for n_prefill sequences). n_prefill > batch, or a
 * null list with n_prefill > 0, is VAPI_KV_EINVAL.
 */
size_t vapi_paged_attention_prepared_workspace_size(const vapi_kv_pool* pool, uint32_t batch,
                                                    uint32_t n_prefill, uint32_t num_heads,
                                                    uint32_t max_seqlen_q,
                                                    uint32_t max_seqlen_k);
int vapi_paged_attention_prepared(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                  void* out, const uint32_t* cu_seqlens_q,
                                  const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                  uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                  uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                  int32_t window_left, int32_t window_right, uint32_t flags,
                                  const uint32_t* prefill_seqs, uint32_t n_prefill,
                                  void* workspace, size_t workspace_bytes,
                                  vapi_stream_t stream);

/*
 * vapi_paged_attention_ex without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The decode workspace is the library's own device array of
 * VAPI_ATTN_SCRATCH_BYTES bytes, one per GPU, held until the process ends;
 * the call allocates nothing. A batch whose workspace
 * (vapi_paged_attention_workspace_size) exceeds it is refused with
 * VAPI_KV_ESPACE before anything is launched. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams not
 * ordered against each other) race and must not be issued. The first call
 * on a device resolves the array's address; the first call not under HIP
 * graph capture clears its XCD shares with a small kernel on `stream` (a
 * captured call records no clear, so replays keep the shares); later calls
 * carry the shares over, as a kept workspace does. The array is reserved in
 * every process that loads the library, whether it calls this or not.
 */
#define VAPI_ATTN_SCRATCH_BYTES (16u << 20)
int vapi_paged_attention_noalloc(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                 void* out, const uint32_t* cu_seqlens_q,
                                 const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                 uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                 uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                 int32_t window_left, int32_t window_right, uint32_t flags,
                                 vapi_stream_t stream);

/*
 * One decode step's K/V append and paged attention in one call: the result
 * is that of vapi_kv_append(k_src, v_src, slot_mapping, n_tokens) followed
 * by vapi_paged_attention(...) with the same arguments. It fuses the
 * per-layer pair the reference issues in every model forward (the cache
 * write, then the attention: models/qwen.rs:371-391, models/llama.rs:157-165).
 *
 * When every row is a decode row (max_seqlen_q == 1) on the MFMA path
 * (bf16/f16, head_dim 64, 128 or 256), it takes one launch fewer: the attention
 * reads the new key of row s (position len_k - 1) straight from token
 * cu_seqlens_q[s] of k_src/v_src, provided slot_mapping sends that token to
 * the slot the row's block table gives position len_k - 1 (checked per row
 * on the device; a row that fails the check reads the pool, as the two-call
 * sequence would), and the pool writes of all n_tokens tokens complete
 * within the call. The fused path also requires that no row reads a slot
 * this call writes other than its own new key at len_k - 1, which holds for
 * the scheduler's slot mapping (scheduler.rs:525-565). Every other shape
 * runs the two calls. Same workspace contract as vapi_paged_attention.
 */
int vapi_paged_attention_append(const vapi_kv_pool* pool, uint32_t layer,
                                const void* k_src, const void* v_src,
                                const uint32_t* slot_mapping, uint32_t n_tokens,
                                const void* q, void* out,
                                const uint32_t* cu_seqlens_q,
                                const uint32_t* cu_seqlens_k,
                                const uint32_t* block_table, uint32_t batch,
                                uint32_t max_blocks, uint32_t max_seqlen_q,
                                uint32_t max_seqlen_k, uint32_t num_heads,
                                float scale, int32_t window_left,
                                int32_t window_right, void* workspace,
                                size_t workspace_bytes, vapi_stream_t stream);

/* vapi_paged_attention_append with the flags of vapi_paged_attention_ex
 * (VAPI_ATTN_NO_DECODE_ROWS has no effect on a fused decode step). */
int vapi_paged_attention_append_ex(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                                   const void* v_src, const uint32_t* slot_mapping,
                                   uint32_t n_tokens, const void* q, void* out,
                                   const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                                   const uint32_t* block_table, uint32_t batch,
                                   uint32_t max_blocks, uint32_t max_seqlen_q,
                                   uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                   int32_t window_left, int32_t window_right, uint32_t flags,
                                   void* workspace, size_t workspace_bytes,
                                   vapi_stream_t stream);

/*
 * Copy-on-write block copy over every layer, K and V, in one launch (one
 * per chained pool; a K-only pool copies K).
 * Replaces CandleBackend::copy_blocks (backend.rs:781-797), which the
 * engine calls with Scheduler::fork's pairs (scheduler.rs:217-281).
 * pairs: device u32[n_pairs][2] = (src, dst). A dst must not also be a src
 * or another pair's dst in the same call. A pair naming a block past the
 * pool is skipped (device ids are not checked on the host).
 */
int vapi_kv_copy_blocks(const vapi_kv_pool* pool, const uint32_t* pairs,
                        uint32_t n_pairs, vapi_stream_t stream);

/*
 * Spill export / import. Block i's blob (vapi_kv_block_bytes bytes) is the
 * reference's byte order (backend.rs:718-734, 738-773): K of layers
 * 0..L-1, then V of layers 0..L-1, each [block_size, num_kv_heads, head_dim]
 * in native little-endian element bytes, whatever the pool layout. Over a
 * pool chain the layers are those of every pool in order, and K-only
 * pools contribute no V segments (rank-1 V buffers are skipped there).
 * ids: device u32[n]; an id past the pool moves nothing (its blob is left
 * as it was). dst/src: n blobs back to back; device memory or host-mapped
 * pinned memory (hipHostMalloc), either is read/written directly by the
 * kernel.
 */
int vapi_kv_export_blocks(const vapi_kv_pool* pool, const uint32_t* ids,
                          uint32_t n, void* dst, vapi_stream_t stream);
int vapi_kv_import_blocks(const vapi_kv_pool* pool, const uint32_t* ids,
                          uint32_t n, const void* src, vapi_stream_t stream);

/*
 * Swap between HBM and pinned host memory through a device staging buffer:
 * swap_out packs blocks into staging and hipMemcpyAsync's them device→host;
 * swap_in copies host→staging and unpacks. Work is chunked to fit
 * staging_bytes (at least one block). All work is enqueued on `stream`
 * (typically a side stream, so a decode launch on another stream overlaps
 * the DMA). host buffers: n * vapi_kv_block_bytes bytes, pinned.
 */
int vapi_kv_swap_out(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n,
                     void* host_dst, void* staging, size_t staging_bytes,
                     vapi_stream_t stream);
int vapi_kv_swap_in(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n,
                    const void* host_src, void* staging, size_t staging_bytes,
                    vapi_stream_t stream);

/*
 * Spill store: exported blocks kept in host memory, with an optional disk
 * tier behind it, both least-recently-used. Replaces SpillStore
 * (crates/vapi-cache/src/spill.rs:43-212) with the same behaviour: put()
 * ignores a hash already held and drops a blob that fits neither tier;
 * host memory over its cap pushes its oldest entries to disk (or drops
 * them without a disk tier); a disk hit is not promoted back into memory;
 * a disk entry that cannot be read is forgotten and counted as an error.
 * Keys are 32-byte block hashes; disk entries are "<64 hex>.kv" files of
 * the export byte order, indexed again when a store opens the directory.
 * The store is host-only and not thread-safe (one engine thread).
 */
typedef struct vapi_spill_store vapi_spill_store;
typedef struct vapi_spill_stats {
  uint64_t ram_blocks, ram_bytes, disk_blocks, disk_bytes;
  uint64_t hits;   /* blocks handed back */
  uint64_t misses; /* blocks asked for and not held */
  uint64_t writes;
  uint64_t drops;  /* blocks dropped because both tiers were full */
  uint64_t errors;
} vapi_spill_stats;

/* dir = NULL (or disk_max = 0): host memory only. Allocates the store. */
int vapi_spill_open(const char* dir, uint64_t ram_max, uint64_t disk_max,
                    vapi_spill_store** out);
void vapi_spill_close(vapi_spill_store* store);
int vapi_spill_contains(const vapi_spill_store* store, const uint8_t* hash32);
int vapi_spill_put(vapi_spill_store* store, const uint8_t* hash32, const void* bytes,
                   size_t len);
/* Copies the blob into out: its length, -1 if not held (a miss), or
 * VAPI_KV_ESPACE if cap is too small (nothing counted). */
int64_t vapi_spill_get(vapi_spill_store* store, const uint8_t* hash32, void* out, size_t cap);
void vapi_spill_get_stats(const vapi_spill_store* store, vapi_spill_stats* out);

/*
 * spill_evicted (crates/vapi-worker/src/engine.rs:369-393) for a batch:
 * ids/hashes (host arrays, n and n*32 bytes) are the blocks the pool just
 * evicted; those the store does not hold are exported in batches with
 * vapi_kv_export_blocks into `pinned` (hipHostMalloc memory of at least
 * 4096 + vapi_kv_block_bytes bytes; its first 4 KiB stage the ids) and put
 * into the store. Synchronous on `stream`: the blocks may be overwritten
 * once it returns. Returns the number exported, or a negative error.
 */
int64_t vapi_spill_evicted(vapi_spill_store* store, const vapi_kv_pool* pool,
                           const uint32_t* ids, const uint8_t* hashes, uint32_t n,
                           void* pinned, size_t pinned_bytes, vapi_stream_t stream);

/*
 * vapi_spill_evicted overlapped with the forward (no counterpart in the
 * reference, whose spill_evicted, engine.rs:369-393, blocks the step). The
 * blocks the store does not hold are packed into device `staging` on
 * `stream` (an HBM copy: the forward may overwrite the blocks once it has
 * run on `stream`), then copied to `pinned` on `side`. The blobs enter the
 * store at a drain: vapi_spill_drain, and every store call drains the
 * exports whose copies have completed (get waits for a blob in flight;
 * vapi_spill_evicted and vapi_spill_promote wait for all); contains() does
 * not report blobs in flight. Blocks already held or in flight are skipped.
 * Up to 16 exports are in flight per store, each owning its staging and
 * pinned buffers until it is drained: rotate a ring of buffers; a call
 * whose buffers overlap an in-flight export's waits for it first. staging
 * must hold every block to export and pinned 4 KiB more; at most 1,024
 * blocks (else VAPI_KV_ESPACE). Returns the number exported.
 */
int64_t vapi_spill_evicted_async(vapi_spill_store* store, const vapi_kv_pool* pool,
                                 const uint32_t* ids, const uint8_t* hashes, uint32_t n,
                                 void* staging, size_t staging_bytes, void* pinned,
                                 size_t pinned_bytes, vapi_stream_t stream, vapi_stream_t side);

/*
 * Puts the blobs of in-flight asynchronous exports into the store, oldest
 * first: all of them if `wait` (blocking on their copies), else those whose
 * copies have completed. Returns the number of blobs stored, or a negative
 * error.
 */
int64_t vapi_spill_drain(vapi_spill_store* store, int wait);

/*
 * The device half of promote_from_spill (engine.rs:400-456): hashes[0..n)
 * are a prompt's block chain and ids[0..n) (host) the blocks allocated for
 * them. Blobs are taken in order up to the first hash the store does not
 * hold (counted as a miss, as the reference's get() does) and imported
 * with vapi_kv_import_blocks through `pinned` (sized as for
 * vapi_spill_evicted). A blob that is not vapi_kv_block_bytes long is an
 * error (backend.rs:739-745). Returns the number restored (a prefix).
 */
int64_t vapi_spill_promote(vapi_spill_store* store, const vapi_kv_pool* pool,
                           const uint8_t* hashes, const uint32_t* ids, uint32_t n,
                           void* pinned, size_t pinned_bytes, vapi_stream_t stream);

/*
 * Host-side check of a step descriptor: ForwardBatch::validate
 * (crates/vapi-engine/src/backend.rs:96-204). All arrays are host memory.
 * block_tables is ragged: row i is table_data[table_offsets[i] ..
 * table_offsets[i+1]] (table_offsets has batch+1 entries). Returns
 * VAPI_KV_EINVAL with the reference's message on the first violation.
 */
int vapi_forward_batch_validate(uint32_t n_tokens, const uint32_t* positions,
                                const uint32_t* slot_mapping,
                                const uint32_t* cu_seqlens_q,
                                const uint32_t* cu_seqlens_k, uint32_t batch,
                                const uint32_t* table_offsets,
                                const uint32_t* table_data,
                                const uint32_t* logits_indices,
                                uint32_t n_logits, uint32_t num_blocks,
                                uint32_t block_size);

/*
 * Host packing of ragged block tables into [batch, width] (pack_block_tables,
 * attention.rs:42-62): width = max(max row length, 1); each row is padded
 * with its own last block (0 for an empty row). out holds batch*width u32;
 * returns width, or a negative code if out_capacity is too small.
 */
int64_t vapi_pack_block_tables(uint32_t batch, const uint32_t* table_offsets,
                               const uint32_t* table_data, uint32_t* out,
                               size_t out_capacity);

/* ---- host-side cache object (PagedKvCache + the backend block methods) -- */

typedef struct vapi_cache vapi_cache;

/* PagedKvCache::new (cache.rs:48-68): zeroed K and V for every layer, in one
 * device allocation. */
int vapi_cache_new(uint32_t num_layers, uint32_t num_blocks,
                   uint32_t block_size, uint32_t num_kv_heads,
                   uint32_t head_dim, uint32_t dtype, uint32_t layout,
                   vapi_cache** out);
void vapi_cache_free(vapi_cache* cache);
/* The pool descriptor the low-level calls take. */
int vapi_cache_pool(const vapi_cache* cache, vapi_kv_pool* out);
/* PagedKvCache::num_slots (cache.rs:115-117). */
uint64_t vapi_cache_num_slots(const vapi_cache* cache);

/* write_kv_to_cache (cache.rs:136-148): k, v device [n_tokens, kvh, d] of
 * src_dtype; slot_mapping is host u32[n_slots]. Errors as the reference:
 * n_tokens != n_slots, src dtype != cache dtype, a slot past the end. */
int vapi_cache_write_kv(vapi_cache* cache, uint32_t layer, const void* k,
                        const void* v, uint32_t n_tokens, uint32_t src_dtype,
                        const uint32_t* slot_mapping, uint32_t n_slots,
                        vapi_stream_t stream);

/* ExecutionBackend::block_bytes / export_block / import_block / copy_blocks
 * (crates/vapi-engine/src/backend.rs:344-367, implementation
 * crates/vapi-backend-candle/src/backend.rs:695-797). Synchronous on the
 * null stream; host buffers may be pageable. */
size_t vapi_cache_block_bytes(const vapi_cache* cache);
int vapi_cache_export_block(vapi_cache* cache, uint32_t id, void* out,
                            size_t out_len);
int vapi_cache_import_block(vapi_cache* cache, uint32_t id, const void* bytes,
                            size_t len);
int vapi_cache_copy_blocks(vapi_cache* cache, const uint32_t* pairs_host,
                           uint32_t n_pairs);

#ifdef __cplusplus
}
#endif

#endif /* VAPI_KV_H */
