// C ABI of paged attention: one varlen call covers decode rows (len_q == 1)
// and chunked-prefill rows (len_q > 1), dispatched to
//  * the persistent MFMA decode stream (attn_decode.hip) for decode rows,
//  * the MFMA prefill kernel (attn_prefill.hip) for prefill rows,
// when the pool is bf16/f16 with head_dim 64, 128 or 256, a power-of-two
// block_size >= 16 and at most 16 query heads per kv head (up to 64 when a
// split into 2 or 4 equal groups of at most 16 exists); an f32 pool of
// that shape (head_dim 64 or 128) runs the decode stream and an f32 prefill
// kernel (attn_prefill_f32.hip) on f32 MFMAs; a 16-bit decode-only call at a
// head_dim that is another multiple of 8 up to 256 runs the decode stream
// padded to the next of 64, 128, 256; every other shape runs the VALU kernel
// (attn_generic.hip).
// Replaces paged_attention_cuda/_windowed/_prepared (vapi
// crates/vapi-backend-candle/src/attention.rs:170-288).
#include <mutex>

#include "attn_common.hpp"

namespace vk {

// The decode's MFMA tile has 16 query-head columns: a group of G > 16
// query heads per kv head runs as n = ceil(G / 16) virtual kv heads of
// ceil(G / n) query heads each (the last one may serve fewer), each reading
// its pool head's K/V. The part count n, or 0 past 16 parts (G > 256).
static uint32_t decode_group_parts(uint32_t G) {
  if (G == 0) return 0;
  const uint32_t n = (G + 15) / 16;
  return n <= 16 ? n : 0;
}

// An f32 pool whose calls run on v_mfma_f32_16x16x4_f32: decode rows on the
// decode stream, prefill rows on paged_prefill_f32. A small pure-decode call
// (at most 512 keys per sequence and 8,192 over the batch, config 0's shape)
// runs the VALU kernel instead, in one launch with no merge. Replayed from
// a graph, 16 q / 8 kv heads: config 0 (8 x <= 512 keys) 14.1 against
// 16.4 us; 16 x 128 10.8 against 14.5; 64 x 256 27.3 against 26.3 and
// 32 x 512 29.2 against 25.8, where the decode stream takes over.
constexpr uint32_t kSmallKeys = 512;
constexpr uint64_t kSmallBatchKeys = 8192;
static bool f32_mfma_ok(const vapi_kv_pool* p, uint32_t num_heads, uint32_t max_q,
                        uint32_t max_k, uint32_t batch) {
  if (p->dtype != VAPI_KV_F32) return false;
  if (max_q <= 1 && max_k <= kSmallKeys && (uint64_t)batch * max_k <= kSmallBatchKeys)
    return false;
  // head_dim 64 or 128, or a multiple of 4 below 128 run at the next of
  // them (elements past head_dim read as zeros and never stored).
  if (p->head_dim == 0 || p->head_dim % 4 || p->head_dim > 128) return false;
  if (p->block_size < 16 || (p->block_size & (p->block_size - 1))) return false;
  if (num_heads == 0 || num_heads % p->num_kv_heads) return false;
  return decode_group_parts(num_heads / p->num_kv_heads) > 0;
}

static bool mfma_ok(const vapi_kv_pool* p, uint32_t num_heads) {
  if (p->dtype != VAPI_KV_BF16 && p->dtype != VAPI_KV_F16) return false;
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) return false;
  if (p->block_size < 16 || (p->block_size & (p->block_size - 1))) return false;
  if (num_heads == 0 || num_heads % p->num_kv_heads) return false;
  return decode_group_parts(num_heads / p->num_kv_heads) > 0;
}

// The decode kernel's D for a pool's head_dim: itself for 64, 128 and 256,
// else the next of them (elements past head_dim are zeros).
static uint32_t decode_dim(uint32_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : 256; }

// A 16-bit pool whose head_dim is not one of the kernels' but a multiple of 8
// below 256 (Phi-2's 80, Phi-3's 96, ...): its calls run the decode stream
// and the prefill kernel at decode_dim, elements past head_dim read as zeros
// and never stored (no fused append, no one-launch mixed step).
static bool pad16_ok(const vapi_kv_pool* p, uint32_t num_heads) {
  if (p->dtype != VAPI_KV_BF16 && p->dtype != VAPI_KV_F16) return false;
  const uint32_t hd = p->head_dim;
  if (hd == 0 || hd % 8 || hd > 256 || hd == 64 || hd == 128 || hd == 256) return false;
  if (p->block_size < 16 || (p->block_size & (p->block_size - 1))) return false;
  if (num_heads == 0 || num_heads % p->num_kv_heads) return false;
  return decode_group_parts(num_heads / p->num_kv_heads) > 0;
}

// A 16-bit pool on the MFMA kernels, at its own head_dim or padded.
static bool mfma16_ok(const vapi_kv_pool* p, uint32_t num_heads) {
  return mfma_ok(p, num_heads) || pad16_ok(p, num_heads);
}

// The decode's view of the kv heads (virtual ones when G > 16).
static size_t decode_ws_for(const vapi_kv_pool* p, uint32_t batch, uint32_t num_heads) {
  const uint32_t G = num_heads / p->num_kv_heads;
  const uint32_t n = decode_group_parts(G);
  return decode_workspace_bytes(batch, p->num_kv_heads * n, (G + n - 1) / n, decode_dim(p->head_dim),
                                decode_num_waves());
}

// The sequences with prefill rows, named by the host (vapi_paged_attention_prepared).
struct PrefillSeqs {
  const uint32_t* seqs;  // device u32[n]
  uint32_t n;
};

// The fused append's new rows (decode batches on the MFMA path only).
struct NewRows {
  const void* k;
  const void* v;
  const uint32_t* slots;
  uint32_t n;
};

// ---- allocation-free variant: the decode workspace in a device array ------
//
// `scratch` is this library's own copy of the decode workspace (XCD shares,
// per-segment ranges, split partials) for callers that cannot allocate.
// Every GPU the library runs on holds one copy, at its own address, until
// the process ends. The host uses `scratch` only through the address
// hipGetSymbolAddress returns on that device: in host code the array's name
// is a host-side stand-in, not device memory.
static __device__ __align__(256) unsigned char scratch[VAPI_ATTN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // per device, set once

// Zeroes the balance block at the start of the scratch (the shares a fresh
// workspace starts from). A kernel, not hipMemsetAsync, so that a call
// recorded into a HIP graph replays it correctly.
__global__ void scratch_clear_kernel(uint32_t* p, uint32_t n_words) {
  for (uint32_t i = threadIdx.x; i < n_words; i += blockDim.x) p[i] = 0u;
}

// The current device's scratch address, resolved by the first call on each
// device. Its balance block is cleared on `stream` by the first call that is
// not being captured into a HIP graph: a clear recorded into a graph would
// reset the shares on every replay. Until then the shares hold whatever the
// array held; any shares give the same results (they only move where the
// work is split, and unusable values count as uniform shares).
static bool g_scratch_cleared[kMaxDevices];

static int scratch_for_device(void** out, hipStream_t stream) {
  int dev = 0;
  VK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention_noalloc: device %d of at most %d", dev,
            kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      VK_FAIL(VAPI_KV_EHIP, "vapi_paged_attention_noalloc: hipGetSymbolAddress(scratch): %s",
              hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  if (!g_scratch_cleared[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    VK_HIP(hipStreamIsCapturing(stream, &cap));
    if (cap == hipStreamCaptureStatusNone) {
      hipLaunchKernelGGL(scratch_clear_kernel, dim3(1), dim3(256), 0, stream,
                         (uint32_t*)g_scratch_ptr[dev],
                         (uint32_t)(kDecodeBalanceBytes / sizeof(uint32_t)));
      VK_LAUNCHED("scratch_clear_kernel");
      g_scratch_cleared[dev] = true;
    }
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace vk

using namespace vk;

static int paged_attention_impl(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                void* out, const uint32_t* cu_seqlens_q,
                                const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                int32_t window_left, int32_t window_right, void* workspace,
                                size_t workspace_bytes, vapi_stream_t stream,
                                const NewRows* fuse, uint32_t flags,
                                const PrefillSeqs* pf = nullptr);

// The workspace a call cannot run without: the decode's (unless the call
// launches no decode kernel) or the VALU kernel's split partials.
static size_t required_workspace(const vapi_kv_pool* pool, uint32_t batch, uint32_t num_heads,
                                 uint32_t max_seqlen_q, uint32_t max_seqlen_k, bool skip_decode) {
  if (!pool || pool->num_kv_heads == 0 || num_heads % pool->num_kv_heads || batch == 0 ||
      num_heads == 0)
    return 0;
  const uint32_t group = num_heads / pool->num_kv_heads;
  if (!mfma16_ok(pool, num_heads) &&
      !f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch))
    return generic_workspace_bytes(batch, pool->num_kv_heads, group, pool->head_dim,
                                   std::max(max_seqlen_q, 1u), max_seqlen_k);
  return skip_decode ? 0 : decode_ws_for(pool, batch, num_heads);
}

// The optional part of the workspace: the prefill key split's partials for
// n_prefill sequences with prefill rows (a batch of `batch`).
static size_t split_bytes(const vapi_kv_pool* pool, uint32_t batch, uint32_t num_heads,
                          uint32_t max_seqlen_q, uint32_t max_seqlen_k, uint32_t n_prefill) {
  if (!pool || pool->num_kv_heads == 0 || num_heads % pool->num_kv_heads || batch == 0 ||
      num_heads == 0)
    return 0;
  const uint32_t kvh = pool->num_kv_heads, group = num_heads / kvh;
  if (mfma16_ok(pool, num_heads))
    return prefill_split_bytes(n_prefill, kvh, group, decode_dim(pool->head_dim), max_seqlen_q,
                               max_seqlen_k);
  if (f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch))
    return prefill_f32_split_bytes(n_prefill, kvh, group, decode_dim(pool->head_dim), max_seqlen_q,
                                   max_seqlen_k);
  return 0;
}

extern "C" {

size_t vapi_paged_attention_workspace_size(const vapi_kv_pool* pool,
                                           uint32_t batch, uint32_t num_heads,
                                           uint32_t max_seqlen_q,
                                           uint32_t max_seqlen_k) {
  const size_t need =
      required_workspace(pool, batch, num_heads, max_seqlen_q, max_seqlen_k, false);
  // Past the decode's part: what a small prefill batch's key split uses
  // (optional: a smaller workspace only means fewer splits).
  return need + split_bytes(pool, batch, num_heads, max_seqlen_q, max_seqlen_k, batch);
}

size_t vapi_paged_attention_prepared_workspace_size(const vapi_kv_pool* pool, uint32_t batch,
                                                    uint32_t n_prefill, uint32_t num_heads,
                                                    uint32_t max_seqlen_q,
                                                    uint32_t max_seqlen_k) {
  const size_t need =
      required_workspace(pool, batch, num_heads, max_seqlen_q, max_seqlen_k, false);
  return need + split_bytes(pool, batch, num_heads, max_seqlen_q, max_seqlen_k,
                            std::min(n_prefill, batch));
}

int vapi_paged_attention_prepared(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                  void* out, const uint32_t* cu_seqlens_q,
                                  const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                  uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                  uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                  int32_t window_left, int32_t window_right, uint32_t flags,
                                  const uint32_t* prefill_seqs, uint32_t n_prefill,
                                  void* workspace, size_t workspace_bytes,
                                  vapi_stream_t stream) {
  if (n_prefill > batch)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention_prepared: %u prefill sequences in a batch of %u",
            n_prefill, batch);
  if (n_prefill && !prefill_seqs)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention_prepared: null prefill_seqs");
  const PrefillSeqs pf{prefill_seqs, n_prefill};
  return paged_attention_impl(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                              batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                              window_left, window_right, workspace, workspace_bytes, stream,
                              nullptr, flags, &pf);
}

int vapi_paged_attention(const vapi_kv_pool* pool, uint32_t layer,
                         const void* q, void* out,
                         const uint32_t* cu_seqlens_q,
                         const uint32_t* cu_seqlens_k,
                         const uint32_t* block_table, uint32_t batch,
                         uint32_t max_blocks, uint32_t max_seqlen_q,
                         uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                         int32_t window_left, int32_t window_right,
                         void* workspace, size_t workspace_bytes,
                         vapi_stream_t stream) {
  return vapi_paged_attention_ex(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                                 batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                                 window_left, window_right, 0u, workspace, workspace_bytes,
                                 stream);
}

int vapi_paged_attention_ex(const vapi_kv_pool* pool, uint32_t layer, const void* q, void* out,
                            const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                            const uint32_t* block_table, uint32_t batch, uint32_t max_blocks,
                            uint32_t max_seqlen_q, uint32_t max_seqlen_k, uint32_t num_heads,
                            float scale, int32_t window_left, int32_t window_right,
                            uint32_t flags, void* workspace, size_t workspace_bytes,
                            vapi_stream_t stream) {
  return paged_attention_impl(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                              batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                              window_left, window_right, workspace, workspace_bytes, stream,
                              nullptr, flags);
}

int vapi_paged_attention_append(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                                const void* v_src, const uint32_t* slot_mapping,
                                uint32_t n_tokens, const void* q, void* out,
                                const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                                const uint32_t* block_table, uint32_t batch,
                                uint32_t max_blocks, uint32_t max_seqlen_q,
                                uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                int32_t window_left, int32_t window_right, void* workspace,
                                size_t workspace_bytes, vapi_stream_t stream) {
  return vapi_paged_attention_append_ex(pool, layer, k_src, v_src, slot_mapping, n_tokens, q,
                                        out, cu_seqlens_q, cu_seqlens_k, block_table, batch,
                                        max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                                        window_left, window_right, 0u, workspace,
                                        workspace_bytes, stream);
}

int vapi_paged_attention_append_ex(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                                   const void* v_src, const uint32_t* slot_mapping,
                                   uint32_t n_tokens, const void* q, void* out,
                                   const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                                   const uint32_t* block_table, uint32_t batch,
                                   uint32_t max_blocks, uint32_t max_seqlen_q,
                                   uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                   int32_t window_left, int32_t window_right, uint32_t flags,
                                   void* workspace, size_t workspace_bytes,
                                   vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_paged_attention_append")) return rc;
  if (!pool->v) VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention_append: a K-only pool has no V to attend over");
  const bool fused = n_tokens > 0 && batch > 0 && max_seqlen_q == 1 && num_heads > 0 &&
                     num_heads % pool->num_kv_heads == 0 && mfma_ok(pool, num_heads) &&
                     num_heads / pool->num_kv_heads <= 16;
  if (!fused) {
    if (int rc = vapi_kv_append(pool, layer, k_src, v_src, slot_mapping, n_tokens, stream))
      return rc;
    return vapi_paged_attention_ex(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                                   batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads,
                                   scale, window_left, window_right, flags, workspace,
                                   workspace_bytes, stream);
  }
  if (!k_src || !v_src || !slot_mapping)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention_append: null source or slot_mapping");
  const NewRows rows{k_src, v_src, slot_mapping, n_tokens};
  return paged_attention_impl(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                              batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                              window_left, window_right, workspace, workspace_bytes, stream,
                              &rows, flags);
}

int vapi_paged_attention_noalloc(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                 void* out, const uint32_t* cu_seqlens_q,
                                 const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                 uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                 uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                 int32_t window_left, int32_t window_right, uint32_t flags,
                                 vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_paged_attention_noalloc")) return rc;
  // Sized before anything is resolved or launched: a call past the limit is
  // refused and changes nothing.
  const bool skip = (flags & VAPI_ATTN_NO_DECODE_ROWS) && max_seqlen_q > 1;
  const size_t need =
      required_workspace(pool, batch, num_heads, max_seqlen_q, max_seqlen_k, skip);
  if (need > VAPI_ATTN_SCRATCH_BYTES)
    VK_FAIL(VAPI_KV_ESPACE,
            "vapi_paged_attention_noalloc: this batch needs %zu bytes of decode workspace, more "
            "than the library's %u-byte scratch (use vapi_paged_attention_ex with a workspace)",
            need, (unsigned)VAPI_ATTN_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_for_device(&ws, hs(stream))) return rc;
  return paged_attention_impl(pool, layer, q, out, cu_seqlens_q, cu_seqlens_k, block_table,
                              batch, max_blocks, max_seqlen_q, max_seqlen_k, num_heads, scale,
                              window_left, window_right, ws, VAPI_ATTN_SCRATCH_BYTES, stream,
                              nullptr, flags);
}

}  // extern "C"

static int paged_attention_impl(const vapi_kv_pool* pool, uint32_t layer, const void* q,
                                void* out, const uint32_t* cu_seqlens_q,
                                const uint32_t* cu_seqlens_k, const uint32_t* block_table,
                                uint32_t batch, uint32_t max_blocks, uint32_t max_seqlen_q,
                                uint32_t max_seqlen_k, uint32_t num_heads, float scale,
                                int32_t window_left, int32_t window_right, void* workspace,
                                size_t workspace_bytes, vapi_stream_t stream,
                                const NewRows* fuse, uint32_t flags, const PrefillSeqs* pf) {
  if (int rc = check_pool(pool, "vapi_paged_attention")) return rc;
  if (!pool->v) VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: a K-only pool has no V to attend over");
  if (layer >= pool->num_layers)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: layer %u of %u", layer,
            pool->num_layers);
  if (num_heads == 0 || num_heads % pool->num_kv_heads != 0)
    VK_FAIL(VAPI_KV_EINVAL,
            "vapi_paged_attention: %u query heads is not a multiple of %u kv heads",
            num_heads, pool->num_kv_heads);
  if (batch == 0 || max_seqlen_q == 0) return 0;
  if (!q || !out || !cu_seqlens_q || !cu_seqlens_k || !block_table)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: null device pointer");
  if (((uintptr_t)q | (uintptr_t)out) & 15)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: q and out must be 16-byte aligned");
  if (pool->num_blocks == 0 && max_seqlen_k > 0)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: keys to attend over in an empty pool");
  if (max_blocks == 0)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: block table width 0");
  if (flags & ~(uint32_t)(VAPI_ATTN_DETERMINISTIC | VAPI_ATTN_NO_DECODE_ROWS))
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: unknown flags 0x%x", flags);
  if (num_heads > 65535 ||
      (batch > 65535 && !mfma16_ok(pool, num_heads) &&
       !f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch)))
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: batch %u / heads %u too large",
            batch, num_heads);
  // A batch the caller says has no decode rows (and which is not a fused
  // decode step) runs one kernel: the prefill kernel then takes every row,
  // len_q == 1 included, so the result does not depend on the hint. It needs
  // no workspace.
  const bool skip_decode = (flags & VAPI_ATTN_NO_DECODE_ROWS) && !fuse && max_seqlen_q > 1 &&
                           (mfma16_ok(pool, num_heads) ||
                            f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch));
  // The sequences the prefill grid covers: those the host named (a mixed
  // step's few prefill chunks among many decode rows), else all of them. A
  // prefill-only call covers every row and ignores the list.
  const bool listed = pf && !skip_decode;
  const uint32_t pf_n = listed ? pf->n : batch;
  // Refused before anything is launched (a refused call writes nothing).
  if (mfma16_ok(pool, num_heads) && max_seqlen_q > 1 && pf_n > 65535)
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: %u prefill sequences > 65535", pf_n);
  if (mfma16_ok(pool, num_heads) && max_seqlen_q > 1 &&
      prefill_grid(pf_n, pool->num_kv_heads, num_heads / pool->num_kv_heads, max_seqlen_q,
                   decode_dim(pool->head_dim)) >
          0xFFFFFFFFull)
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: prefill batch too large for one launch");
  if (f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch) && max_seqlen_q > 1 &&
      prefill_f32_items(pf_n, pool->num_kv_heads, num_heads / pool->num_kv_heads,
                        max_seqlen_q) > 0xFFFFFFFFull)
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: prefill batch too large for one launch");
  const size_t need =
      required_workspace(pool, batch, num_heads, max_seqlen_q, max_seqlen_k, skip_decode);
  if (workspace_bytes < need || (need && !workspace))
    VK_FAIL(VAPI_KV_ESPACE, "vapi_paged_attention: workspace %zu bytes < %zu",
            workspace_bytes, need);

  const Geom g = make_geom(pool);
  LayerPtrs lp = layer_ptrs(pool, layer);
  AttnArgs a;
  a.k = lp.k;
  a.v = lp.v;
  a.q = (const char*)q;
  a.out = (char*)out;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.table = block_table;
  a.seg_ranges = nullptr;
  a.ws_ml = nullptr;
  a.ws_o = nullptr;
  a.bal = nullptr;
  a.k_new = fuse ? (const char*)fuse->k : nullptr;
  a.v_new = fuse ? (const char*)fuse->v : nullptr;
  a.slots = fuse ? fuse->slots : nullptr;
  a.n_new = fuse ? fuse->n : 0;
  a.num_slots = g.num_blocks * g.block_size;
  a.last_blk = g.num_blocks ? g.num_blocks - 1 : 0;
  a.blk_e = g.blk;
  a.head_e = g.head;
  a.tok_e = (uint32_t)g.tok;
  a.max_blocks = max_blocks;
  a.batch = batch;
  a.num_heads = num_heads;
  a.kvh = g.kvh;
  a.group = num_heads / g.kvh;
  a.block_size = g.block_size;
  a.bs_shift = 0;
  while ((1u << a.bs_shift) < g.block_size) ++a.bs_shift;
  a.num_waves = 0;
  a.scale = scale;
  // A zero scale is kept positive so that masked scores (-inf) times it stay -inf.
  a.scale_log2 = fmaxf(fabsf(scale) * kLog2e, 1e-30f);
  a.q_sign = scale < 0.f ? 0x80008000u : 0u;
  a.wl = window_left < 0 ? -1 : window_left;
  a.wr = window_right < 0 ? -1 : window_right;
  a.deterministic = (flags & VAPI_ATTN_DETERMINISTIC) ? 1u : 0u;
  a.pf_min_q = 2;
  a.pf_seqs = listed ? pf->seqs : nullptr;
  a.pf_seqs_n = pf_n;
  a.kv_parts = FastDiv(1);
  a.g_real = a.group;
  a.hd = g.d;
  const hipStream_t s = hs(stream);
  // The decode kernels' arguments: with G > 16 query heads per kv head, the
  // virtual kv heads of at most 16 query heads each.
  const uint32_t parts = decode_group_parts(a.group);
  AttnArgs dec = a;
  if (parts > 1) {
    dec.kvh = a.kvh * parts;
    dec.group = (a.group + parts - 1) / parts;
    dec.kv_parts = FastDiv(parts);
  }

  if (mfma16_ok(pool, num_heads)) {
    const bool bf16 = pool->dtype == VAPI_KV_BF16;
    const uint32_t D = decode_dim(g.d);
    a.num_waves = decode_num_waves();
    const size_t off = std::max<size_t>((need + 255) & ~(size_t)255, 256);
    const bool room = workspace && workspace_bytes > off;
    // Decode rows and prefill rows in one step: both kernels in one launch.
    // (At most 4,000 sequences: the launch's dynamic LDS, 4 bytes per
    // sequence, then still lets a decode and a prefill workgroup share a CU.
    // At head_dim 256 neither kernel fits half a CU's registers; a padded
    // head_dim below 128 runs the padded kernels.)
    const bool mixed = !skip_decode && !fuse && parts == 1 && D <= 128 &&
                       max_seqlen_q > 1 &&
                       pf_n > 0 &&
                       batch <= std::min(decode_max_plan_seqs(), 4000u) &&
                       mixed_prefill_items(pf_n, g.kvh, num_heads / g.kvh, max_seqlen_q) <
                           (1ull << 30);
    if (mixed) {
      launch_mixed(a, workspace, max_seqlen_q, max_seqlen_k, D, bf16,
                   room ? (char*)workspace + off : nullptr, room ? workspace_bytes - off : 0, s);
      VK_LAUNCHED("paged_attention");
      return 0;
    }
    if (skip_decode) {
      a.pf_min_q = 1;
    } else {
      dec.num_waves = a.num_waves;
      launch_decode(dec, workspace, D, pool->dtype, s);
    }
    if (max_seqlen_q > 1 && pf_n > 0) {
      // The workspace past the decode's part serves the prefill's key split
      // (never its first 256 bytes, which carry the decode's XCD shares
      // from call to call).
      launch_prefill(a, max_seqlen_q, max_seqlen_k, D, bf16,
                     room ? (char*)workspace + off : nullptr, room ? workspace_bytes - off : 0, s);
    }
  } else if (f32_mfma_ok(pool, num_heads, max_seqlen_q, max_seqlen_k, batch)) {
    if (skip_decode) {
      a.pf_min_q = 1;
    } else {
      dec.num_waves = decode_num_waves();
      launch_decode(dec, workspace, decode_dim(g.d), pool->dtype, s);
    }
    if (max_seqlen_q > 1 && pf_n > 0) {
      // The workspace past the decode's part (never its first 256 bytes,
      // the XCD shares) serves the key split, as for 16-bit pools.
      const size_t off = std::max<size_t>((need + 255) & ~(size_t)255, 256);
      const bool room = workspace && workspace_bytes > off;
      launch_prefill_f32(a, max_seqlen_q, max_seqlen_k, decode_dim(g.d),
                         room ? (char*)workspace + off : nullptr,
                         room ? workspace_bytes - off : 0, s);
    }
  } else {
    if (g.d > 256)
      VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: head_dim %u > 256", g.d);
    if (generic_grid(batch, g.kvh, num_heads / g.kvh, max_seqlen_q, max_seqlen_k) > 0xFFFFFFFFull)
      VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: batch too large for one launch");
    launch_generic(a, max_seqlen_q, max_seqlen_k, g.d, pool->dtype, workspace, s);
  }
  VK_LAUNCHED("paged_attention");
  return 0;
}
