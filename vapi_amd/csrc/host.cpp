// Host side of the boundary: the cache object that owns the pool (vapi's
// PagedKvCache plus the ExecutionBackend block methods) and the host checks
// a step descriptor goes through (ForwardBatch::validate, pack_block_tables).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

using namespace vk;

struct vapi_cache {
  vapi_kv_pool pool;
  void* slab = nullptr;      // K layers then V layers, one allocation
  uint32_t* upload = nullptr;  // device staging for host index arrays
  size_t upload_cap = 0;       // in u32
  void* blob = nullptr;        // device staging of one exported block
};

static int ensure_upload(vapi_cache* c, size_t n) {
  if (n <= c->upload_cap) return 0;
  if (c->upload) VK_HIP(hipFree(c->upload));
  c->upload = nullptr;
  c->upload_cap = 0;
  size_t cap = std::max<size_t>(n, 1024);
  VK_HIP(hipMalloc((void**)&c->upload, cap * sizeof(uint32_t)));
  c->upload_cap = cap;
  return 0;
}

extern "C" {

// PagedKvCache::new (cache.rs:48-106): every layer's K and V zeroed.
int vapi_cache_new(uint32_t num_layers, uint32_t num_blocks,
                   uint32_t block_size, uint32_t num_kv_heads,
                   uint32_t head_dim, uint32_t dtype, uint32_t layout,
                   vapi_cache** out) {
  clear_error();
  if (!out) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_new: null out");
  *out = nullptr;
  vapi_cache* c = new vapi_cache();
  vapi_kv_pool& p = c->pool;
  p.num_layers = num_layers;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.dtype = dtype;
  p.layout = layout;
  p.next = nullptr;
  p.block_stride_bytes = 0;
  const size_t layer_bytes = vapi_kv_layer_bytes(&p);
  // Align each layer buffer to 256 bytes.
  p.layer_stride_bytes = (layer_bytes + 255) & ~(size_t)255;
  const size_t half = p.layer_stride_bytes * num_layers;
  if (num_blocks > 0 && half > 0) {
    hipError_t e = hipMalloc(&c->slab, 2 * half);
    if (e != hipSuccess) {
      delete c;
      VK_FAIL(VAPI_KV_EHIP, "vapi_cache_new: hipMalloc(%zu) failed: %s", 2 * half,
              hipGetErrorString(e));
    }
    e = hipMemset(c->slab, 0, 2 * half);
    if (e != hipSuccess) {
      (void)hipFree(c->slab);
      delete c;
      VK_FAIL(VAPI_KV_EHIP, "vapi_cache_new: hipMemset failed: %s",
              hipGetErrorString(e));
    }
  }
  p.k = c->slab;
  p.v = c->slab ? (char*)c->slab + half : nullptr;
  // check_pool wants non-null bases for a non-empty pool; an empty pool is a
  // legal (useless) object.
  if (num_blocks > 0) {
    if (int rc = check_pool(&p, "vapi_cache_new")) {
      if (c->slab) (void)hipFree(c->slab);
      delete c;
      return rc;
    }
  }
  *out = c;
  return 0;
}

void vapi_cache_free(vapi_cache* c) {
  if (!c) return;
  if (c->slab) (void)hipFree(c->slab);
  if (c->upload) (void)hipFree(c->upload);
  if (c->blob) (void)hipFree(c->blob);
  delete c;
}

int vapi_cache_pool(const vapi_cache* c, vapi_kv_pool* out) {
  if (!c || !out) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_pool: null argument");
  *out = c->pool;
  return 0;
}

uint64_t vapi_cache_num_slots(const vapi_cache* c) {
  return c ? (uint64_t)c->pool.num_blocks * c->pool.block_size : 0;
}

// write_kv_to_cache + write_rows checks (cache.rs:136-148, 223-240).
int vapi_cache_write_kv(vapi_cache* c, uint32_t layer, const void* k,
                        const void* v, uint32_t n_tokens, uint32_t src_dtype,
                        const uint32_t* slot_mapping, uint32_t n_slots,
                        vapi_stream_t stream) {
  clear_error();
  if (!c) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_write_kv: null cache");
  if (layer >= c->pool.num_layers)
    VK_FAIL(VAPI_KV_EINVAL, "layer %u of %u", layer, c->pool.num_layers);
  if (n_tokens != n_slots)
    VK_FAIL(VAPI_KV_EINVAL, "%u tokens but %u cache slots", n_tokens, n_slots);
  if (src_dtype != c->pool.dtype)
    VK_FAIL(VAPI_KV_EINVAL, "cache is dtype %u but the rows are dtype %u",
            c->pool.dtype, src_dtype);
  if (n_tokens == 0) return 0;
  const uint64_t num_slots = vapi_cache_num_slots(c);
  uint32_t mx = 0;
  for (uint32_t i = 0; i < n_slots; ++i)
    if (slot_mapping[i] != VAPI_KV_SLOT_SKIP) mx = std::max(mx, slot_mapping[i]);
  if (mx >= num_slots)
    VK_FAIL(VAPI_KV_EINVAL, "slot %u is past the end of the cache", mx);
  if (int rc = ensure_upload(c, n_slots)) return rc;
  VK_HIP(hipMemcpyAsync(c->upload, slot_mapping, n_slots * sizeof(uint32_t),
                        hipMemcpyHostToDevice, hs(stream)));
  return vapi_kv_append(&c->pool, layer, k, v, c->upload, n_tokens, stream);
}

size_t vapi_cache_block_bytes(const vapi_cache* c) {
  return c ? vapi_kv_block_bytes(&c->pool) : 0;
}

// CandleBackend::export_block (backend.rs:718-734): one device pack, one
// copy to the host.
int vapi_cache_export_block(vapi_cache* c, uint32_t id, void* out,
                            size_t out_len) {
  clear_error();
  if (!c) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_export_block: null cache");
  const size_t bb = vapi_kv_block_bytes(&c->pool);
  if (id >= c->pool.num_blocks)
    VK_FAIL(VAPI_KV_EINVAL, "block %u of %u", id, c->pool.num_blocks);
  if (out_len < bb)
    VK_FAIL(VAPI_KV_ESPACE, "export buffer is %zu bytes, a block is %zu", out_len, bb);
  if (!c->blob) VK_HIP(hipMalloc(&c->blob, bb));
  if (int rc = ensure_upload(c, 1)) return rc;
  VK_HIP(hipMemcpy(c->upload, &id, sizeof id, hipMemcpyHostToDevice));
  if (int rc = vapi_kv_export_blocks(&c->pool, c->upload, 1, c->blob, nullptr))
    return rc;
  VK_HIP(hipMemcpy(out, c->blob, bb, hipMemcpyDeviceToHost));
  return 0;
}

// CandleBackend::import_block (backend.rs:738-773), length check included.
int vapi_cache_import_block(vapi_cache* c, uint32_t id, const void* bytes,
                            size_t len) {
  clear_error();
  if (!c) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_import_block: null cache");
  const size_t bb = vapi_kv_block_bytes(&c->pool);
  if (len != bb)
    VK_FAIL(VAPI_KV_EINVAL, "spilled block is %zu bytes, this cache wants %zu", len,
            bb);
  if (id >= c->pool.num_blocks)
    VK_FAIL(VAPI_KV_EINVAL, "block %u of %u", id, c->pool.num_blocks);
  if (!c->blob) VK_HIP(hipMalloc(&c->blob, bb));
  if (int rc = ensure_upload(c, 1)) return rc;
  VK_HIP(hipMemcpy(c->upload, &id, sizeof id, hipMemcpyHostToDevice));
  VK_HIP(hipMemcpy(c->blob, bytes, bb, hipMemcpyHostToDevice));
  if (int rc = vapi_kv_import_blocks(&c->pool, c->upload, 1, c->blob, nullptr))
    return rc;
  VK_HIP(hipDeviceSynchronize());
  return 0;
}

// CandleBackend::copy_blocks (backend.rs:781-797): every pair, every layer,
// K and V, as one launch.
int vapi_cache_copy_blocks(vapi_cache* c, const uint32_t* pairs_host,
                           uint32_t n_pairs) {
  clear_error();
  if (!c) VK_FAIL(VAPI_KV_EINVAL, "vapi_cache_copy_blocks: null cache");
  if (n_pairs == 0) return 0;
  for (uint32_t i = 0; i < 2 * n_pairs; ++i)
    if (pairs_host[i] >= c->pool.num_blocks)
      VK_FAIL(VAPI_KV_EINVAL, "copy pair %u names block %u of %u", i / 2,
              pairs_host[i], c->pool.num_blocks);
  if (int rc = ensure_upload(c, 2 * (size_t)n_pairs)) return rc;
  VK_HIP(hipMemcpy(c->upload, pairs_host, 2 * sizeof(uint32_t) * n_pairs,
                   hipMemcpyHostToDevice));
  if (int rc = vapi_kv_copy_blocks(&c->pool, c->upload, n_pairs, nullptr)) return rc;
  VK_HIP(hipDeviceSynchronize());
  return 0;
}

// ForwardBatch::validate (crates/vapi-engine/src/backend.rs:96-204), with
// the token ids themselves omitted (they do not reach the KV path).
int vapi_forward_batch_validate(uint32_t n_tokens, const uint32_t* positions,
                                const uint32_t* slot_mapping,
                                const uint32_t* cu_q, const uint32_t* cu_k,
                                uint32_t batch, const uint32_t* table_offsets,
                                const uint32_t* table_data,
                                const uint32_t* logits_indices,
                                uint32_t n_logits, uint32_t num_blocks,
                                uint32_t block_size) {
  clear_error();
  if (block_size == 0) VK_FAIL(VAPI_KV_EINVAL, "block_size is 0");
  if (batch > 0 && cu_q[0] != 0)
    VK_FAIL(VAPI_KV_EINVAL, "cumulative lengths must start at 0");
  for (uint32_t i = 0; i < batch; ++i) {
    if (cu_q[i + 1] < cu_q[i])
      VK_FAIL(VAPI_KV_EINVAL, "cu_seqlens_q is not monotonic");
  }
  for (uint32_t i = 0; i < batch; ++i) {
    if (cu_k[i + 1] < cu_k[i])
      VK_FAIL(VAPI_KV_EINVAL, "cu_seqlens_k is not monotonic");
  }
  const uint32_t last = batch > 0 ? cu_q[batch] : 0;
  if (batch > 0 && last != n_tokens)
    VK_FAIL(VAPI_KV_EINVAL, "cu_seqlens_q ends at %u but there are %u tokens", last,
            n_tokens);
  for (uint32_t i = 0; i < batch; ++i) {
    const uint32_t q = cu_q[i + 1] - cu_q[i];
    const uint32_t k = cu_k[i + 1] - cu_k[i];
    if (q > k)
      VK_FAIL(VAPI_KV_EINVAL,
              "sequence %u has %u query tokens but only %u key tokens; a token "
              "cannot attend to fewer positions than it contributes",
              i, q, k);
    const uint32_t need = (k + block_size - 1) / block_size;
    const uint32_t have = table_offsets[i + 1] - table_offsets[i];
    if (have < need)
      VK_FAIL(VAPI_KV_EINVAL,
              "sequence %u needs %u blocks to cover %u keys but its table has %u",
              i, need, k, have);
    for (uint32_t t = table_offsets[i]; t < table_offsets[i + 1]; ++t)
      if (table_data[t] >= num_blocks)
        VK_FAIL(VAPI_KV_EINVAL, "sequence %u references block %u of %u", i,
                table_data[t], num_blocks);
    const uint32_t lo = cu_q[i];
    for (uint32_t j = lo + 1; j < lo + q; ++j)
      if (positions[j] != positions[j - 1] + 1)
        VK_FAIL(VAPI_KV_EINVAL,
                "sequence %u has non-contiguous positions at %u: %u then %u", i,
                j, positions[j - 1], positions[j]);
  }
  std::vector<uint32_t> slots(slot_mapping, slot_mapping + n_tokens);
  std::sort(slots.begin(), slots.end());
  for (size_t i = 1; i < slots.size(); ++i)
    if (slots[i] == slots[i - 1])
      VK_FAIL(VAPI_KV_EINVAL, "two tokens both write KV cache slot %u", slots[i]);
  if (!slots.empty() && (uint64_t)slots.back() >= (uint64_t)num_blocks * block_size)
    VK_FAIL(VAPI_KV_EINVAL, "slot %u is past the end of the cache", slots.back());
  for (uint32_t i = 0; i < n_logits; ++i)
    if (logits_indices[i] >= n_tokens)
      VK_FAIL(VAPI_KV_EINVAL, "logits index %u is past the end of the batch",
              logits_indices[i]);
  return 0;
}

// pack_block_tables (attention.rs:42-62).
int64_t vapi_pack_block_tables(uint32_t batch, const uint32_t* off,
                               const uint32_t* data, uint32_t* out,
                               size_t out_capacity) {
  clear_error();
  uint32_t width = 1;
  for (uint32_t i = 0; i < batch; ++i) width = std::max(width, off[i + 1] - off[i]);
  if ((size_t)batch * width > out_capacity)
    VK_FAIL(VAPI_KV_ESPACE, "packed table needs %zu entries, capacity %zu",
            (size_t)batch * width, out_capacity);
  for (uint32_t i = 0; i < batch; ++i) {
    const uint32_t n = off[i + 1] - off[i];
    const uint32_t pad = n ? data[off[i + 1] - 1] : 0;
    for (uint32_t j = 0; j < width; ++j)
      out[(size_t)i * width + j] = j < n ? data[off[i] + j] : pad;
  }
  return width;
}

}  // extern "C"
