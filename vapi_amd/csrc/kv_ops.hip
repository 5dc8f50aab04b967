// Data-movement kernels of the paged KV pool: append (slot_mapping scatter),
// block-table gather, copy-on-write block copy and spill export/import/swap.
//
// All of them are HBM-bound byte movers. Each thread moves ITEMS chunks of C
// bytes (C = 16 whenever the row size allows it, so every lane issues
// dwordx4 loads and stores); item indices are laid out so that consecutive
// lanes touch consecutive bytes of the contiguous side (source rows for
// append, destination blobs for export) and full head_dim rows of the paged
// side. Loads for all ITEMS are issued before any store.
#include <mutex>

#include "common.hpp"

namespace vk {

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
}
void clear_error() { g_err.clear(); }

int check_pool(const vapi_kv_pool* p, const char* who) {
  if (!p) VK_FAIL(VAPI_KV_EINVAL, "%s: null pool", who);
  if (dtype_size(p->dtype) == 0)
    VK_FAIL(VAPI_KV_EINVAL, "%s: unknown dtype %u", who, p->dtype);
  if (p->layout != VAPI_KV_LAYOUT_HND && p->layout != VAPI_KV_LAYOUT_NHD)
    VK_FAIL(VAPI_KV_EINVAL, "%s: unknown layout %u", who, p->layout);
  if (p->num_layers == 0 || p->block_size == 0 || p->num_kv_heads == 0 ||
      p->head_dim == 0)
    VK_FAIL(VAPI_KV_EINVAL,
            "%s: empty pool geometry (layers %u, block_size %u, kv_heads %u, "
            "head_dim %u)",
            who, p->num_layers, p->block_size, p->num_kv_heads, p->head_dim);
  if ((uint64_t)p->num_blocks * p->block_size >= 0xFFFFFFFFull)
    VK_FAIL(VAPI_KV_EINVAL, "%s: %u blocks of %u slots overflow u32 slots", who,
            p->num_blocks, p->block_size);
  const uint64_t block_bytes =
      (uint64_t)p->block_size * p->num_kv_heads * p->head_dim * dtype_size(p->dtype);
  if (p->block_stride_bytes == 0) {
    const uint64_t layer_bytes = (uint64_t)p->num_blocks * block_bytes;
    if (p->num_layers > 1 && p->layer_stride_bytes < layer_bytes)
      VK_FAIL(VAPI_KV_EINVAL, "%s: layer stride %llu < layer size %llu", who,
              (unsigned long long)p->layer_stride_bytes,
              (unsigned long long)layer_bytes);
  } else {
    // Block-major: a block's layers side by side, blocks apart by the stride.
    if (p->block_stride_bytes & 15)
      VK_FAIL(VAPI_KV_EINVAL, "%s: block stride %llu is not a multiple of 16 bytes", who,
              (unsigned long long)p->block_stride_bytes);
    if (p->num_layers > 1 && p->layer_stride_bytes < block_bytes)
      VK_FAIL(VAPI_KV_EINVAL, "%s: layer stride %llu < block size %llu", who,
              (unsigned long long)p->layer_stride_bytes, (unsigned long long)block_bytes);
    if (p->block_stride_bytes < (p->num_layers - 1) * p->layer_stride_bytes + block_bytes)
      VK_FAIL(VAPI_KV_EINVAL, "%s: block stride %llu < the %u layers' extent in a block", who,
              (unsigned long long)p->block_stride_bytes, p->num_layers);
  }
  if (p->num_blocks > 0 && !p->k) VK_FAIL(VAPI_KV_EINVAL, "%s: null K base pointer", who);
  // Every kernel moves 16-byte chunks of rows that start at these bases
  // (the attention kernels load 16 bytes per lane, also into LDS).
  if (((uintptr_t)p->k | (uintptr_t)p->v) & 15)
    VK_FAIL(VAPI_KV_EINVAL, "%s: K/V base pointers must be 16-byte aligned", who);
  if (p->num_layers > 1 && (p->layer_stride_bytes & 15))
    VK_FAIL(VAPI_KV_EINVAL, "%s: layer stride %llu is not a multiple of 16 bytes", who,
            (unsigned long long)p->layer_stride_bytes);
  // Further layer groups of the same cache (block-level calls walk them):
  // each is a pool of its own, on the same blocks.
  uint32_t links = 0;
  for (const vapi_kv_pool* q = p->next; q; q = q->next) {
    if (++links > kMaxPoolChain)
      VK_FAIL(VAPI_KV_EINVAL, "%s: more than %u chained pools (a cycle?)", who, kMaxPoolChain);
    if (q->num_blocks != p->num_blocks || q->block_size != p->block_size)
      VK_FAIL(VAPI_KV_EINVAL,
              "%s: chained pool %u has %u blocks of %u slots, the first %u of %u", who, links,
              q->num_blocks, q->block_size, p->num_blocks, p->block_size);
    vapi_kv_pool head = *q;
    head.next = nullptr;
    if (int rc = check_pool(&head, who)) return rc;
  }
  return 0;
}

// Bytes of one block in the K buffers (or V buffers) of a pool's layers.
static uint64_t pool_k_block_bytes(const vapi_kv_pool* p) {
  return (uint64_t)p->num_layers * p->block_size * p->num_kv_heads * p->head_dim *
         dtype_size(p->dtype);
}
static uint64_t pool_v_block_bytes(const vapi_kv_pool* p) {
  return p->v ? pool_k_block_bytes(p) : 0;
}

// ---- append ---------------------------------------------------------------

struct AppendArgs {
  const char* k_src;
  const char* v_src;
  char* k_dst;
  char* v_dst;
  const uint32_t* slots;
  uint32_t total;  // n_tokens * (2 or 1) * kvh * upr
  uint32_t num_slots;
  uint32_t has_v;  // 0: a K-only pool (kernel template kKV = false)
  FastDiv upr, kvh, bs;
  uint32_t row_bytes;  // head_dim * elt
  uint64_t blk_b, head_b, tok_b;  // byte strides
  uint64_t src_layer_b, dst_layer_b;  // layer strides (grid y = layer)
};

template <int C, int ITEMS, bool kStream, bool kKV, bool kLoadNT = false>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  using V = typename Chunk<C>::T;
  // Layer blockIdx.y of a multi-layer append (0 for one layer).
  const uint64_t ly = blockIdx.y;
  a.k_src += ly * a.src_layer_b;
  a.v_src += ly * a.src_layer_b;
  a.k_dst += ly * a.dst_layer_b;
  a.v_dst += ly * a.dst_layer_b;
  const uint32_t base = blockIdx.x * (256u * ITEMS) + threadIdx.x;
  V val[ITEMS];
  char* dst[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint32_t i = base + j * 256u;
    dst[j] = nullptr;
    if (i < a.total) {
      const uint32_t r = a.upr.div(i);
      const uint32_t u = i - r * a.upr.d;
      const uint32_t r2 = a.kvh.div(r);
      const uint32_t h = r - r2 * a.kvh.d;
      // kKV: K and V rows of a token interleave; else K only.
      const uint32_t kv = kKV ? r2 & 1u : 0u, t = kKV ? r2 >> 1 : r2;
      // The source row and the slot are loaded together (the source address
      // does not depend on the slot), so one memory round trip precedes the
      // store.
      const uint64_t src_off = ((uint64_t)t * a.kvh.d + h) * a.row_bytes + (uint64_t)u * C;
      const V* sp = (const V*)((kv ? a.v_src : a.k_src) + src_off);
      val[j] = kLoadNT ? load_stream(sp) : *sp;
      const uint32_t slot = a.slots[t];
      if (slot < a.num_slots) {  // VAPI_KV_SLOT_SKIP and out-of-range drop
        const uint32_t blk = a.bs.div(slot);
        const uint32_t off = slot - blk * a.bs.d;
        dst[j] = (kv ? a.v_dst : a.k_dst) + blk * a.blk_b + h * a.head_b +
                 off * a.tok_b + (uint64_t)u * C;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    if (dst[j]) {
      if (kStream) store_stream((V*)dst[j], val[j]);
      else *(V*)dst[j] = val[j];
    }
}

// A single-layer append moves two chunks per thread (both loads issued
// before either store). Config 1 replayed from a graph, sources warm (in
// the last-level cache, as the rows a projection just wrote are) / cold
// (rotated over 384 MB of sources): 1 chunk 4.1-4.2 / 9.2 us, 2 chunks
// 4.2-4.4 / 8.1 us, 4 chunks 4.8-4.9 / 8.9 us. Two chunks make the grid one
// wave of resident workgroups (2,048 of 256 threads, 8 per CU), so a cold
// source costs one HBM round trip per thread instead of two rounds of
// them. A multi-layer append already has layers times that grid and keeps
// one chunk per thread (4 layers: 21.2 us against 29.5 us with two).
template <int C>
static void launch_append(const AppendArgs& a, uint32_t layers, uint32_t flags, hipStream_t s) {
  if (!a.has_v) {
    const uint32_t grid = (a.total + 255) / 256;
    hipLaunchKernelGGL((kv_append_kernel<C, 1, false, false>), dim3(grid, layers), dim3(256),
                       0, s, a);
  } else if (layers == 1) {
    constexpr int ITEMS = 2;
    const uint32_t grid = (a.total + 256 * ITEMS - 1) / (256 * ITEMS);
    // A cold source (VAPI_APPEND_COLD_SOURCE) is read with streaming loads:
    // config 1 with its sources rotated over 384 MB, graph replays, two
    // boxes: 7.1-7.5 against 7.9-8.1 us; with a warm source they cost
    // 5.2-7.2 against 4.5-4.6 us. Ordinary stores with the streaming loads
    // measured the same cold and slower warm; 1 or 4 chunks per thread, and
    // lanes walking four tokens of one tile instead of four heads of one
    // token, slower.
    if (flags & VAPI_APPEND_COLD_SOURCE)
      hipLaunchKernelGGL((kv_append_kernel<C, ITEMS, true, true, true>), dim3(grid), dim3(256), 0,
                         s, a);
    else
      hipLaunchKernelGGL((kv_append_kernel<C, ITEMS, true, true>), dim3(grid), dim3(256), 0, s, a);
  } else {
    const uint32_t grid = (a.total + 255) / 256;
    hipLaunchKernelGGL((kv_append_kernel<C, 1, false, true>), dim3(grid, layers), dim3(256),
                       0, s, a);
  }
}

// ---- gather -----------------------------------------------------------------

struct GatherArgs {
  const char* k_src;
  const char* v_src;
  char* k_out;
  char* v_out;
  const uint32_t* table;
  uint32_t total;  // 2 * len_k * kvh * upr
  uint32_t len_k, num_blocks;
  FastDiv upr, kvh, bs, len;
  uint32_t row_bytes;
  uint64_t blk_b, head_b, tok_b;
};

// Item i -> (kv, token t, head h, chunk u), walked in the output's order.
// Streaming loads and stores: 8,192 keys of K and V (67 MB) in 9.8 us
// against 22.4 us with ordinary stores (walking an HND pool tile by tile instead measured the
// same either way).
template <int C, int ITEMS>
__global__ __launch_bounds__(256) void kv_gather_kernel(GatherArgs a) {
  using V = typename Chunk<C>::T;
  const uint32_t base = blockIdx.x * (256u * ITEMS) + threadIdx.x;
  V val[ITEMS];
  char* dst[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint32_t i = base + j * 256u;
    dst[j] = nullptr;
    if (i < a.total) {
      const uint32_t r = a.upr.div(i);
      const uint32_t u = i - r * a.upr.d;
      const uint32_t r2 = a.kvh.div(r);
      const uint32_t h = r - r2 * a.kvh.d;
      const uint32_t kv = a.len.div(r2);
      const uint32_t t = r2 - kv * a.len.d;
      char* out = kv ? a.v_out : a.k_out;
      if (out) {
        const uint32_t bi = a.bs.div(t);
        const uint32_t off = t - bi * a.bs.d;
        const uint32_t blk = a.table[bi];
        const char* src = (kv ? a.v_src : a.k_src) + blk * a.blk_b +
                          h * a.head_b + off * a.tok_b + (uint64_t)u * C;
        // A table entry past the pool reads nothing and gathers zeros.
        val[j] = blk < a.num_blocks ? load_stream((const V*)src) : V{};
        dst[j] = out + ((uint64_t)t * a.kvh.d + h) * a.row_bytes +
                 (uint64_t)u * C;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    if (dst[j]) store_stream((V*)dst[j], val[j]);
}

// ---- block copy ---------------------------------------------------------------

struct CopyArgs {
  char* k;
  char* v;
  const uint32_t* pairs;
  uint64_t layer_b, blk_b;
  uint32_t total;  // n_pairs * L * 2 * upb
  FastDiv upb, two_l;
  uint32_t num_layers, num_blocks;
};

// Streaming loads and stores (each byte is moved once). Measured on config
// 4a (3.76 GB, 28 layers): 5.0-5.1 TB/s, what a trivial copy of the same
// random 16 KiB runs reaches and 85% of a sequential copy of the same
// bytes; the order the runs are walked in, a persistent grid-stride
// variant and two runs per workgroup measured no better.
template <int C, int ITEMS, int NT>
__global__ __launch_bounds__(NT) void kv_copy_kernel(CopyArgs a) {
  using V = typename Chunk<C>::T;
  const uint32_t base = blockIdx.x * (NT * ITEMS) + threadIdx.x;
  V val[ITEMS];
  char* dst[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint32_t i = base + j * (uint32_t)NT;
    dst[j] = nullptr;
    if (i < a.total) {
      const uint32_t r = a.upb.div(i);
      const uint32_t u = i - r * a.upb.d;
      const uint32_t p = a.two_l.div(r);
      const uint32_t s = r - p * a.two_l.d;  // K layers, then V layers (if any)
      const uint32_t kv = s >= a.num_layers;
      const uint32_t layer = kv ? s - a.num_layers : s;
      const uint32_t src_blk = a.pairs[2 * p], dst_blk = a.pairs[2 * p + 1];
      char* buf = (kv ? a.v : a.k) + layer * a.layer_b;
      const uint64_t o = (uint64_t)u * C;
      if (src_blk < a.num_blocks && dst_blk < a.num_blocks) {  // else skipped
        val[j] = load_stream((const V*)(buf + src_blk * a.blk_b + o));
        dst[j] = buf + dst_blk * a.blk_b + o;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    if (dst[j]) store_stream((V*)dst[j], val[j]);
}

// A block-major pool whose blocks hold every layer's K and V contiguously
// (layer stride = one layer's block, V right after the K layers, block
// stride = all of them): a pair is one run of run_units 16-byte chunks.
// Workgroup w copies 64 chunks of run w / wgs_per_run.
struct CopyRunsArgs {
  char* base;
  const uint32_t* pairs;
  uint64_t run_b;       // block stride = run bytes
  uint32_t run_units;   // 16-byte chunks per run
  FastDiv wgs_per_run;
  uint32_t num_blocks;
};

__global__ __launch_bounds__(64) void kv_copy_runs_kernel(CopyRunsArgs a) {
  const uint32_t p = a.wgs_per_run.div(blockIdx.x);
  const uint32_t u = (blockIdx.x - p * a.wgs_per_run.d) * 64u + threadIdx.x;
  const uint32_t src_blk = a.pairs[2 * p], dst_blk = a.pairs[2 * p + 1];
  if (u >= a.run_units || src_blk >= a.num_blocks || dst_blk >= a.num_blocks) return;
  const uint4 x = load_stream((const uint4*)(a.base + src_blk * a.run_b) + u);
  store_stream((uint4*)(a.base + dst_blk * a.run_b) + u, x);
}

// ---- export / import (reference blob order) ----------------------------------

// Blob of block i: the K block of every layer of the cache in order, then
// the V block of every layer that has V, each NHD [bs, kvh, d]. One launch
// covers one pool of the chain: its segments s = 0..nbuf*L-1 (K layers, then
// V layers) sit at k_off + l*seg_bytes and v_off + l*seg_bytes of each blob.
// Item index = (((i*nbuf*L + s)*bs + t)*kvh + h)*upr + u, so a segment's blob
// side is walked contiguously.
struct BlobArgs {
  char* k;
  char* v;
  char* blob;
  const uint32_t* ids;
  uint64_t layer_b, blk_b, head_b, tok_b;
  uint64_t block_bytes;  // blob stride: one block of the whole pool chain
  uint64_t k_off, v_off; // this pool's first K and first V segment in a blob
  uint32_t total;
  FastDiv upr, kvh, bs, two_l;
  uint32_t num_layers, row_bytes, seg_bytes, num_blocks;
};

template <int C, int ITEMS, bool EXPORT>
__global__ __launch_bounds__(256) void kv_blob_kernel(BlobArgs a) {
  using V = typename Chunk<C>::T;
  const uint32_t base = blockIdx.x * (256u * ITEMS) + threadIdx.x;
  V val[ITEMS];
  char* dst[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint32_t i = base + j * 256u;
    dst[j] = nullptr;
    if (i < a.total) {
      const uint32_t r = a.upr.div(i);
      const uint32_t u = i - r * a.upr.d;
      const uint32_t r2 = a.kvh.div(r);
      const uint32_t h = r - r2 * a.kvh.d;
      const uint32_t r3 = a.bs.div(r2);
      const uint32_t t = r2 - r3 * a.bs.d;
      const uint32_t bi = a.two_l.div(r3);
      const uint32_t s = r3 - bi * a.two_l.d;
      const uint32_t kv = s >= a.num_layers;
      const uint32_t layer = kv ? s - a.num_layers : s;
      const uint32_t blk = a.ids[bi];
      if (blk >= a.num_blocks) continue;  // an id past the pool moves nothing
      char* pool = (kv ? a.v : a.k) + layer * a.layer_b + blk * a.blk_b +
                   h * a.head_b + t * a.tok_b + (uint64_t)u * C;
      char* blob = a.blob + bi * a.block_bytes + (kv ? a.v_off : a.k_off) +
                   (uint64_t)layer * a.seg_bytes +
                   ((uint64_t)t * a.kvh.d + h) * a.row_bytes + (uint64_t)u * C;
      if (EXPORT) {
        val[j] = load_stream((const V*)pool);
        dst[j] = blob;
      } else {
        val[j] = *(const V*)blob;
        dst[j] = pool;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    if (dst[j]) *(V*)dst[j] = val[j];
}

// Dispatch a kernel template over the chunk size chosen at runtime.
#define VK_DISPATCH_CHUNK(c, LAUNCH) \
  switch (c) {                       \
    case 16: LAUNCH(16); break;      \
    case 8: LAUNCH(8); break;        \
    case 4: LAUNCH(4); break;        \
    case 2: LAUNCH(2); break;        \
    default: LAUNCH(1); break;       \
  }

}  // namespace vk

using namespace vk;

extern "C" {

const char* vapi_kv_last_error(void) { return g_err.c_str(); }

const char* vapi_kv_version(void) { return "vapi_kv 0.1.0 gfx950"; }

size_t vapi_kv_block_bytes(const vapi_kv_pool* p) {
  size_t bytes = 0;
  uint32_t links = 0;
  for (; p && links <= kMaxPoolChain; p = p->next, ++links)
    bytes += pool_k_block_bytes(p) + pool_v_block_bytes(p);
  return bytes;
}

size_t vapi_kv_layer_bytes(const vapi_kv_pool* p) {
  if (!p) return 0;
  return (size_t)p->num_blocks * p->block_size * p->num_kv_heads *
         p->head_dim * dtype_size(p->dtype);
}

// One launch over layers [layer0, layer0 + n_layers): layer l's rows at
// k_src/v_src + (l - layer0) * src_layer_stride bytes.
static int append_impl(const char* who, const vapi_kv_pool* pool, uint32_t layer0,
                       uint32_t n_layers, const void* k_src, const void* v_src,
                       uint64_t src_layer_stride, const uint32_t* slot_mapping,
                       uint32_t n_tokens, uint32_t flags, vapi_stream_t stream) {
  if (int rc = check_pool(pool, who)) return rc;
  if (flags & ~VAPI_APPEND_COLD_SOURCE)
    VK_FAIL(VAPI_KV_EINVAL, "%s: unknown flags %#x", who, flags);
  if (n_layers == 0 || layer0 >= pool->num_layers || n_layers > pool->num_layers - layer0)
    VK_FAIL(VAPI_KV_EINVAL, "%s: layers %u..%u of %u", who, layer0, layer0 + n_layers,
            pool->num_layers);
  if (n_tokens == 0) return 0;
  const bool has_v = pool->v != nullptr;
  if (!has_v && v_src)
    VK_FAIL(VAPI_KV_EINVAL, "%s: V rows for a K-only pool (a rows layer stores K only)", who);
  if (!k_src || (has_v && !v_src) || !slot_mapping)
    VK_FAIL(VAPI_KV_EINVAL, "%s: null source or slot_mapping", who);
  if (n_layers > 65535) VK_FAIL(VAPI_KV_EUNSUP, "%s: %u layers in one call", who, n_layers);
  const Geom g = make_geom(pool);
  const uint32_t elt = dtype_size(pool->dtype);
  const uint32_t row_bytes = g.d * elt;
  if (n_layers > 1 && src_layer_stride < (uint64_t)n_tokens * g.kvh * row_bytes)
    VK_FAIL(VAPI_KV_EINVAL, "%s: source layer stride %llu < %u rows of %u heads", who,
            (unsigned long long)src_layer_stride, n_tokens, g.kvh);
  // Chunk size: the largest power of two up to 16 B that divides the row,
  // the source addresses and (several layers) both layer strides.
  int c = chunk_bytes_for(row_bytes);
  const uint64_t align = (uint64_t)(uintptr_t)k_src | (uint64_t)(uintptr_t)(has_v ? v_src : k_src) |
                         (n_layers > 1 ? src_layer_stride | pool->layer_stride_bytes : 0);
  while (c > 1 && align % c) c >>= 1;
  const uint64_t total = (uint64_t)n_tokens * (has_v ? 2 : 1) * g.kvh * (row_bytes / c);
  if (total >= (1ull << 31))
    VK_FAIL(VAPI_KV_EUNSUP, "%s: %u tokens is too many for one call", who, n_tokens);
  LayerPtrs lp = layer_ptrs(pool, layer0);
  AppendArgs a;
  a.k_src = (const char*)k_src;
  a.v_src = (const char*)(has_v ? v_src : k_src);
  a.k_dst = lp.k;
  a.v_dst = has_v ? lp.v : lp.k;
  a.has_v = has_v ? 1u : 0u;
  a.slots = slot_mapping;
  a.total = (uint32_t)total;
  a.num_slots = g.num_blocks * g.block_size;
  a.upr = FastDiv(row_bytes / c);
  a.kvh = FastDiv(g.kvh);
  a.bs = FastDiv(g.block_size);
  a.row_bytes = row_bytes;
  a.blk_b = g.blk * elt;
  a.head_b = g.head * elt;
  a.tok_b = g.tok * elt;
  a.src_layer_b = n_layers > 1 ? src_layer_stride : 0;
  a.dst_layer_b = n_layers > 1 ? pool->layer_stride_bytes : 0;
#define L_APPEND(C) launch_append<C>(a, n_layers, flags, hs(stream))
  VK_DISPATCH_CHUNK(c, L_APPEND)
#undef L_APPEND
  VK_LAUNCHED("kv_append");
  return 0;
}

int vapi_kv_append(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                   const void* v_src, const uint32_t* slot_mapping,
                   uint32_t n_tokens, vapi_stream_t stream) {
  return append_impl("vapi_kv_append", pool, layer, 1, k_src, v_src, 0, slot_mapping,
                     n_tokens, 0, stream);
}

int vapi_kv_append_ex(const vapi_kv_pool* pool, uint32_t layer, const void* k_src,
                      const void* v_src, const uint32_t* slot_mapping, uint32_t n_tokens,
                      uint32_t flags, vapi_stream_t stream) {
  return append_impl("vapi_kv_append_ex", pool, layer, 1, k_src, v_src, 0, slot_mapping,
                     n_tokens, flags, stream);
}

int vapi_kv_append_layers(const vapi_kv_pool* pool, uint32_t layer0, uint32_t n_layers,
                          const void* k_src, const void* v_src, uint64_t src_layer_stride,
                          const uint32_t* slot_mapping, uint32_t n_tokens,
                          vapi_stream_t stream) {
  return append_impl("vapi_kv_append_layers", pool, layer0, n_layers, k_src, v_src,
                     src_layer_stride, slot_mapping, n_tokens, 0, stream);
}

int vapi_kv_gather(const vapi_kv_pool* pool, uint32_t layer,
                   const uint32_t* block_table, uint32_t n_table,
                   uint32_t len_k, void* k_out, void* v_out,
                   vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_kv_gather")) return rc;
  if (layer >= pool->num_layers)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_gather: layer %u of %u", layer,
            pool->num_layers);
  if ((uint64_t)len_k > (uint64_t)n_table * pool->block_size)
    VK_FAIL(VAPI_KV_EINVAL,
            "vapi_kv_gather: len_k %u exceeds %u blocks of %u slots", len_k,
            n_table, pool->block_size);
  if (!pool->v && v_out)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_gather: V output for a K-only pool");
  if (len_k == 0 || (!k_out && !v_out)) return 0;
  if (!block_table)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_gather: null block_table");
  const Geom g = make_geom(pool);
  const uint32_t elt = dtype_size(pool->dtype);
  const uint32_t row_bytes = g.d * elt;
  const int c = chunk_bytes_for(row_bytes);
  const uint64_t total = (uint64_t)(pool->v ? 2 : 1) * len_k * g.kvh * (row_bytes / c);
  if (total >= (1ull << 31))
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_kv_gather: len_k %u too large", len_k);
  LayerPtrs lp = layer_ptrs(pool, layer);
  GatherArgs a;
  a.k_src = lp.k;
  a.v_src = lp.v;
  a.k_out = (char*)k_out;
  a.v_out = (char*)v_out;
  a.table = block_table;
  a.total = (uint32_t)total;
  a.len_k = len_k;
  a.num_blocks = pool->num_blocks;
  a.upr = FastDiv(row_bytes / c);
  a.kvh = FastDiv(g.kvh);
  a.bs = FastDiv(g.block_size);
  a.len = FastDiv(len_k);
  a.row_bytes = row_bytes;
  a.blk_b = g.blk * elt;
  a.head_b = g.head * elt;
  a.tok_b = g.tok * elt;
  // One chunk per thread: 8,192 keys 13.8-13.9 against 15.0-15.5 us with
  // four (two with 128 threads 14.7-14.9, one or two with 64 threads
  // 14.2-14.3; one box, runs alternated).
  constexpr int ITEMS = 1;
  const uint32_t grid = (a.total + 256 * ITEMS - 1) / (256 * ITEMS);
#define L_GATHER(C)                                                        \
  hipLaunchKernelGGL((kv_gather_kernel<C, ITEMS>), dim3(grid), dim3(256), 0, \
                     hs(stream), a)
  VK_DISPATCH_CHUNK(c, L_GATHER)
#undef L_GATHER
  VK_LAUNCHED("kv_gather");
  return 0;
}

// One pool of the chain: every layer's K and (if present) V block.
static int copy_pool(const vapi_kv_pool* pool, const uint32_t* pairs, uint32_t n_pairs,
                     hipStream_t stream) {
  const Geom g = make_geom(pool);
  const uint32_t elt = dtype_size(pool->dtype);
  const uint64_t blk_b = g.blk_elems * elt;  // one layer's block
  const int c = chunk_bytes_for(blk_b);
  const uint64_t upb = blk_b / c;
  const uint32_t nbuf = pool->v ? 2 : 1;
  const uint64_t per_pair = (uint64_t)pool->num_layers * nbuf * upb;
  if (per_pair >= (1ull << 31))
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_kv_copy_blocks: block too large");
  const uint32_t pairs_per_launch =
      (uint32_t)std::min<uint64_t>(n_pairs, ((1ull << 31) - 1) / per_pair);
  const uint64_t stride_b = g.blk * elt;
  const uint64_t run_b = (uint64_t)nbuf * pool->num_layers * blk_b;
  if (pool->block_stride_bytes == run_b && (pool->num_layers == 1 ||
                                            pool->layer_stride_bytes == blk_b) &&
      (!pool->v || (const char*)pool->v == (const char*)pool->k + pool->num_layers * blk_b) &&
      run_b % 16 == 0 && run_b / 16 < (1ull << 31)) {
    // Each pair is one contiguous run (config 4 at block-major: 6.2 TB/s
    // against 5.1 TB/s for its 56 runs of 16 KiB in a layer-major pool).
    CopyRunsArgs r;
    r.base = (char*)pool->k;
    r.run_b = run_b;
    r.run_units = (uint32_t)(run_b / 16);
    const uint32_t wpr = (r.run_units + 63) / 64;
    r.wgs_per_run = FastDiv(wpr);
    r.num_blocks = pool->num_blocks;
    // FastDiv is exact below 2^31: at most that many workgroups per launch.
    const uint32_t per_launch = (uint32_t)std::min<uint64_t>(n_pairs, 0x7FFFFFFFull / wpr);
    for (uint32_t p0 = 0; p0 < n_pairs; p0 += per_launch) {
      const uint32_t np = std::min(per_launch, n_pairs - p0);
      r.pairs = pairs + 2ull * p0;
      hipLaunchKernelGGL(kv_copy_runs_kernel, dim3(np * wpr), dim3(64), 0, stream, r);
      VK_LAUNCHED("kv_copy_blocks");
    }
    return 0;
  }
  CopyArgs a;
  a.k = (char*)pool->k;
  a.v = (char*)pool->v;
  a.layer_b = pool->layer_stride_bytes;
  a.blk_b = stride_b;  // block stride
  a.upb = FastDiv((uint32_t)upb);
  a.two_l = FastDiv(nbuf * pool->num_layers);  // segment s >= num_layers is V
  a.num_layers = pool->num_layers;
  a.num_blocks = pool->num_blocks;
  // One chunk per thread in workgroups of 64: a block-major pool's pairs
  // (917,504-byte runs at config 4's shape) copy at 6.42 against 5.24 TB/s
  // with four chunks per thread in workgroups of 256; config 4's 16 KiB
  // runs of a layer-major pool copy the same either way (5.0-5.1 TB/s).
  constexpr int ITEMS = 1, NT = 64;
  for (uint32_t p0 = 0; p0 < n_pairs; p0 += pairs_per_launch) {
    const uint32_t np = std::min(pairs_per_launch, n_pairs - p0);
    a.pairs = pairs + 2ull * p0;
    a.total = (uint32_t)(np * per_pair);
    const uint32_t grid = (a.total + NT * ITEMS - 1) / (NT * ITEMS);
#define L_COPY(C)                                                            \
  hipLaunchKernelGGL((kv_copy_kernel<C, ITEMS, NT>), dim3(grid), dim3(NT), 0, \
                     stream, a)
    VK_DISPATCH_CHUNK(c, L_COPY)
#undef L_COPY
    VK_LAUNCHED("kv_copy_blocks");
  }
  return 0;
}

int vapi_kv_copy_blocks(const vapi_kv_pool* pool, const uint32_t* pairs,
                        uint32_t n_pairs, vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_kv_copy_blocks")) return rc;
  if (n_pairs == 0) return 0;
  if (!pairs) VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_copy_blocks: null pairs");
  for (const vapi_kv_pool* p = pool; p; p = p->next)
    if (int rc = copy_pool(p, pairs, n_pairs, hs(stream))) return rc;
  return 0;
}

static int blob_pool(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n, char* blob,
                     uint64_t blob_stride, uint64_t k_off, uint64_t v_off, bool do_export,
                     hipStream_t stream, const char* who) {
  const Geom g = make_geom(pool);
  const uint32_t elt = dtype_size(pool->dtype);
  const uint32_t row_bytes = g.d * elt;
  const int c = chunk_bytes_for(row_bytes);
  const uint32_t nbuf = pool->v ? 2 : 1;
  const uint64_t per_block = (uint64_t)nbuf * pool->num_layers * g.block_size *
                             g.kvh * (row_bytes / c);
  if (per_block >= (1ull << 31))
    VK_FAIL(VAPI_KV_EUNSUP, "%s: block too large", who);
  const uint32_t blocks_per_launch =
      (uint32_t)std::min<uint64_t>(n, ((1ull << 31) - 1) / per_block);
  BlobArgs a;
  a.k = (char*)pool->k;
  a.v = (char*)pool->v;
  a.layer_b = pool->layer_stride_bytes;
  a.blk_b = g.blk * elt;
  a.head_b = g.head * elt;
  a.tok_b = g.tok * elt;
  a.block_bytes = blob_stride;
  a.k_off = k_off;
  a.v_off = v_off;
  a.upr = FastDiv(row_bytes / c);
  a.kvh = FastDiv(g.kvh);
  a.bs = FastDiv(g.block_size);
  a.two_l = FastDiv(nbuf * pool->num_layers);
  a.num_layers = pool->num_layers;
  a.row_bytes = row_bytes;
  a.seg_bytes = (uint32_t)(g.blk_elems * elt);
  a.num_blocks = pool->num_blocks;
  constexpr int ITEMS = 4;
  for (uint32_t b0 = 0; b0 < n; b0 += blocks_per_launch) {
    const uint32_t nb = std::min(blocks_per_launch, n - b0);
    a.ids = ids + b0;
    a.blob = blob + (uint64_t)b0 * blob_stride;
    a.total = (uint32_t)(nb * per_block);
    const uint32_t grid = (a.total + 256 * ITEMS - 1) / (256 * ITEMS);
    if (do_export) {
#define L_EXP(C)                                                               \
  hipLaunchKernelGGL((kv_blob_kernel<C, ITEMS, true>), dim3(grid), dim3(256), \
                     0, stream, a)
      VK_DISPATCH_CHUNK(c, L_EXP)
#undef L_EXP
    } else {
#define L_IMP(C)                                                                \
  hipLaunchKernelGGL((kv_blob_kernel<C, ITEMS, false>), dim3(grid), dim3(256), \
                     0, stream, a)
      VK_DISPATCH_CHUNK(c, L_IMP)
#undef L_IMP
    }
    VK_LAUNCHED(who);
  }
  return 0;
}

// Export or import over the whole pool chain: one launch per pool, each
// placing its segments at their offsets in the blob (backend.rs:718-773
// order: K of every layer, then V of every layer with V).
static int blob_move(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n,
                     char* blob, bool do_export, hipStream_t stream,
                     const char* who) {
  if (int rc = check_pool(pool, who)) return rc;
  if (n == 0) return 0;
  if (!ids || !blob) VK_FAIL(VAPI_KV_EINVAL, "%s: null ids or buffer", who);
  const uint64_t stride = vapi_kv_block_bytes(pool);
  uint64_t k_off = 0, v_off = 0;
  for (const vapi_kv_pool* p = pool; p; p = p->next) v_off += pool_k_block_bytes(p);
  for (const vapi_kv_pool* p = pool; p; p = p->next) {
    if (int rc = blob_pool(p, ids, n, blob, stride, k_off, v_off, do_export, stream, who))
      return rc;
    k_off += pool_k_block_bytes(p);
    v_off += pool_v_block_bytes(p);
  }
  return 0;
}

int vapi_kv_export_blocks(const vapi_kv_pool* pool, const uint32_t* ids,
                          uint32_t n, void* dst, vapi_stream_t stream) {
  return blob_move(pool, ids, n, (char*)dst, true, hs(stream),
                   "vapi_kv_export_blocks");
}

int vapi_kv_import_blocks(const vapi_kv_pool* pool, const uint32_t* ids,
                          uint32_t n, const void* src, vapi_stream_t stream) {
  return blob_move(pool, ids, n, (char*)src, false, hs(stream),
                   "vapi_kv_import_blocks");
}

int vapi_kv_swap_out(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n,
                     void* host_dst, void* staging, size_t staging_bytes,
                     vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_kv_swap_out")) return rc;
  const size_t bb = vapi_kv_block_bytes(pool);
  if (n == 0) return 0;
  if (!host_dst || !staging)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_swap_out: null host or staging buffer");
  const size_t per = staging_bytes / bb;
  if (per == 0)
    VK_FAIL(VAPI_KV_ESPACE, "vapi_kv_swap_out: staging %zu bytes < one block (%zu)",
            staging_bytes, bb);
  for (uint32_t b0 = 0; b0 < n; b0 += (uint32_t)per) {
    const uint32_t nb = (uint32_t)std::min<size_t>(per, n - b0);
    if (int rc = vapi_kv_export_blocks(pool, ids + b0, nb, staging, stream))
      return rc;
    VK_HIP(hipMemcpyAsync((char*)host_dst + (size_t)b0 * bb, staging,
                          (size_t)nb * bb, hipMemcpyDeviceToHost, hs(stream)));
  }
  return 0;
}

int vapi_kv_swap_in(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n,
                    const void* host_src, void* staging, size_t staging_bytes,
                    vapi_stream_t stream) {
  if (int rc = check_pool(pool, "vapi_kv_swap_in")) return rc;
  const size_t bb = vapi_kv_block_bytes(pool);
  if (n == 0) return 0;
  if (!host_src || !staging)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_kv_swap_in: null host or staging buffer");
  const size_t per = staging_bytes / bb;
  if (per == 0)
    VK_FAIL(VAPI_KV_ESPACE, "vapi_kv_swap_in: staging %zu bytes < one block (%zu)",
            staging_bytes, bb);
  for (uint32_t b0 = 0; b0 < n; b0 += (uint32_t)per) {
    const uint32_t nb = (uint32_t)std::min<size_t>(per, n - b0);
    VK_HIP(hipMemcpyAsync(staging, (const char*)host_src + (size_t)b0 * bb,
                          (size_t)nb * bb, hipMemcpyHostToDevice, hs(stream)));
    if (int rc = vapi_kv_import_blocks(pool, ids + b0, nb, staging, stream))
      return rc;
  }
  return 0;
}

}  // extern "C"
