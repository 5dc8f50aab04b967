/*
 * vapi_kv.hpp — C++17 host-side mirror of the reference backend's paged-KV
 * interface, over the C ABI in vapi_kv.h.
 *
 * The reference is Rust: its backend crate (crates/vapi-backend-candle) owns
 * the paged cache and implements the engine's ExecutionBackend block methods
 * (crates/vapi-engine/src/backend.rs:301-368). This header is the same
 * surface in C++, for a host that links libvapi_kv.so directly:
 *
 *   vapi::Result / vapi::Error       vapi_core::Result, Error::Engine
 *   vapi::ForwardBatch (+ validate)  crates/vapi-engine/src/backend.rs:47-204
 *   vapi::LayerLayout, PagedKvCache  crates/vapi-backend-candle/src/cache.rs:12-118
 *   write_kv_to_cache / write_k_to_cache / gather_kv   cache.rs:136-159, 283-290
 *   pack_block_tables, cu_seqlens    attention.rs:42-71
 *   PreparedAttention, paged_attention[_prepared|_windowed]  attention.rs:165-288
 *   HipBackend::{num_blocks, block_bytes, export_block, import_block,
 *                copy_blocks}        backend.rs:339-367 as CandleBackend
 *                                    implements them (candle backend.rs:695-797)
 *   fork_copy_pairs                  the copy pairs of Scheduler::fork
 *                                    (crates/vapi-engine/src/scheduler.rs:217-281)
 *
 * Errors are values, never exceptions (shape, dtype and range violations are
 * errors, as cache.rs:438-445 tests). Tensors are device buffers with a
 * shape and a dtype; the helpers that build them from host vectors or read
 * them back synchronise, as the reference's Tensor::from_vec / to_vec do.
 * The per-layer calls take a stream and do not allocate beyond their small
 * per-call uploads (slot mappings); a serving loop that must not allocate
 * uses the C ABI with persistent buffers instead (PreparedAttention here
 * uploads once per step, as its reference does).
 *
 * Host code only: include with hipcc or any C++17 compiler that sees the
 * HIP runtime headers (define __HIP_PLATFORM_AMD__), link libvapi_kv.so and
 * libamdhip64.so.
 */
#ifndef VAPI_KV_HPP
#define VAPI_KV_HPP

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "vapi_kv.h"

namespace vapi {

// ---- Result ---------------------------------------------------------------

/* vapi_core::Error::Engine(String): the message of a failed call. */
struct Error {
  std::string message;
};

/* vapi_core::Result<T>: a value or an Error. */
template <class T>
class [[nodiscard]] Result {
 public:
  Result(T value) : value_(std::move(value)) {}
  Result(Error error) : error_(std::move(error)) {}
  bool is_ok() const { return value_.has_value(); }
  bool is_err() const { return !value_.has_value(); }
  T& value() { return *value_; }
  const T& value() const { return *value_; }
  const Error& error() const { return error_; }

 private:
  std::optional<T> value_;
  Error error_;
};

template <>
class [[nodiscard]] Result<void> {
 public:
  Result() = default;
  Result(Error error) : ok_(false), error_(std::move(error)) {}
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  const Error& error() const { return error_; }

 private:
  bool ok_ = true;
  Error error_;
};

inline Result<void> ok() { return {}; }
inline Error engine_err(std::string message) { return Error{std::move(message)}; }

namespace detail {
/* A C ABI status as a Result, with the library's message. */
inline Result<void> check(int rc) {
  if (rc == VAPI_KV_OK) return ok();
  return engine_err(vapi_kv_last_error());
}
inline Result<void> hip(hipError_t rc, const char* what) {
  if (rc == hipSuccess) return ok();
  return engine_err(std::string(what) + ": " + hipGetErrorString(rc));
}
#define VAPI_TRY(expr)                                 \
  do {                                                 \
    auto vapi_try_r_ = (expr);                         \
    if (vapi_try_r_.is_err()) return vapi_try_r_.error(); \
  } while (0)

struct HipFree {
  void operator()(void* p) const {
    if (p) (void)hipFree(p);
  }
};
using DevicePtr = std::unique_ptr<void, HipFree>;

inline Result<DevicePtr> device_alloc(size_t bytes) {
  void* p = nullptr;
  if (bytes) VAPI_TRY(hip(hipMalloc(&p, bytes), "hipMalloc"));
  return DevicePtr(p);
}

/* Round to nearest even, as the device kernels convert. */
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
inline float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint16_t f32_to_f16(float f) {
  const _Float16 h = (_Float16)f;
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}
inline float f16_to_f32(uint16_t u) {
  _Float16 h;
  std::memcpy(&h, &u, 2);
  return (float)h;
}
}  // namespace detail

// ---- dtypes and tensors ---------------------------------------------------

enum class DType : uint32_t { F32 = VAPI_KV_F32, F16 = VAPI_KV_F16, BF16 = VAPI_KV_BF16 };

inline size_t dtype_size(DType d) { return d == DType::F32 ? 4 : 2; }

/* A dense device tensor: dims, dtype and a shared device buffer. */
class Tensor {
 public:
  Tensor() = default;

  static Result<Tensor> zeros(std::vector<size_t> dims, DType dtype) {
    Tensor t;
    t.dims_ = std::move(dims);
    t.dtype_ = dtype;
    auto buf = detail::device_alloc(t.bytes());
    if (buf.is_err()) return buf.error();
    t.buf_ = std::shared_ptr<void>(buf.value().release(), detail::HipFree());
    if (t.bytes()) VAPI_TRY(detail::hip(hipMemset(t.buf_.get(), 0, t.bytes()), "hipMemset"));
    return t;
  }

  /* Tensor::from_vec: host f32 values, stored as `dtype`. */
  static Result<Tensor> from_vec(const std::vector<float>& values, std::vector<size_t> dims,
                                 DType dtype) {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    if (n != values.size())
      return engine_err("from_vec: " + std::to_string(values.size()) + " values for " +
                        std::to_string(n) + " elements");
    auto t = zeros(std::move(dims), dtype);
    if (t.is_err()) return t;
    std::vector<uint8_t> host(t.value().bytes());
    for (size_t i = 0; i < n; ++i) {
      if (dtype == DType::F32) {
        std::memcpy(host.data() + 4 * i, &values[i], 4);
      } else {
        const uint16_t h =
            dtype == DType::BF16 ? detail::f32_to_bf16(values[i]) : detail::f32_to_f16(values[i]);
        std::memcpy(host.data() + 2 * i, &h, 2);
      }
    }
    if (!host.empty())
      VAPI_TRY(detail::hip(hipMemcpy(t.value().data(), host.data(), host.size(),
                                     hipMemcpyHostToDevice),
                           "hipMemcpy"));
    return t;
  }

  /* The elements as f32 on the host (synchronous). */
  Result<std::vector<float>> to_vec_f32() const {
    std::vector<uint8_t> host(bytes());
    if (!host.empty())
      VAPI_TRY(detail::hip(hipMemcpy(host.data(), data(), host.size(), hipMemcpyDeviceToHost),
                           "hipMemcpy"));
    std::vector<float> out(numel());
    for (size_t i = 0; i < out.size(); ++i) {
      if (dtype_ == DType::F32) {
        std::memcpy(&out[i], host.data() + 4 * i, 4);
      } else {
        uint16_t h;
        std::memcpy(&h, host.data() + 2 * i, 2);
        out[i] = dtype_ == DType::BF16 ? detail::bf16_to_f32(h) : detail::f16_to_f32(h);
      }
    }
    return out;
  }

  const std::vector<size_t>& dims() const { return dims_; }
  DType dtype() const { return dtype_; }
  size_t numel() const {
    size_t n = 1;
    for (size_t d : dims_) n *= d;
    return dims_.empty() ? 0 : n;
  }
  size_t bytes() const { return numel() * dtype_size(dtype_); }
  void* data() const { return buf_.get(); }

 private:
  std::vector<size_t> dims_;
  DType dtype_ = DType::F32;
  std::shared_ptr<void> buf_;
};

inline std::string dims_str(const std::vector<size_t>& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) s += (i ? ", " : "") + std::to_string(d[i]);
  return s + "]";
}

// ---- the paged cache --------------------------------------------------------

/* What one layer stores per token (cache.rs:22-44). */
struct LayerLayout {
  enum class Kind { Kv, Rows } kind = Kind::Kv;
  size_t num_kv_heads = 0, head_dim = 0, width = 0;

  static LayerLayout Kv(size_t num_kv_heads, size_t head_dim) {
    return {Kind::Kv, num_kv_heads, head_dim, 0};
  }
  static LayerLayout Rows(size_t width) { return {Kind::Rows, 0, 0, width}; }
  size_t elems_per_token() const {
    return kind == Kind::Kv ? 2 * num_kv_heads * head_dim : width;
  }
  bool operator==(const LayerLayout& o) const {
    return kind == o.kind && num_kv_heads == o.num_kv_heads && head_dim == o.head_dim &&
           width == o.width;
  }
};

/* How a layer's blocks sit in memory (vapi_kv_layout): HND keeps each
 * (block, head) contiguous (the MI355X default); NHD is the reference's own
 * [blocks, block_size, heads, head_dim]. */
enum class MemoryLayout : uint32_t { HND = VAPI_KV_LAYOUT_HND, NHD = VAPI_KV_LAYOUT_NHD };

/*
 * PagedKvCache (cache.rs:12-118): every layer's K and V blocks. Layers with
 * the same layout run together in one device allocation, described by one
 * vapi_kv_pool; the pools are chained in layer order, so the block calls
 * (export/import/copy) walk every layer in the reference's order. Move-only:
 * the pool descriptors point at each other. block_major: each run's
 * allocation holds, per block, every layer's K block then every layer's V
 * block (vapi_kv_pool.block_stride_bytes), so a copy-on-write pair is one
 * contiguous run; blocks must then be a multiple of 16 bytes.
 */
class PagedKvCache {
 public:
  static Result<PagedKvCache> create(size_t num_layers, size_t num_blocks, size_t block_size,
                                     size_t num_kv_heads, size_t head_dim, DType dtype,
                                     MemoryLayout layout = MemoryLayout::HND,
                                     bool block_major = false) {
    return with_layouts(std::vector<LayerLayout>(num_layers,
                                                 LayerLayout::Kv(num_kv_heads, head_dim)),
                        num_blocks, block_size, dtype, layout, block_major);
  }

  static Result<PagedKvCache> with_layouts(const std::vector<LayerLayout>& layouts,
                                           size_t num_blocks, size_t block_size, DType dtype,
                                           MemoryLayout layout = MemoryLayout::HND,
                                           bool block_major = false) {
    PagedKvCache c;
    c.layouts_ = layouts;
    c.num_blocks_ = num_blocks;
    c.block_size_ = block_size;
    c.dtype_ = dtype;
    // Runs of alike layers.
    std::vector<std::pair<size_t, size_t>> runs;  // (first layer, count)
    for (size_t l = 0; l < layouts.size(); ++l) {
      if (!runs.empty() && layouts[runs.back().first] == layouts[l])
        ++runs.back().second;
      else
        runs.push_back({l, 1});
    }
    c.n_pools_ = runs.size();
    c.pools_.reset(new vapi_kv_pool[std::max<size_t>(runs.size(), 1)]);
    for (size_t p = 0; p < runs.size(); ++p) {
      const LayerLayout& ll = layouts[runs[p].first];
      const bool rows = ll.kind == LayerLayout::Kind::Rows;
      const size_t heads = rows ? 1 : ll.num_kv_heads, d = rows ? ll.width : ll.head_dim;
      const size_t block = block_size * heads * d * dtype_size(dtype);
      const size_t tensor = num_blocks * block;
      const size_t stride = (tensor + 255) / 256 * 256;  // 16-byte alignment and more
      const size_t per_layer = stride * (rows ? 1 : 2);
      if (block_major && block % 16)
        return Error{"a block-major cache needs blocks of a multiple of 16 bytes"};
      // Layer-major: per layer a K then a V buffer. Block-major: per block,
      // the run's K blocks then its V blocks.
      const size_t run_blocks = runs[p].second * (rows ? 1 : 2);
      const size_t bytes = block_major ? num_blocks * block * run_blocks
                                       : per_layer * runs[p].second;
      auto buf = detail::device_alloc(bytes);
      if (buf.is_err()) return buf.error();
      char* base = (char*)buf.value().get();
      if (bytes) VAPI_TRY(detail::hip(hipMemset(base, 0, bytes), "hipMemset"));
      vapi_kv_pool& pool = c.pools_[p];
      std::memset(&pool, 0, sizeof pool);
      pool.k = base;
      if (block_major) {
        pool.v = rows ? nullptr : base + runs[p].second * block;
        pool.layer_stride_bytes = block;
        pool.block_stride_bytes = block * run_blocks;
      } else {
        pool.v = rows ? nullptr : base + stride;
        pool.layer_stride_bytes = per_layer;
      }
      pool.num_layers = (uint32_t)runs[p].second;
      pool.num_blocks = (uint32_t)num_blocks;
      pool.block_size = (uint32_t)block_size;
      pool.num_kv_heads = (uint32_t)heads;
      pool.head_dim = (uint32_t)d;
      pool.dtype = (uint32_t)dtype;
      pool.layout = (uint32_t)layout;
      pool.next = nullptr;
      if (p) c.pools_[p - 1].next = &pool;
      c.buffers_.push_back(std::move(buf.value()));
      for (size_t i = 0; i < runs[p].second; ++i) c.layer_pool_.push_back({p, (uint32_t)i});
    }
    return std::move(c);
  }

  /* Elements per token across all layers, for sizing (cache.rs:109-111). */
  static size_t elems_per_token(const std::vector<LayerLayout>& layouts) {
    size_t n = 0;
    for (const auto& l : layouts) n += l.elems_per_token();
    return n;
  }

  /* Flat slot count, the addressing of ForwardBatch::slot_mapping. */
  size_t num_slots() const { return num_blocks_ * block_size_; }
  size_t num_blocks() const { return num_blocks_; }
  size_t block_size() const { return block_size_; }
  size_t num_layers() const { return layouts_.size(); }
  DType dtype() const { return dtype_; }
  const LayerLayout& layout(size_t layer) const { return layouts_[layer]; }

  /* The pool holding `layer` and the layer's index within it. */
  const vapi_kv_pool* pool_of(size_t layer, uint32_t* layer_in_pool) const {
    *layer_in_pool = layer_pool_[layer].second;
    return &pools_[layer_pool_[layer].first];
  }
  /* The head of the pool chain (every layer), for the block calls. */
  const vapi_kv_pool* chain() const { return n_pools_ ? &pools_[0] : nullptr; }

 private:
  std::vector<LayerLayout> layouts_;
  size_t num_blocks_ = 0, block_size_ = 0, n_pools_ = 0;
  DType dtype_ = DType::F32;
  std::unique_ptr<vapi_kv_pool[]> pools_;
  std::vector<detail::DevicePtr> buffers_;
  std::vector<std::pair<size_t, uint32_t>> layer_pool_;
};

namespace detail {
/* The checks write_rows makes (cache.rs:217-278), then the append. */
inline Result<void> append_rows(const PagedKvCache& cache, size_t layer, const Tensor& k,
                                const Tensor* v, const std::vector<uint32_t>& slot_mapping,
                                hipStream_t stream) {
  if (layer >= cache.num_layers())
    return engine_err("layer " + std::to_string(layer) + " of " +
                      std::to_string(cache.num_layers()));
  const LayerLayout& ll = cache.layout(layer);
  const bool rows = ll.kind == LayerLayout::Kind::Rows;
  if (rows != (v == nullptr))
    return engine_err(rows ? "a Rows layer stores K only" : "a Kv layer needs K and V");
  const std::vector<size_t> want = {slot_mapping.size(), rows ? 1 : ll.num_kv_heads,
                                    rows ? ll.width : ll.head_dim};
  if (k.dims().size() != 3 || k.dims()[1] != want[1] || k.dims()[2] != want[2])
    return engine_err("rows " + dims_str(k.dims()) + " do not match the cache row " +
                      dims_str({want[1], want[2]}));
  if (k.dims()[0] != slot_mapping.size())
    return engine_err(std::to_string(k.dims()[0]) + " rows for " +
                      std::to_string(slot_mapping.size()) + " slots");
  if (k.dtype() != cache.dtype() || (v && v->dtype() != cache.dtype()))
    return engine_err("rows dtype differs from the cache dtype");
  for (uint32_t s : slot_mapping)
    if (s != VAPI_KV_SLOT_SKIP && s >= cache.num_slots())
      return engine_err("slot " + std::to_string(s) + " is past the cache's " +
                        std::to_string(cache.num_slots()) + " slots");
  if (slot_mapping.empty()) return ok();
  auto slots = device_alloc(slot_mapping.size() * 4);
  if (slots.is_err()) return slots.error();
  VAPI_TRY(hip(hipMemcpyAsync(slots.value().get(), slot_mapping.data(), slot_mapping.size() * 4,
                              hipMemcpyHostToDevice, stream),
               "hipMemcpyAsync"));
  uint32_t lp = 0;
  const vapi_kv_pool* pool = cache.pool_of(layer, &lp);
  VAPI_TRY(check(vapi_kv_append(pool, lp, k.data(), v ? v->data() : nullptr,
                                (const uint32_t*)slots.value().get(),
                                (uint32_t)slot_mapping.size(), (vapi_stream_t)stream)));
  // The slot upload is freed on return: wait for the append that reads it.
  return hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
}
}  // namespace detail

/* write_kv_to_cache (cache.rs:136-148): k and v [n_tokens, kvh, d]; token i
 * lands at slot_mapping[i] (VAPI_KV_SLOT_SKIP writes nothing). */
inline Result<void> write_kv_to_cache(const PagedKvCache& cache, size_t layer, const Tensor& k,
                                      const Tensor& v, const std::vector<uint32_t>& slot_mapping,
                                      hipStream_t stream = nullptr) {
  if (v.dims() != k.dims())
    return engine_err("k " + dims_str(k.dims()) + " and v " + dims_str(v.dims()) +
                      " differ in shape");
  return detail::append_rows(cache, layer, k, &v, slot_mapping, stream);
}

/* write_k_to_cache (cache.rs:150-159): a Rows layer, rows [n_tokens, 1, width]. */
inline Result<void> write_k_to_cache(const PagedKvCache& cache, size_t layer, const Tensor& rows,
                                     const std::vector<uint32_t>& slot_mapping,
                                     hipStream_t stream = nullptr) {
  return detail::append_rows(cache, layer, rows, nullptr, slot_mapping, stream);
}

enum class Which { K, V };

/* gather_kv (cache.rs:283-290): the layer's K (or V) of one sequence in
 * logical order, [len_k, kvh, d]. */
inline Result<Tensor> gather_kv(const PagedKvCache& cache, size_t layer, Which which,
                                const std::vector<uint32_t>& table, size_t len_k) {
  if (layer >= cache.num_layers()) return engine_err("layer out of range");
  const LayerLayout& ll = cache.layout(layer);
  const bool rows = ll.kind == LayerLayout::Kind::Rows;
  if (rows && which == Which::V) return engine_err("a Rows layer has no V");
  if (table.size() * cache.block_size() < len_k)
    return engine_err("the table covers " + std::to_string(table.size() * cache.block_size()) +
                      " keys, not " + std::to_string(len_k));
  auto out = Tensor::zeros({len_k, rows ? 1 : ll.num_kv_heads, rows ? ll.width : ll.head_dim},
                           cache.dtype());
  if (out.is_err() || len_k == 0) return out;
  auto tab = detail::device_alloc(table.size() * 4);
  if (tab.is_err()) return tab.error();
  VAPI_TRY(detail::hip(hipMemcpy(tab.value().get(), table.data(), table.size() * 4,
                                 hipMemcpyHostToDevice),
                       "hipMemcpy"));
  uint32_t lp = 0;
  const vapi_kv_pool* pool = cache.pool_of(layer, &lp);
  void* k_out = which == Which::K ? out.value().data() : nullptr;
  void* v_out = which == Which::V ? out.value().data() : nullptr;
  VAPI_TRY(detail::check(vapi_kv_gather(pool, lp, (const uint32_t*)tab.value().get(),
                                        (uint32_t)table.size(), (uint32_t)len_k, k_out, v_out,
                                        nullptr)));
  VAPI_TRY(detail::hip(hipDeviceSynchronize(), "hipDeviceSynchronize"));
  return out;
}

// ---- the step descriptor ---------------------------------------------------

/* ForwardBatch (crates/vapi-engine/src/backend.rs:47-94). */
struct ForwardBatch {
  std::vector<uint32_t> tokens, positions, cu_seqlens_q, cu_seqlens_k, slot_mapping;
  std::vector<std::vector<uint32_t>> block_tables;
  std::vector<uint32_t> logits_indices;
  size_t max_seqlen_q = 0, max_seqlen_k = 0;

  size_t batch_size() const { return cu_seqlens_q.empty() ? 0 : cu_seqlens_q.size() - 1; }
  size_t num_tokens() const { return tokens.size(); }
  bool is_empty() const { return tokens.empty(); }

  /* ForwardBatch::validate (backend.rs:96-204), with its messages. */
  Result<void> validate(size_t num_blocks, size_t block_size) const {
    if (tokens.size() != positions.size())
      return engine_err("tokens (" + std::to_string(tokens.size()) + ") and positions (" +
                        std::to_string(positions.size()) + ") disagree");
    if (tokens.size() != slot_mapping.size())
      return engine_err("tokens (" + std::to_string(tokens.size()) + ") and slot_mapping (" +
                        std::to_string(slot_mapping.size()) + ") disagree");
    if (cu_seqlens_q.size() != cu_seqlens_k.size())
      return engine_err("cu_seqlens_q and cu_seqlens_k differ in length");
    if (!cu_seqlens_q.empty() && cu_seqlens_q[0] != 0)
      return engine_err("cumulative lengths must start at 0");
    if (block_tables.size() != batch_size())
      return engine_err(std::to_string(block_tables.size()) + " block tables for " +
                        std::to_string(batch_size()) + " sequences");
    std::vector<uint32_t> offs(1, 0), data;
    for (const auto& t : block_tables) {
      data.insert(data.end(), t.begin(), t.end());
      offs.push_back((uint32_t)data.size());
    }
    return detail::check(vapi_forward_batch_validate(
        (uint32_t)tokens.size(), positions.data(), slot_mapping.data(), cu_seqlens_q.data(),
        cu_seqlens_k.data(), (uint32_t)batch_size(), offs.data(), data.data(),
        logits_indices.data(), (uint32_t)logits_indices.size(), (uint32_t)num_blocks,
        (uint32_t)block_size));
  }
};

/* pack_block_tables (attention.rs:42-62) on the host: [batch, width], each
 * row padded with its own last block. Returns (rows, width). */
inline std::pair<std::vector<uint32_t>, size_t> pack_block_tables(const ForwardBatch& batch) {
  std::vector<uint32_t> offs(1, 0), data;
  for (const auto& t : batch.block_tables) {
    data.insert(data.end(), t.begin(), t.end());
    offs.push_back((uint32_t)data.size());
  }
  size_t width = 1;
  for (const auto& t : batch.block_tables) width = std::max(width, t.size());
  std::vector<uint32_t> out(batch.block_tables.size() * width);
  const int64_t w = vapi_pack_block_tables((uint32_t)batch.block_tables.size(), offs.data(),
                                           data.data(), out.data(), out.size());
  return {std::move(out), w < 0 ? 0 : (size_t)w};
}

/* cu_seqlens (attention.rs:64-71): the cumulative lengths on the device, u32. */
inline Result<detail::DevicePtr> cu_seqlens(const std::vector<uint32_t>& values) {
  auto buf = detail::device_alloc(std::max<size_t>(values.size(), 1) * 4);
  if (buf.is_err()) return buf;
  if (!values.empty())
    VAPI_TRY(detail::hip(hipMemcpy(buf.value().get(), values.data(), values.size() * 4,
                                   hipMemcpyHostToDevice),
                         "hipMemcpy"));
  return buf;
}

// ---- attention ---------------------------------------------------------------

/*
 * PreparedAttention (attention.rs:234-256): the step's device inputs, built
 * once per step and shared by every layer: the packed block table, the
 * cumulative lengths, the sequences with prefill rows (len_q > 1, for
 * vapi_paged_attention_prepared) and the attention workspace (sized for the
 * cache's largest attention layer and `num_heads`, zeroed once).
 */
class PreparedAttention {
 public:
  static Result<PreparedAttention> from_batch(const ForwardBatch& batch,
                                              const PagedKvCache& cache, size_t num_heads,
                                              bool deterministic = false) {
    PreparedAttention p;
    auto packed = pack_block_tables(batch);
    p.width_ = packed.second;
    p.batch_ = batch.batch_size();
    p.max_q_ = batch.max_seqlen_q;
    p.max_k_ = batch.max_seqlen_k;
    if (!p.max_q_ || !p.max_k_) {  // derive what a caller left at 0
      for (size_t i = 0; i < p.batch_; ++i) {
        p.max_q_ = std::max<size_t>(p.max_q_, batch.cu_seqlens_q[i + 1] - batch.cu_seqlens_q[i]);
        p.max_k_ = std::max<size_t>(p.max_k_, batch.cu_seqlens_k[i + 1] - batch.cu_seqlens_k[i]);
      }
    }
    bool any_decode = false;
    std::vector<uint32_t> pf;
    for (size_t i = 0; i < p.batch_; ++i) {
      const uint32_t lq = batch.cu_seqlens_q[i + 1] - batch.cu_seqlens_q[i];
      any_decode |= lq == 1;
      if (lq > 1) pf.push_back((uint32_t)i);
    }
    p.flags_ = (deterministic ? VAPI_ATTN_DETERMINISTIC : 0u) |
               (!any_decode && p.max_q_ > 1 ? VAPI_ATTN_NO_DECODE_ROWS : 0u);
    auto tab = detail::device_alloc(std::max<size_t>(packed.first.size(), 1) * 4);
    if (tab.is_err()) return tab.error();
    if (!packed.first.empty())
      VAPI_TRY(detail::hip(hipMemcpy(tab.value().get(), packed.first.data(),
                                     packed.first.size() * 4, hipMemcpyHostToDevice),
                           "hipMemcpy"));
    p.table_ = std::move(tab.value());
    auto cq = cu_seqlens(batch.cu_seqlens_q);
    if (cq.is_err()) return cq.error();
    auto ck = cu_seqlens(batch.cu_seqlens_k);
    if (ck.is_err()) return ck.error();
    p.cu_q_ = std::move(cq.value());
    p.cu_k_ = std::move(ck.value());
    auto pfd = detail::device_alloc(std::max<size_t>(pf.size(), 1) * 4);
    if (pfd.is_err()) return pfd.error();
    if (!pf.empty())
      VAPI_TRY(detail::hip(hipMemcpy(pfd.value().get(), pf.data(), pf.size() * 4,
                                     hipMemcpyHostToDevice),
                           "hipMemcpy"));
    p.pf_ = std::move(pfd.value());
    p.n_pf_ = pf.size();
    size_t ws = 0;
    for (size_t l = 0; l < cache.num_layers(); ++l) {
      if (cache.layout(l).kind != LayerLayout::Kind::Kv) continue;
      uint32_t lp = 0;
      ws = std::max(ws, vapi_paged_attention_prepared_workspace_size(
                            cache.pool_of(l, &lp), (uint32_t)p.batch_, (uint32_t)p.n_pf_,
                            (uint32_t)num_heads, (uint32_t)p.max_q_, (uint32_t)p.max_k_));
    }
    auto w = detail::device_alloc(ws);
    if (w.is_err()) return w.error();
    if (ws) VAPI_TRY(detail::hip(hipMemset(w.value().get(), 0, ws), "hipMemset"));
    p.ws_ = std::move(w.value());
    p.ws_bytes_ = ws;
    return std::move(p);
  }

  const uint32_t* block_table() const { return (const uint32_t*)table_.get(); }
  const uint32_t* seqlens_q() const { return (const uint32_t*)cu_q_.get(); }
  const uint32_t* seqlens_k() const { return (const uint32_t*)cu_k_.get(); }
  size_t batch() const { return batch_; }
  size_t width() const { return width_; }
  size_t max_seqlen_q() const { return max_q_; }
  size_t max_seqlen_k() const { return max_k_; }
  uint32_t flags() const { return flags_; }
  const uint32_t* prefill_seqs() const { return (const uint32_t*)pf_.get(); }
  size_t n_prefill() const { return n_pf_; }
  void* workspace() const { return ws_.get(); }
  size_t workspace_bytes() const { return ws_bytes_; }

 private:
  detail::DevicePtr table_, cu_q_, cu_k_, pf_, ws_;
  size_t batch_ = 0, width_ = 0, max_q_ = 0, max_k_ = 0, ws_bytes_ = 0, n_pf_ = 0;
  uint32_t flags_ = 0;
};

/*
 * paged_attention_cuda_prepared (attention.rs:262-288): q [total_q,
 * num_heads, d] in the cache's dtype; the output has q's shape. The window
 * arguments are the kernel's: window_size_left/right, none = unbounded
 * (right 0 is causal).
 */
inline Result<Tensor> paged_attention_prepared(const Tensor& q, const PagedKvCache& cache,
                                               size_t layer, const PreparedAttention& prepared,
                                               float softmax_scale,
                                               std::optional<size_t> window_size_left,
                                               std::optional<size_t> window_size_right,
                                               hipStream_t stream = nullptr) {
  if (layer >= cache.num_layers()) return engine_err("layer out of range");
  if (q.dims().size() != 3) return engine_err("q must be [total_q, num_heads, head_dim]");
  auto out = Tensor::zeros(q.dims(), q.dtype());
  if (out.is_err() || q.numel() == 0) return out;
  uint32_t lp = 0;
  const vapi_kv_pool* pool = cache.pool_of(layer, &lp);
  const int32_t wl = window_size_left ? (int32_t)*window_size_left : -1;
  const int32_t wr = window_size_right ? (int32_t)*window_size_right : -1;
  VAPI_TRY(detail::check(vapi_paged_attention_prepared(
      pool, lp, q.data(), out.value().data(), prepared.seqlens_q(), prepared.seqlens_k(),
      prepared.block_table(), (uint32_t)prepared.batch(), (uint32_t)prepared.width(),
      (uint32_t)prepared.max_seqlen_q(), (uint32_t)prepared.max_seqlen_k(),
      (uint32_t)q.dims()[1], softmax_scale, wl, wr, prepared.flags(), prepared.prefill_seqs(),
      (uint32_t)prepared.n_prefill(), prepared.workspace(), prepared.workspace_bytes(),
      (vapi_stream_t)stream)));
  VAPI_TRY(detail::hip(hipStreamSynchronize(stream), "hipStreamSynchronize"));
  return out;
}

/* paged_attention_cuda_windowed (attention.rs:196-232): prepares the step
 * inputs for this one call. */
inline Result<Tensor> paged_attention_windowed(const Tensor& q, const PagedKvCache& cache,
                                               size_t layer, const ForwardBatch& batch,
                                               float softmax_scale,
                                               std::optional<size_t> window_size_left,
                                               std::optional<size_t> window_size_right) {
  if (q.dims().size() != 3) return engine_err("q must be [total_q, num_heads, head_dim]");
  auto prep = PreparedAttention::from_batch(batch, cache, q.dims()[1]);
  if (prep.is_err()) return prep.error();
  return paged_attention_prepared(q, cache, layer, prep.value(), softmax_scale,
                                  window_size_left, window_size_right);
}

/* paged_attention_cuda (attention.rs:165-194): causal, with an optional
 * sliding window of w keys (HF's q - k < w), i.e. window_size_left w - 1. */
inline Result<Tensor> paged_attention(const Tensor& q, const PagedKvCache& cache, size_t layer,
                                      const ForwardBatch& batch, float softmax_scale,
                                      std::optional<size_t> sliding_window) {
  std::optional<size_t> wl;
  if (sliding_window) wl = *sliding_window ? *sliding_window - 1 : 0;
  return paged_attention_windowed(q, cache, layer, batch, softmax_scale, wl, size_t(0));
}

// ---- the backend's block methods ---------------------------------------------

using BlockId = uint32_t;

/*
 * The copy pairs Scheduler::fork hands to copy_blocks
 * (crates/vapi-engine/src/scheduler.rs:217-281), for `extra` children of a
 * sequence whose table is `parent` and whose prompt has `computed` tokens:
 * the blocks the prompt fills completely are shared; the open block after
 * them (if the parent has one) is replaced by a fresh block per child,
 * `allocate()`, and a (parent's open block, child's block) pair is emitted
 * only when the open block holds content (computed % block_size != 0).
 */
struct ForkPlan {
  std::vector<std::vector<BlockId>> children;
  std::vector<std::pair<BlockId, BlockId>> pairs;
};
template <class Allocate>
ForkPlan fork_copy_pairs(const std::vector<BlockId>& parent, size_t computed, size_t block_size,
                         size_t extra, Allocate allocate) {
  const size_t full = computed / block_size;
  const bool has_content = computed % block_size != 0;
  ForkPlan plan;
  for (size_t c = 0; c < extra; ++c) {
    std::vector<BlockId> child(parent.begin(), parent.begin() + std::min(full, parent.size()));
    if (parent.size() > full) {
      const BlockId fresh = allocate();
      if (has_content) plan.pairs.push_back({parent[full], fresh});
      child.push_back(fresh);
    }
    plan.children.push_back(std::move(child));
  }
  return plan;
}

/*
 * ExecutionBackend's block methods (crates/vapi-engine/src/backend.rs:339-367)
 * over a PagedKvCache, as CandleBackend implements them
 * (crates/vapi-backend-candle/src/backend.rs:695-797): one blob per block,
 * every layer's K then every layer's V (each NHD [block_size, kvh, d]);
 * copies cover every layer, K and V.
 */
class HipBackend {
 public:
  explicit HipBackend(PagedKvCache cache) : cache_(std::move(cache)) {}

  size_t num_blocks() const { return cache_.num_blocks(); }

  size_t block_bytes() const { return vapi_kv_block_bytes(cache_.chain()); }

  Result<std::vector<uint8_t>> export_block(BlockId id) const {
    if (id >= cache_.num_blocks())
      return engine_err("block " + std::to_string(id) + " of " +
                        std::to_string(cache_.num_blocks()));
    const size_t bb = block_bytes();
    auto dev = detail::device_alloc(bb + 4);
    if (dev.is_err()) return dev.error();
    char* base = (char*)dev.value().get();
    VAPI_TRY(detail::hip(hipMemcpy(base + bb, &id, 4, hipMemcpyHostToDevice), "hipMemcpy"));
    VAPI_TRY(detail::check(
        vapi_kv_export_blocks(cache_.chain(), (const uint32_t*)(base + bb), 1, base, nullptr)));
    std::vector<uint8_t> out(bb);
    VAPI_TRY(detail::hip(hipMemcpy(out.data(), base, bb, hipMemcpyDeviceToHost), "hipMemcpy"));
    return out;
  }

  Result<void> import_block(BlockId id, const uint8_t* bytes, size_t len) {
    const size_t bb = block_bytes();
    // backend.rs:739-745: a blob of another length is an error.
    if (len != bb)
      return engine_err("block blob is " + std::to_string(len) + " bytes, expected " +
                        std::to_string(bb));
    if (id >= cache_.num_blocks())
      return engine_err("block " + std::to_string(id) + " of " +
                        std::to_string(cache_.num_blocks()));
    auto dev = detail::device_alloc(bb + 4);
    if (dev.is_err()) return dev.error();
    char* base = (char*)dev.value().get();
    VAPI_TRY(detail::hip(hipMemcpy(base, bytes, bb, hipMemcpyHostToDevice), "hipMemcpy"));
    VAPI_TRY(detail::hip(hipMemcpy(base + bb, &id, 4, hipMemcpyHostToDevice), "hipMemcpy"));
    VAPI_TRY(detail::check(
        vapi_kv_import_blocks(cache_.chain(), (const uint32_t*)(base + bb), 1, base, nullptr)));
    return detail::hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
  }

  Result<void> copy_blocks(const std::vector<std::pair<BlockId, BlockId>>& pairs) {
    if (pairs.empty()) return ok();
    std::vector<uint32_t> flat;
    for (const auto& p : pairs) {
      if (p.first >= cache_.num_blocks() || p.second >= cache_.num_blocks())
        return engine_err("copy pair (" + std::to_string(p.first) + ", " +
                          std::to_string(p.second) + ") past " +
                          std::to_string(cache_.num_blocks()) + " blocks");
      flat.push_back(p.first);
      flat.push_back(p.second);
    }
    auto dev = detail::device_alloc(flat.size() * 4);
    if (dev.is_err()) return dev.error();
    VAPI_TRY(detail::hip(hipMemcpy(dev.value().get(), flat.data(), flat.size() * 4,
                                   hipMemcpyHostToDevice),
                         "hipMemcpy"));
    VAPI_TRY(detail::check(vapi_kv_copy_blocks(cache_.chain(),
                                               (const uint32_t*)dev.value().get(),
                                               (uint32_t)pairs.size(), nullptr)));
    return detail::hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
  }

  PagedKvCache& cache() { return cache_; }
  const PagedKvCache& cache() const { return cache_; }

 private:
  PagedKvCache cache_;
};

}  // namespace vapi

#undef VAPI_TRY

#endif  // VAPI_KV_HPP
