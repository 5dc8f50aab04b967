// The reference backend's own tests, run against the C++ mirror in
// include/vapi_kv.hpp (and through it libvapi_kv.so on the GPU). Each test
// keeps the name and the assertions of the Rust test it restates:
//   crates/vapi-backend-candle/src/cache.rs:292-446      (cache tests)
//   crates/vapi-backend-candle/src/attention.rs:318-431  (CPU-path tests)
//   crates/vapi-backend-candle/src/attention.rs:432-714  (GPU-vs-CPU tests)
// plus the block methods (backend.rs:695-797), ForwardBatch::validate
// (crates/vapi-engine/src/backend.rs:96-204) and the fork's copy pairs
// (crates/vapi-engine/tests/scheduler.rs:524-637).
//
// Usage: backend_tests [--host-only] [name-substring]
//   --host-only runs the tests that touch no GPU (validate, table packing,
//   layout sizing); the default runs every test and needs a GPU.
// Exit status 0 when every selected test passed.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "vapi_kv.hpp"

using namespace vapi;

namespace {

struct Case {
  std::string name;
  bool gpu;
  std::function<void()> fn;
};
std::vector<Case>& registry() {
  static std::vector<Case> r;
  return r;
}
struct Registrar {
  Registrar(const char* n, bool gpu, std::function<void()> f) {
    registry().push_back({n, gpu, std::move(f)});
  }
};
std::vector<std::string> g_failures;

#define TEST(name, gpu)                                  \
  static void name();                                    \
  static Registrar reg_##name(#name, gpu, name);         \
  static void name()

#define EXPECT(cond)                                                                 \
  do {                                                                               \
    if (!(cond)) g_failures.push_back(std::string(#cond) + " (line " +              \
                                      std::to_string(__LINE__) + ")");               \
  } while (0)

// Unwrap a Result, recording the error and leaving the test on failure.
#define OK(expr)                                                                     \
  ({                                                                                 \
    auto r_ = (expr);                                                                \
    if (r_.is_err()) {                                                               \
      g_failures.push_back(std::string(#expr) + ": " + r_.error().message +         \
                           " (line " + std::to_string(__LINE__) + ")");              \
      return;                                                                        \
    }                                                                                \
    std::move(r_.value());                                                           \
  })
#define OK_VOID(expr)                                                                \
  do {                                                                               \
    auto r_ = (expr);                                                                \
    if (r_.is_err()) {                                                               \
      g_failures.push_back(std::string(#expr) + ": " + r_.error().message +         \
                           " (line " + std::to_string(__LINE__) + ")");              \
      return;                                                                        \
    }                                                                                \
  } while (0)

// ---- cache.rs:292-446 ------------------------------------------------------

constexpr size_t BS = 4;

Result<PagedKvCache> cache(size_t num_blocks, MemoryLayout layout = MemoryLayout::HND) {
  return PagedKvCache::create(2, num_blocks, BS, 2, 3, DType::F32, layout);
}

// Every element distinct, so a misplaced row is detectable.
Result<Tensor> rows(size_t n, float base) {
  std::vector<float> data(n * 2 * 3);
  for (size_t i = 0; i < data.size(); ++i) data[i] = base + (float)i;
  return Tensor::from_vec(data, {n, 2, 3}, DType::F32);
}

// The layer's K as [num_slots, 2, 3] on the host, in slot order.
Result<std::vector<float>> flat_k(const PagedKvCache& c, size_t layer) {
  std::vector<uint32_t> all(c.num_blocks());
  for (size_t b = 0; b < all.size(); ++b) all[b] = (uint32_t)b;
  auto t = gather_kv(c, layer, Which::K, all, c.num_slots());
  if (t.is_err()) return t.error();
  return t.value().to_vec_f32();
}

TEST(a_write_spanning_non_adjacent_blocks_lands_in_exactly_those_slots, true) {
  auto c = OK(cache(8));
  // A prefill chunk of 9 tokens over block table [6, 1, 3]: slots 24..28,
  // 4..8, 12, three separate runs.
  const std::vector<uint32_t> slots = {24, 25, 26, 27, 4, 5, 6, 7, 12};
  auto k = OK(rows(9, 100.f));
  auto v = OK(rows(9, 1000.f));
  OK_VOID(write_kv_to_cache(c, 1, k, v, slots));
  auto got_k = OK(gather_kv(c, 1, Which::K, {6, 1, 3}, 9));
  auto got_v = OK(gather_kv(c, 1, Which::V, {6, 1, 3}, 9));
  EXPECT(OK(got_k.to_vec_f32()) == OK(k.to_vec_f32()));
  EXPECT(OK(got_v.to_vec_f32()) == OK(v.to_vec_f32()));
  // Nothing else moved: the other layer is untouched, and every slot not in
  // the mapping is still zero.
  const auto other = OK(flat_k(c, 0));
  double sum = 0;
  for (float x : other) sum += x;
  EXPECT(sum == 0.0);
  const auto flat = OK(flat_k(c, 1));
  const std::set<uint32_t> written(slots.begin(), slots.end());
  for (size_t slot = 0; slot < 32; ++slot) {
    bool nonzero = false;
    for (size_t e = 0; e < 6; ++e) nonzero |= flat[slot * 6 + e] != 0.f;
    EXPECT(nonzero == (written.count((uint32_t)slot) == 1));
  }
}

TEST(the_flat_view_really_shares_storage_with_the_paged_tensor, true) {
  // Slot 5 is block 1, offset 1: written through the slot mapping, read back
  // through the block table and through the block's exported bytes (the
  // reference's [block_size, kvh, d] order, K of layer 0 first).
  auto c = OK(cache(2, MemoryLayout::NHD));
  OK_VOID(write_kv_to_cache(c, 0, OK(rows(1, 7.f)), OK(rows(1, 9.f)), {5}));
  auto block1 = OK(gather_kv(c, 0, Which::K, {1}, BS));
  const auto b = OK(block1.to_vec_f32());
  const std::vector<float> row(b.begin() + 6, b.begin() + 12);
  EXPECT((row == std::vector<float>{7, 8, 9, 10, 11, 12}));
  HipBackend be(std::move(c));
  const auto blob = OK(be.export_block(1));
  float first_row[6];
  std::memcpy(first_row, blob.data() + 6 * sizeof(float), sizeof first_row);
  EXPECT(first_row[0] == 7.f && first_row[5] == 12.f);
}

TEST(a_decode_batch_is_many_single_slot_runs, true) {
  auto c = OK(cache(4));
  const std::vector<uint32_t> slots = {3, 9, 0, 14, 6, 11};
  auto k = OK(rows(6, 1.f));
  OK_VOID(write_kv_to_cache(c, 0, k, k, slots));
  const auto flat = OK(flat_k(c, 0));
  const auto want = OK(k.to_vec_f32());
  for (size_t i = 0; i < slots.size(); ++i)
    for (size_t e = 0; e < 6; ++e) EXPECT(flat[slots[i] * 6 + e] == want[i * 6 + e]);
}

TEST(the_scatter_path_and_the_run_path_agree, true) {
  // Same rows, same slots, written all at once and one row at a time.
  const std::vector<uint32_t> slots = {30, 31, 5, 6, 7, 12, 20, 2};
  const std::vector<float> kh = OK(OK(rows(8, 3.f)).to_vec_f32());
  auto k = OK(Tensor::from_vec(kh, {8, 2, 3}, DType::F32));
  auto a = OK(cache(8));
  auto b = OK(cache(8));
  OK_VOID(write_kv_to_cache(a, 0, k, k, slots));
  for (size_t i = 0; i < slots.size(); ++i) {
    auto row = OK(Tensor::from_vec(std::vector<float>(kh.begin() + 6 * i, kh.begin() + 6 * i + 6),
                                   {1, 2, 3}, DType::F32));
    OK_VOID(write_kv_to_cache(b, 0, row, row, {slots[i]}));
  }
  const auto fa = OK(flat_k(a, 0)), fb = OK(flat_k(b, 0));
  EXPECT(fa == fb);
  size_t nonzero = 0;
  for (float x : fa) nonzero += x != 0.f;
  EXPECT(nonzero > 0);
}

TEST(a_second_write_overwrites_rather_than_accumulates, true) {
  auto c = OK(cache(2));
  OK_VOID(write_kv_to_cache(c, 0, OK(rows(1, 1.f)), OK(rows(1, 1.f)), {2}));
  OK_VOID(write_kv_to_cache(c, 0, OK(rows(1, 50.f)), OK(rows(1, 50.f)), {2}));
  EXPECT(OK(flat_k(c, 0))[2 * 6] == 50.f);
}

TEST(a_rows_layer_stores_one_row_per_token_and_no_v, true) {
  const std::vector<LayerLayout> layouts = {LayerLayout::Kv(2, 3), LayerLayout::Rows(5)};
  auto c = OK(PagedKvCache::with_layouts(layouts, 4, BS, DType::F32));
  EXPECT(PagedKvCache::elems_per_token(layouts) == 2 * 2 * 3 + 5);
  uint32_t lp = 0;
  EXPECT(c.pool_of(1, &lp)->v == nullptr);
  EXPECT(c.pool_of(1, &lp)->head_dim == 5);
  std::vector<float> data(10);
  for (size_t i = 0; i < 10; ++i) data[i] = (float)i;
  auto r = OK(Tensor::from_vec(data, {2, 1, 5}, DType::F32));
  OK_VOID(write_k_to_cache(c, 1, r, {9, 10}));
  const auto got = OK(OK(gather_kv(c, 1, Which::K, {2}, 3)).to_vec_f32());  // slots 8..11
  EXPECT((std::vector<float>(got.begin(), got.begin() + 5) == std::vector<float>(5, 0.f)));
  EXPECT((std::vector<float>(got.begin() + 5, got.begin() + 10) ==
          std::vector<float>{0, 1, 2, 3, 4}));
  EXPECT((std::vector<float>(got.begin() + 10, got.begin() + 15) ==
          std::vector<float>{5, 6, 7, 8, 9}));
  // A Rows layer has no V to gather, and a Kv layer takes no K-only write.
  EXPECT(gather_kv(c, 1, Which::V, {2}, 3).is_err());
  EXPECT(write_k_to_cache(c, 0, r, {9, 10}).is_err());
}

TEST(mismatched_shapes_and_out_of_range_slots_are_errors, true) {
  auto c = OK(cache(2));
  EXPECT(write_kv_to_cache(c, 0, OK(rows(2, 0.f)), OK(rows(2, 0.f)), {0}).is_err());
  EXPECT(write_kv_to_cache(c, 0, OK(rows(1, 0.f)), OK(rows(1, 0.f)), {8}).is_err());
  auto wrong = OK(Tensor::from_vec(std::vector<float>(6, 0.f), {1, 2, 3}, DType::F16));
  EXPECT(write_kv_to_cache(c, 0, wrong, wrong, {0}).is_err());
  EXPECT(write_kv_to_cache(c, 0, OK(rows(1, 0.f)), OK(rows(2, 0.f)), {0}).is_err());
}

// ---- attention.rs:318-431 (the CPU path's tests, on the device) ---------------

// Dense attention over one sequence, the long way (attention.rs:297-321):
// bottom-right causal, optional left window of w keys (q - k < w).
std::vector<std::vector<double>> dense_causal(const std::vector<std::vector<float>>& q,
                                              const std::vector<std::vector<float>>& k,
                                              const std::vector<std::vector<float>>& v,
                                              double scale, size_t window = 0) {
  const size_t len_k = k.size(), len_q = q.size(), off = len_k - len_q;
  std::vector<std::vector<double>> out;
  for (size_t i = 0; i < len_q; ++i) {
    const size_t p = off + i;
    std::vector<double> s;
    double mx = -INFINITY;
    for (size_t j = 0; j <= p; ++j) {
      if (window && p - j >= window) {
        s.push_back(-INFINITY);
        continue;
      }
      double d = 0;
      for (size_t e = 0; e < q[i].size(); ++e) d += (double)q[i][e] * k[j][e];
      s.push_back(d * scale);
      mx = std::max(mx, d * scale);
    }
    double sum = 0;
    for (double& x : s) sum += (x = std::exp(x - mx));
    std::vector<double> o(v[0].size(), 0.0);
    for (size_t j = 0; j <= p; ++j)
      for (size_t e = 0; e < o.size(); ++e) o[e] += s[j] / sum * v[j][e];
    out.push_back(o);
  }
  return out;
}

TEST(a_sliding_window_hides_keys_older_than_the_window, true) {
  // One head, head_dim 2, six keys, six queries. With window 3 the query at
  // position p sees keys p-2..=p. Zero queries make the attention uniform
  // over visible keys, so the output's second component is the mean
  // visible key index.
  auto c = OK(PagedKvCache::create(1, 2, 4, 1, 2, DType::F32));
  std::vector<float> k, v;
  for (int i = 0; i < 6; ++i) k.insert(k.end(), {(float)i, 0.f}), v.insert(v.end(), {1.f, (float)i});
  OK_VOID(write_kv_to_cache(c, 0, OK(Tensor::from_vec(k, {6, 1, 2}, DType::F32)),
                            OK(Tensor::from_vec(v, {6, 1, 2}, DType::F32)), {0, 1, 2, 3, 4, 5}));
  auto q = OK(Tensor::zeros({6, 1, 2}, DType::F32));
  ForwardBatch batch;
  batch.cu_seqlens_q = {0, 6};
  batch.cu_seqlens_k = {0, 6};
  batch.block_tables = {{0, 1}};
  const auto out = OK(OK(paged_attention(q, c, 0, batch, 1.f, size_t(3))).to_vec_f32());
  std::vector<float> means;
  for (size_t r = 0; r < 6; ++r) means.push_back(out[2 * r + 1]);
  EXPECT((means == std::vector<float>{0.f, 0.5f, 1.f, 2.f, 3.f, 4.f}));
}

TEST(the_cpu_reference_matches_dense_attention_for_a_mixed_batch, true) {
  // One kv head, one q head, head_dim 4, block size 4. Sequence A is a
  // prefill chunk of 3 on 5 cached tokens; B a decode over 6 keys. Blocks
  // deliberately not contiguous.
  auto c = OK(PagedKvCache::create(1, 8, 4, 1, 4, DType::F32));
  auto rnd = [](size_t n, float seed) {
    std::vector<std::vector<float>> r(n, std::vector<float>(4));
    for (size_t i = 0; i < n; ++i)
      for (size_t d = 0; d < 4; ++d) r[i][d] = std::sin((float)(i * 7 + d * 3) * 0.37f + seed);
    return r;
  };
  auto flat = [](const std::vector<std::vector<float>>& r) {
    std::vector<float> f;
    for (const auto& x : r) f.insert(f.end(), x.begin(), x.end());
    return f;
  };
  auto to_t = [&](const std::vector<std::vector<float>>& r) {
    return Tensor::from_vec(flat(r), {r.size(), 1, 4}, DType::F32);
  };
  auto slots = [](const std::vector<uint32_t>& table, size_t n) {
    std::vector<uint32_t> s;
    for (size_t p = 0; p < n; ++p) s.push_back(table[p / 4] * 4 + (uint32_t)(p % 4));
    return s;
  };
  const auto ka = rnd(8, 0.1f), va = rnd(8, 0.2f), kb = rnd(6, 0.3f), vb = rnd(6, 0.4f);
  const std::vector<uint32_t> ta = {5, 2}, tb = {7, 0};
  OK_VOID(write_kv_to_cache(c, 0, OK(to_t(ka)), OK(to_t(va)), slots(ta, 8)));
  OK_VOID(write_kv_to_cache(c, 0, OK(to_t(kb)), OK(to_t(vb)), slots(tb, 6)));
  const auto qa = rnd(3, 0.5f), qb = rnd(1, 0.6f);
  std::vector<std::vector<float>> qall = qa;
  qall.push_back(qb[0]);
  ForwardBatch batch;
  batch.cu_seqlens_q = {0, 3, 4};
  batch.cu_seqlens_k = {0, 8, 14};
  batch.block_tables = {ta, tb};
  const float scale = 0.5f;
  auto out_t = OK(paged_attention(OK(to_t(qall)), c, 0, batch, scale, std::nullopt));
  EXPECT((out_t.dims() == std::vector<size_t>{4, 1, 4}));
  const auto out = OK(out_t.to_vec_f32());
  auto want = dense_causal(qa, ka, va, scale);
  const auto wb = dense_causal(qb, kb, vb, scale);
  want.insert(want.end(), wb.begin(), wb.end());
  for (size_t r = 0; r < 4; ++r)
    for (size_t e = 0; e < 4; ++e) EXPECT(std::fabs(out[4 * r + e] - want[r][e]) < 1e-5);
}

TEST(ragged_block_tables_are_padded_to_a_rectangle, false) {
  ForwardBatch b;
  b.block_tables = {{0, 1, 2}, {7}};
  const auto packed = pack_block_tables(b);
  EXPECT(packed.second == 3);
  EXPECT((packed.first == std::vector<uint32_t>{0, 1, 2, 7, 7, 7}));
}

TEST(cumulative_lengths_are_u32_as_the_kernel_reads_them, true) {
  auto t = OK(cu_seqlens({0, 4, 9}));
  uint32_t host[3] = {};
  EXPECT(hipMemcpy(host, t.get(), sizeof host, hipMemcpyDeviceToHost) == hipSuccess);
  EXPECT(host[0] == 0 && host[1] == 4 && host[2] == 9);
}

// ---- attention.rs:432-714 (the GPU kernel against the CPU path) ----------------

constexpr size_t HEADS = 4, KV_HEADS = 2, HEAD_DIM = 64, BLOCK_SIZE = 32;

std::vector<float> sin_rows(size_t n, size_t heads, size_t d, float seed, float mul, bool cosine) {
  std::vector<float> x(n * heads * d);
  for (size_t i = 0; i < x.size(); ++i)
    x[i] = (cosine ? std::cos((float)i * mul + seed) : std::sin((float)i * mul + seed)) * 0.5f;
  return x;
}

std::vector<uint32_t> slots_of(const std::vector<uint32_t>& table, size_t lo, size_t hi,
                               size_t bs = BLOCK_SIZE) {
  std::vector<uint32_t> s;
  for (size_t p = lo; p < hi; ++p) s.push_back(table[p / bs] * (uint32_t)bs + (uint32_t)(p % bs));
  return s;
}

// The value of a Result that must hold one (test helpers without a way to
// report): an error ends the program with its message.
template <class T>
T must(Result<T> r) {
  if (r.is_err()) {
    std::fprintf(stderr, "fatal: %s\n", r.error().message.c_str());
    std::exit(2);
  }
  return std::move(r.value());
}

// paged_attention_cpu (attention.rs:73-163) on host copies of the cache: f32
// math over the stored values, GQA by head group, bottom-right causal, a left
// window of w keys, the output rounded to the input dtype. right_causal =
// false is the bidirectional case.
std::vector<float> cpu_reference(const std::vector<float>& q_stored, size_t heads,
                                 const PagedKvCache& c, const ForwardBatch& batch, float scale,
                                 std::optional<size_t> window, DType dtype,
                                 bool right_causal = true) {
  const size_t kvh = c.layout(0).num_kv_heads, d = c.layout(0).head_dim, g = heads / kvh;
  std::vector<float> out(q_stored.size(), 0.f);
  for (size_t s = 0; s + 1 < batch.cu_seqlens_q.size(); ++s) {
    const size_t q0 = batch.cu_seqlens_q[s], lq = batch.cu_seqlens_q[s + 1] - q0;
    const size_t lk = batch.cu_seqlens_k[s + 1] - batch.cu_seqlens_k[s];
    if (!lq) continue;
    const auto k = must(must(gather_kv(c, 0, Which::K, batch.block_tables[s], lk)).to_vec_f32());
    const auto v = must(must(gather_kv(c, 0, Which::V, batch.block_tables[s], lk)).to_vec_f32());
    for (size_t j = 0; j < lq; ++j) {
      const size_t p = lk - lq + j;
      for (size_t h = 0; h < heads; ++h) {
        const size_t kh = h / g;
        std::vector<double> sc(lk, -INFINITY);
        double mx = -INFINITY;
        for (size_t t = 0; t < lk; ++t) {
          if (right_causal && t > p) continue;
          if (window && t < p && p - t >= *window) continue;
          double dot = 0;
          for (size_t e = 0; e < d; ++e)
            dot += (double)q_stored[((q0 + j) * heads + h) * d + e] * k[(t * kvh + kh) * d + e];
          sc[t] = dot * scale;
          mx = std::max(mx, sc[t]);
        }
        double sum = 0;
        for (double& x : sc) sum += (x = std::isinf(x) ? 0.0 : std::exp(x - mx));
        for (size_t e = 0; e < d; ++e) {
          double o = 0;
          for (size_t t = 0; t < lk; ++t) o += sc[t] / sum * v[(t * kvh + kh) * d + e];
          float f = (float)o;
          if (dtype == DType::BF16) f = detail::bf16_to_f32(detail::f32_to_bf16(f));
          if (dtype == DType::F16) f = detail::f16_to_f32(detail::f32_to_f16(f));
          out[((q0 + j) * heads + h) * d + e] = f;
        }
      }
    }
  }
  return out;
}

// A: 70 cached tokens plus a 20-token prefill chunk (seqlen_q < seqlen_k);
// B: a decode over 40 keys. Blocks out of order.
struct Mixed {
  PagedKvCache cache;
  Tensor q;
  std::vector<float> q_stored;
  ForwardBatch batch;
};
Result<Mixed> mixed(DType dtype) {
  auto c = PagedKvCache::create(1, 8, BLOCK_SIZE, KV_HEADS, HEAD_DIM, dtype);
  if (c.is_err()) return c.error();
  const std::vector<uint32_t> ta = {5, 1, 6}, tb = {7, 2};
  const size_t len_a = 90, chunk_a = 20, len_b = 40;
  auto rw = [&](size_t n, float seed) {
    return Tensor::from_vec(sin_rows(n, KV_HEADS, HEAD_DIM, seed, 0.173f, false),
                            {n, KV_HEADS, HEAD_DIM}, dtype);
  };
  auto w1 = write_kv_to_cache(c.value(), 0, must(rw(len_a, 0.1f)), must(rw(len_a, 0.2f)),
                              slots_of(ta, 0, len_a));
  if (w1.is_err()) return w1.error();
  auto w2 = write_kv_to_cache(c.value(), 0, must(rw(len_b, 0.3f)), must(rw(len_b, 0.4f)),
                              slots_of(tb, 0, len_b));
  if (w2.is_err()) return w2.error();
  auto q = Tensor::from_vec(sin_rows(chunk_a + 1, HEADS, HEAD_DIM, 0.5f, 0.131f, true),
                            {chunk_a + 1, HEADS, HEAD_DIM}, dtype);
  if (q.is_err()) return q.error();
  ForwardBatch batch;
  batch.cu_seqlens_q = {0, (uint32_t)chunk_a, (uint32_t)chunk_a + 1};
  batch.cu_seqlens_k = {0, (uint32_t)len_a, (uint32_t)(len_a + len_b)};
  batch.block_tables = {ta, tb};
  batch.max_seqlen_q = chunk_a;
  batch.max_seqlen_k = len_a;
  auto stored = q.value().to_vec_f32();
  if (stored.is_err()) return stored.error();
  return Mixed{std::move(c.value()), q.value(), stored.value(), batch};
}

double max_abs_diff(const std::vector<float>& a, const std::vector<float>& b, size_t n = 0) {
  double m = 0;
  for (size_t i = 0; i < (n ? n : a.size()); ++i) m = std::max(m, (double)std::fabs(a[i] - b[i]));
  return m;
}

void check_dtype(DType dtype, double tol) {
  auto m = OK(mixed(dtype));
  const float scale = 1.f / std::sqrt((float)HEAD_DIM);
  const auto want = cpu_reference(m.q_stored, HEADS, m.cache, m.batch, scale, std::nullopt, dtype);
  auto got_t = OK(paged_attention(m.q, m.cache, 0, m.batch, scale, std::nullopt));
  EXPECT(got_t.dims() == m.q.dims());
  const double diff = max_abs_diff(OK(got_t.to_vec_f32()), want);
  EXPECT(diff < tol);
}

TEST(the_flash_kernel_matches_the_cpu_reference_in_bf16, true) { check_dtype(DType::BF16, 1e-2); }

TEST(the_flash_kernel_matches_the_cpu_reference_in_f16, true) { check_dtype(DType::F16, 1e-3); }

TEST(laguna_shapes_match_the_cpu_reference, true) {
  // head_dim 16, 6 or 8 query heads over 2 kv heads, a 6-token window, a
  // pure prefill plus a decode.
  const std::vector<std::pair<size_t, std::optional<size_t>>> shapes = {
      {6, std::nullopt}, {8, size_t(6)}, {6, size_t(6)}};
  for (const auto& [heads, window] : shapes) {
    const size_t kvh = 2, hd = 16;
    auto c = OK(PagedKvCache::create(1, 8, BLOCK_SIZE, kvh, hd, DType::BF16));
    auto mk = [&](size_t n, size_t h, float seed) {
      return Tensor::from_vec(sin_rows(n, h, hd, seed, 0.173f, false), {n, h, hd}, DType::BF16);
    };
    const std::vector<uint32_t> ta = {4}, tb = {6, 1};
    const size_t len_a = 18, len_b = 40;
    OK_VOID(write_kv_to_cache(c, 0, OK(mk(len_a, kvh, 0.1f)), OK(mk(len_a, kvh, 0.2f)),
                              slots_of(ta, 0, len_a)));
    OK_VOID(write_kv_to_cache(c, 0, OK(mk(len_b, kvh, 0.3f)), OK(mk(len_b, kvh, 0.4f)),
                              slots_of(tb, 0, len_b)));
    auto q = OK(mk(len_a + 1, heads, 0.5f));
    ForwardBatch batch;
    batch.cu_seqlens_q = {0, (uint32_t)len_a, (uint32_t)len_a + 1};
    batch.cu_seqlens_k = {0, (uint32_t)len_a, (uint32_t)(len_a + len_b)};
    batch.block_tables = {ta, tb};
    batch.max_seqlen_q = len_a;
    batch.max_seqlen_k = len_b;
    const float scale = 1.f / std::sqrt((float)hd);
    const auto want =
        cpu_reference(OK(q.to_vec_f32()), heads, c, batch, scale, window, DType::BF16);
    const auto got = OK(OK(paged_attention(q, c, 0, batch, scale, window)).to_vec_f32());
    EXPECT(max_abs_diff(got, want) < 1e-2);
  }
}

TEST(a_sliding_window_matches_the_cpu_reference_and_differs_from_full, true) {
  auto m = OK(mixed(DType::BF16));
  const float scale = 1.f / std::sqrt((float)HEAD_DIM);
  const auto want =
      cpu_reference(m.q_stored, HEADS, m.cache, m.batch, scale, size_t(16), DType::BF16);
  const auto got = OK(OK(paged_attention(m.q, m.cache, 0, m.batch, scale, size_t(16))).to_vec_f32());
  EXPECT(max_abs_diff(got, want) < 1e-2);
  const auto full =
      cpu_reference(m.q_stored, HEADS, m.cache, m.batch, scale, std::nullopt, DType::BF16);
  EXPECT(max_abs_diff(full, want) > 1e-2);  // the window must hide something
}

TEST(a_bidirectional_window_is_not_causal, true) {
  auto m = OK(mixed(DType::BF16));
  const float scale = 1.f / std::sqrt((float)HEAD_DIM);
  const auto causal = OK(OK(paged_attention_windowed(m.q, m.cache, 0, m.batch, scale,
                                                     std::nullopt, size_t(0)))
                             .to_vec_f32());
  const auto bidirectional = OK(OK(paged_attention_windowed(m.q, m.cache, 0, m.batch, scale,
                                                            std::nullopt, std::nullopt))
                                    .to_vec_f32());
  const auto want =
      cpu_reference(m.q_stored, HEADS, m.cache, m.batch, scale, std::nullopt, DType::BF16);
  EXPECT(max_abs_diff(causal, want) < 1e-2);
  // The decode row (the last) sees every key either way; the 20 prefill rows
  // must differ.
  EXPECT(max_abs_diff(bidirectional, want, 20 * HEADS * HEAD_DIM) > 1e-2);
}

// ---- the backend's block methods (backend.rs:695-797) --------------------------

Result<HipBackend> filled_backend(size_t layers, size_t blocks, bool block_major = false) {
  auto c = PagedKvCache::create(layers, blocks, 16, 4, 128, DType::BF16, MemoryLayout::HND,
                                block_major);
  if (c.is_err()) return c.error();
  for (size_t l = 0; l < layers; ++l) {
    std::vector<float> kv(blocks * 16 * 4 * 128);
    for (size_t i = 0; i < kv.size(); ++i) kv[i] = std::sin((float)(i + 7919 * l) * 0.01f);
    const Tensor k = must(Tensor::from_vec(kv, {blocks * 16, 4, 128}, DType::BF16));
    for (float& x : kv) x = -x;
    const Tensor v = must(Tensor::from_vec(kv, {blocks * 16, 4, 128}, DType::BF16));
    std::vector<uint32_t> slots(blocks * 16);
    for (size_t s = 0; s < slots.size(); ++s) slots[s] = (uint32_t)s;
    auto w = write_kv_to_cache(c.value(), l, k, v, slots);
    if (w.is_err()) return w.error();
  }
  return HipBackend(std::move(c.value()));
}

TEST(block_bytes_cover_every_layer_k_and_v, true) {
  auto be = OK(filled_backend(3, 4));
  EXPECT(be.block_bytes() == 3 * 2 * 16 * 4 * 128 * 2);
  EXPECT(be.num_blocks() == 4);
}

TEST(an_exported_block_imports_back_to_the_same_bytes, true) {
  // engine.rs:1282-1293: import(export(b)) is the identity, into another id.
  auto be = OK(filled_backend(3, 4));
  const auto blob = OK(be.export_block(1));
  OK_VOID(be.import_block(3, blob.data(), blob.size()));
  EXPECT(OK(be.export_block(3)) == blob);
  EXPECT(OK(be.export_block(0)) != blob);
}

TEST(an_import_of_the_wrong_length_is_an_error, true) {
  // backend.rs:739-745.
  auto be = OK(filled_backend(2, 2));
  const auto blob = OK(be.export_block(0));
  EXPECT(be.import_block(1, blob.data(), blob.size() - 2).is_err());
  EXPECT(be.export_block(2).is_err());
}

TEST(copy_blocks_copies_every_layer_k_and_v, true) {
  auto be = OK(filled_backend(3, 6));
  const auto b0 = OK(be.export_block(0)), b2 = OK(be.export_block(2)), b5 = OK(be.export_block(5));
  OK_VOID(be.copy_blocks({{0, 4}, {2, 1}}));
  EXPECT(OK(be.export_block(4)) == b0);
  EXPECT(OK(be.export_block(1)) == b2);
  EXPECT(OK(be.export_block(5)) == b5);  // untouched
  EXPECT(be.copy_blocks({{0, 6}}).is_err());
}

TEST(a_block_major_cache_moves_blocks_like_a_layer_major_one, true) {
  // The same contents in both allocations: every block exports the same
  // blob, and a copy (one run per pair in the block-major one) and an
  // import leave them equal.
  auto lm = OK(filled_backend(3, 6));
  auto bm = OK(filled_backend(3, 6, true));
  for (BlockId b = 0; b < 6; ++b) EXPECT(OK(bm.export_block(b)) == OK(lm.export_block(b)));
  OK_VOID(lm.copy_blocks({{0, 4}, {2, 1}}));
  OK_VOID(bm.copy_blocks({{0, 4}, {2, 1}}));
  const auto b3 = OK(lm.export_block(3));
  OK_VOID(lm.import_block(5, b3.data(), b3.size()));
  OK_VOID(bm.import_block(5, b3.data(), b3.size()));
  for (BlockId b = 0; b < 6; ++b) EXPECT(OK(bm.export_block(b)) == OK(lm.export_block(b)));
}

// ---- Scheduler::fork's copy pairs (crates/vapi-engine/tests/scheduler.rs:524-637) ----

std::function<BlockId()> counter(BlockId start) {
  auto next = std::make_shared<BlockId>(start);
  return [next] { return (*next)++; };
}

TEST(a_partial_prompt_block_is_copied_once_per_child, false) {
  // 10 tokens over 4-token blocks, two forks: two full blocks shared, the
  // partial third copied per fork.
  const std::vector<BlockId> parent = {5, 9, 2};
  const auto plan = fork_copy_pairs(parent, 10, 4, 2, counter(100));
  EXPECT(plan.children.size() == 2 && plan.pairs.size() == 2);
  for (size_t c = 0; c < plan.children.size(); ++c) {
    EXPECT(plan.pairs[c].first == parent[2]);
    EXPECT(plan.children[c][0] == parent[0] && plan.children[c][1] == parent[1]);
    EXPECT(plan.children[c][2] == plan.pairs[c].second && plan.children[c][2] != parent[2]);
  }
  EXPECT(plan.pairs[0].second != plan.pairs[1].second);
}

TEST(a_block_aligned_prompt_copies_nothing_but_still_takes_a_private_open_block, false) {
  const std::vector<BlockId> parent = {3, 4, 11};
  const auto plan = fork_copy_pairs(parent, 8, 4, 1, counter(100));
  EXPECT(plan.pairs.empty());
  EXPECT(plan.children[0][0] == 3 && plan.children[0][1] == 4 && plan.children[0][2] != 11);
}

TEST(a_parent_without_an_open_block_shares_everything, false) {
  int calls = 0;
  const auto plan = fork_copy_pairs({7, 8}, 8, 4, 3, [&] { ++calls; return BlockId(99); });
  EXPECT(plan.pairs.empty() && calls == 0);
  for (const auto& child : plan.children) EXPECT((child == std::vector<BlockId>{7, 8}));
}

TEST(a_fork_copies_the_open_block_into_each_child_on_the_device, true) {
  // The fork's pairs through copy_blocks: each child's private block holds
  // the parent's open block, every layer, K and V; the shared blocks are
  // untouched.
  auto be = OK(filled_backend(3, 8));
  const std::vector<BlockId> parent = {5, 1, 6};
  const auto plan = fork_copy_pairs(parent, 10 * 16 / 4, 16, 2, counter(2));  // 40 tokens
  EXPECT(plan.pairs.size() == 2);
  const auto open = OK(be.export_block(6)), shared = OK(be.export_block(5));
  OK_VOID(be.copy_blocks(plan.pairs));
  for (const auto& child : plan.children) {
    EXPECT(OK(be.export_block(child[2])) == open);
    EXPECT(child[0] == 5 && child[1] == 1);
  }
  EXPECT(OK(be.export_block(5)) == shared);
}

// ---- ForwardBatch::validate (crates/vapi-engine/src/backend.rs:96-204) ----------

ForwardBatch valid_batch() {
  // A 3-token prefill on 5 cached keys and a decode over 6 keys, blocks of 4.
  ForwardBatch b;
  b.tokens = {11, 12, 13, 14};
  b.positions = {5, 6, 7, 5};
  b.slot_mapping = {21, 22, 23, 1};
  b.cu_seqlens_q = {0, 3, 4};
  b.cu_seqlens_k = {0, 8, 6 + 8};
  b.block_tables = {{4, 5}, {7, 0}};
  b.logits_indices = {2, 3};
  b.max_seqlen_q = 3;
  b.max_seqlen_k = 8;
  return b;
}

std::string validate_message(const ForwardBatch& b) {
  auto r = b.validate(8, 4);
  return r.is_ok() ? std::string("ok") : r.error().message;
}

TEST(a_well_formed_batch_validates, false) { EXPECT(validate_message(valid_batch()) == "ok"); }

TEST(validate_names_the_first_violation_as_the_reference_does, false) {
  auto b = valid_batch();
  b.positions.pop_back();
  EXPECT(validate_message(b) == "tokens (4) and positions (3) disagree");
  b = valid_batch();
  b.slot_mapping.push_back(2);
  EXPECT(validate_message(b) == "tokens (4) and slot_mapping (5) disagree");
  b = valid_batch();
  b.block_tables.pop_back();
  EXPECT(validate_message(b) == "1 block tables for 2 sequences");
  b = valid_batch();
  b.slot_mapping[3] = 21;
  EXPECT(validate_message(b) == "two tokens both write KV cache slot 21");
  b = valid_batch();
  b.positions[1] = 9;
  EXPECT(validate_message(b) == "sequence 0 has non-contiguous positions at 1: 5 then 9");
  b = valid_batch();
  b.block_tables[0] = {4};
  EXPECT(validate_message(b) == "sequence 0 needs 2 blocks to cover 8 keys but its table has 1");
  b = valid_batch();
  b.logits_indices = {4};
  EXPECT(validate_message(b) == "logits index 4 is past the end of the batch");
}

TEST(elems_per_token_sums_the_layers, false) {
  EXPECT(PagedKvCache::elems_per_token({LayerLayout::Kv(8, 128), LayerLayout::Rows(64),
                                        LayerLayout::Kv(8, 128)}) == 2 * 2 * 8 * 128 + 64);
}

}  // namespace

int main(int argc, char** argv) {
  bool host_only = false;
  std::string filter;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--host-only")
      host_only = true;
    else
      filter = a;
  }
  int failed = 0, ran = 0;
  for (const auto& c : registry()) {
    if (host_only && c.gpu) continue;
    if (!filter.empty() && c.name.find(filter) == std::string::npos) continue;
    std::printf("%s ... ", c.name.c_str());
    std::fflush(stdout);
    g_failures.clear();
    c.fn();
    ++ran;
    if (g_failures.empty()) {
      std::printf("ok\n");
    } else {
      ++failed;
      std::printf("FAILED\n");
      for (const auto& f : g_failures) std::printf("    %s\n", f.c_str());
    }
    std::fflush(stdout);
  }
  std::printf("%d of %d passed\n", ran - failed, ran);
  return failed ? 1 : 0;
}
