/*
 * CPU oracle for the paged KV hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of vapi's candle CPU path, used by tests/ as the
 * checker and by bench.py's cpu_baseline leg as the timed CPU baseline.
 * Nothing in the product (vapi_amd/) may link or call this.
 *
 * The reference (Rust, candle 0.11) cannot be built here: no cargo/rustc and
 * candle is not vendored. Each function below cites the reference code it
 * restates. Pools are in the reference's own layout (cache.rs:7-11):
 * per layer [num_blocks, block_size, num_kv_heads, head_dim], i.e. a flat
 * [num_slots, kvh, d] view addressed by slot = block*block_size + offset.
 *
 * Pinning (what checks each function beyond itself) is listed in
 * tests/test_oracle.py; every function here has at least one independent
 * check (reference known-answer vectors, closed forms, f64 brute force).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_SKIP 0xFFFFFFFFu

/* write_rows (crates/vapi-backend-candle/src/cache.rs:217-273).
 * pool: byte buffer of num_slots rows of row_bytes (kvh*d*elt).
 * src: n rows. Tokens whose slot is ORACLE_SKIP are dropped first (the
 * padded-slot convention, not present in the reference; see slot_mapping
 * docs). Returns 0, -1 if a slot is past the end (cache.rs:236-240), or the
 * number of runs as a positive count via *runs_out. force_scatter selects
 * the scatter branch (cache.rs:265-272) regardless of the run count.
 * nthreads > 1 spreads the copies over OpenMP threads (for timing the CPU
 * baseline on every core); the result equals the serial one only when no
 * two kept tokens share a slot, which is what callers passing it ensure. */
int oracle_write_rows(uint8_t* pool, uint64_t num_slots, uint64_t row_bytes,
                      const uint8_t* src, const uint32_t* slots, uint32_t n,
                      int force_scatter, uint32_t* runs_out, int nthreads) {
  uint32_t* keep = (uint32_t*)malloc(sizeof(uint32_t) * (n ? n : 1));
  uint32_t m = 0;
  for (uint32_t i = 0; i < n; ++i)
    if (slots[i] != ORACLE_SKIP) keep[m++] = i;
  /* cache.rs:236-240: the max slot must be inside the cache. */
  for (uint32_t i = 0; i < m; ++i)
    if ((uint64_t)slots[keep[i]] >= num_slots) {
      free(keep);
      return -1;
    }
  /* cache.rs:244-253: maximal runs of consecutive slots (over kept tokens;
   * a run also needs consecutive source rows). */
  uint32_t runs = 0;
  uint32_t start = 0;
  uint32_t* run_start = (uint32_t*)malloc(sizeof(uint32_t) * (m ? m : 1));
  uint32_t* run_end = (uint32_t*)malloc(sizeof(uint32_t) * (m ? m : 1));
  while (start < m) {
    uint32_t end = start + 1;
    while (end < m && slots[keep[end]] == slots[keep[end - 1]] + 1 &&
           keep[end] == keep[end - 1] + 1)
      ++end;
    run_start[runs] = start;
    run_end[runs] = end;
    ++runs;
    start = end;
  }
  if (runs_out) *runs_out = runs;
  if (runs <= 4 && !force_scatter) {
    /* cache.rs:255-263: one slice_set per run. */
    for (uint32_t r = 0; r < runs; ++r) {
      const uint32_t s0 = run_start[r], s1 = run_end[r];
      memcpy(pool + (uint64_t)slots[keep[s0]] * row_bytes,
             src + (uint64_t)keep[s0] * row_bytes, (uint64_t)(s1 - s0) * row_bytes);
    }
  } else {
    /* cache.rs:265-272: one scatter of every row to its slot. */
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
    for (uint32_t i = 0; i < m; ++i)
      memcpy(pool + (uint64_t)slots[keep[i]] * row_bytes,
             src + (uint64_t)keep[i] * row_bytes, row_bytes);
  }
  free(keep);
  free(run_start);
  free(run_end);
  return 0;
}

/* gather_kv (cache.rs:283-290): index_select the table's blocks, flatten to
 * (n_table*bs, kvh, d), keep the first len_k rows. Returns -1 if len_k
 * exceeds the table's slots (narrow would fail). */
int oracle_gather_kv(const uint8_t* pool, uint64_t block_bytes,
                     uint32_t block_size, const uint32_t* table,
                     uint32_t n_table, uint32_t len_k, uint8_t* out) {
  if ((uint64_t)len_k > (uint64_t)n_table * block_size) return -1;
  const uint64_t row = block_bytes / block_size;
  for (uint32_t t = 0; t < len_k; ++t) {
    const uint32_t blk = table[t / block_size];
    memcpy(out + (uint64_t)t * row,
           pool + (uint64_t)blk * block_bytes + (uint64_t)(t % block_size) * row, row);
  }
  return 0;
}

/* pack_block_tables (attention.rs:42-62). Returns the width. */
uint32_t oracle_pack_block_tables(uint32_t batch, const uint32_t* offsets,
                                  const uint32_t* data, uint32_t* out) {
  uint32_t width = 1;
  for (uint32_t i = 0; i < batch; ++i) {
    uint32_t n = offsets[i + 1] - offsets[i];
    if (n > width) width = n;
  }
  for (uint32_t i = 0; i < batch; ++i) {
    uint32_t n = offsets[i + 1] - offsets[i];
    uint32_t pad = n ? data[offsets[i + 1] - 1] : 0;
    for (uint32_t j = 0; j < width; ++j)
      out[(uint64_t)i * width + j] = j < n ? data[offsets[i] + j] : pad;
  }
  return width;
}

/* One sequence's attention, all heads — the body of the per-sequence loop in
 * paged_attention_cpu (attention.rs:105-158), in f32:
 *   qi  = q[q0..q0+len_q] as (heads, len_q, d)                 (:115-119)
 *   ki/vi = gather_kv(...) as (kv_heads, len_k, d), repeated
 *           n_rep = heads/kv_heads times (repeat_kv)           (:121-134)
 *   att = qi @ ki^T * scale                                    (:136)
 *   mask: k > p, or (window w) k < p && p - k >= w, with
 *         p = len_k - len_q + j                                (:139-154)
 *   softmax_last_dim; y = att @ vi                             (:155-156)
 * window_right extends the reference (which is always causal) to the flash
 * parameterisation: < 0 removes the k > p condition, else k > p + wr.
 * kc/vc are the layer's f32 pools [slots, kvh, d]. */
static void attend_one(const float* q, uint32_t q0, uint32_t len_q,
                       uint32_t len_k, const float* kc, const float* vc,
                       const uint32_t* table, uint32_t block_size,
                       uint32_t heads, uint32_t kvh, uint32_t d, float scale,
                       int32_t window, int32_t window_right, float* out,
                       float* att /* len_k scratch */) {
  const uint32_t n_rep = heads / kvh;
  const uint32_t offset = len_k - len_q;
  for (uint32_t h = 0; h < heads; ++h) {
    const uint32_t kh = h / n_rep; /* repeat_kv: head h reads kv head h / n_rep */
    for (uint32_t j = 0; j < len_q; ++j) {
      const float* qr = q + ((uint64_t)(q0 + j) * heads + h) * d;
      const uint32_t p = offset + j;
      float mx = -INFINITY;
      for (uint32_t k = 0; k < len_k; ++k) {
        const uint64_t slot = (uint64_t)table[k / block_size] * block_size + k % block_size;
        const float* kr = kc + (slot * kvh + kh) * d;
        float dot = 0.f;
        for (uint32_t x = 0; x < d; ++x) dot += qr[x] * kr[x];
        float s = dot * scale;
        int hidden = window_right < 0 ? 0 : (k > p + (uint32_t)window_right);
        if (window >= 0 && k < p && p - k >= (uint32_t)window) hidden = 1;
        att[k] = hidden ? -INFINITY : s;
        if (att[k] > mx) mx = att[k];
      }
      /* softmax_last_dim: exp(x - max) / sum */
      float sum = 0.f;
      for (uint32_t k = 0; k < len_k; ++k) {
        att[k] = expf(att[k] - mx);
        sum += att[k];
      }
      for (uint32_t k = 0; k < len_k; ++k) att[k] /= sum;
      float* yr = out + ((uint64_t)(q0 + j) * heads + h) * d;
      for (uint32_t x = 0; x < d; ++x) yr[x] = 0.f;
      for (uint32_t k = 0; k < len_k; ++k) {
        const uint64_t slot = (uint64_t)table[k / block_size] * block_size + k % block_size;
        const float* vr = vc + (slot * kvh + kh) * d;
        const float w = att[k];
        for (uint32_t x = 0; x < d; ++x) yr[x] += w * vr[x];
      }
    }
  }
}

/* paged_attention_cpu (attention.rs:90-163) over a ragged batch.
 * q/out: [cu_q[batch], heads, d] f32. tables: ragged (offsets[batch+1]).
 * window: sliding window w (HF q - k < w), -1 for None.
 * Sequences with len_q == 0 are skipped (:109-111). nthreads > 1 runs
 * sequences in parallel (OpenMP), for the CPU baseline timing. */
void oracle_paged_attention(const float* q, const float* kc, const float* vc,
                            const uint32_t* cu_q, const uint32_t* cu_k,
                            uint32_t batch, const uint32_t* tbl_off,
                            const uint32_t* tbl, uint32_t block_size,
                            uint32_t heads, uint32_t kvh, uint32_t d,
                            float scale, int32_t window, int32_t window_right,
                            float* out, int nthreads) {
  uint32_t max_k = 1;
  for (uint32_t i = 0; i < batch; ++i) {
    uint32_t lk = cu_k[i + 1] - cu_k[i];
    if (lk > max_k) max_k = lk;
  }
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    float* att = (float*)malloc(sizeof(float) * max_k);
#pragma omp for schedule(dynamic, 1)
    for (uint32_t i = 0; i < batch; ++i) {
      const uint32_t q0 = cu_q[i], len_q = cu_q[i + 1] - q0;
      const uint32_t len_k = cu_k[i + 1] - cu_k[i];
      if (len_q == 0) continue;
      attend_one(q, q0, len_q, len_k, kc, vc, tbl + tbl_off[i], block_size, heads,
                 kvh, d, scale, window, window_right, out, att);
    }
    free(att);
  }
}

/* Dense causal attention over one sequence in f64 — the hand-written oracle
 * of attention.rs:297-321 (dense_causal), extended with GQA and the window.
 * q: [len_q, heads, d]; k, v: [len_k, kvh, d] (logical order); out f64. */
void oracle_dense_attention_f64(const double* q, const double* k,
                                const double* v, uint32_t len_q, uint32_t len_k,
                                uint32_t heads, uint32_t kvh, uint32_t d,
                                double scale, int32_t window,
                                int32_t window_right, double* out) {
  const uint32_t n_rep = heads / kvh;
  double* w = (double*)malloc(sizeof(double) * (len_k ? len_k : 1));
  for (uint32_t h = 0; h < heads; ++h) {
    const uint32_t kh = h / n_rep;
    for (uint32_t j = 0; j < len_q; ++j) {
      const int64_t p = (int64_t)len_k - len_q + j;
      double mx = -INFINITY;
      for (uint32_t t = 0; t < len_k; ++t) {
        int vis = 1;
        if (window_right >= 0 && (int64_t)t > p + window_right) vis = 0;
        if (window >= 0 && (int64_t)t < p && p - t >= window) vis = 0;
        if (!vis) {
          w[t] = -INFINITY;
          continue;
        }
        double s = 0;
        for (uint32_t x = 0; x < d; ++x)
          s += q[((uint64_t)j * heads + h) * d + x] * k[((uint64_t)t * kvh + kh) * d + x];
        w[t] = s * scale;
        if (w[t] > mx) mx = w[t];
      }
      double z = 0;
      for (uint32_t t = 0; t < len_k; ++t) {
        w[t] = w[t] == -INFINITY ? 0.0 : exp(w[t] - mx);
        z += w[t];
      }
      for (uint32_t x = 0; x < d; ++x) {
        double acc = 0;
        for (uint32_t t = 0; t < len_k; ++t) acc += w[t] / z * v[((uint64_t)t * kvh + kh) * d + x];
        out[((uint64_t)j * heads + h) * d + x] = acc;
      }
    }
  }
  free(w);
}

/* The block methods below take the cache's buffers in the reference's
 * iteration order, k[0..L] ++ v[0..L] (backend.rs:697-700, 720, 751-757),
 * as `nbuf` pointers with each buffer's per-block byte count (the product of
 * its dims past the first, times the element size). A buffer that is not
 * at least rank 2 (a rows layer's empty V, cache.rs:96) is passed as NULL
 * with 0 bytes and skipped, as the reference skips it. */

/* block_bytes (backend.rs:695-708): the sum of the per-block bytes. */
uint64_t oracle_block_bytes(const uint64_t* blk_bytes, uint32_t nbuf) {
  uint64_t sum = 0;
  for (uint32_t i = 0; i < nbuf; ++i) sum += blk_bytes[i];
  return sum;
}

/* export_block (backend.rs:718-734): each buffer's block `id`, flattened,
 * concatenated in buffer order. */
void oracle_export_block(uint8_t* const* bufs, const uint64_t* blk_bytes, uint32_t nbuf,
                         uint32_t id, uint8_t* out) {
  uint64_t at = 0;
  for (uint32_t i = 0; i < nbuf; ++i) {
    if (!bufs[i] || !blk_bytes[i]) continue;
    memcpy(out + at, bufs[i] + (uint64_t)id * blk_bytes[i], blk_bytes[i]);
    at += blk_bytes[i];
  }
}

/* import_block (backend.rs:738-773): the length must equal block_bytes,
 * then the same order is sliced back. Returns -1 on a length mismatch. */
int oracle_import_block(uint8_t* const* bufs, const uint64_t* blk_bytes, uint32_t nbuf,
                        uint32_t id, const uint8_t* bytes, uint64_t len) {
  if (len != oracle_block_bytes(blk_bytes, nbuf)) return -1;
  uint64_t at = 0;
  for (uint32_t i = 0; i < nbuf; ++i) {
    if (!bufs[i] || !blk_bytes[i]) continue;
    memcpy(bufs[i] + (uint64_t)id * blk_bytes[i], bytes + at, blk_bytes[i]);
    at += blk_bytes[i];
  }
  return 0;
}

/* copy_blocks (backend.rs:781-797): pairs in order; for each, every layer,
 * K then V (`nbuf` = 2L, k[l] at l and v[l] at L + l), dst := src.
 * nthreads > 1 spreads the pairs over OpenMP threads (CPU-baseline timing);
 * that equals the ordered result only when no destination is also a source
 * or a second destination, which callers passing it ensure. */
void oracle_copy_blocks(uint8_t* const* bufs, const uint64_t* blk_bytes, uint32_t nbuf,
                        const uint32_t* pairs, uint32_t n_pairs, int nthreads) {
  const uint32_t layers = nbuf / 2;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (uint32_t p = 0; p < n_pairs; ++p) {
    const uint32_t src = pairs[2 * p], dst = pairs[2 * p + 1];
    for (uint32_t l = 0; l < layers; ++l)
      for (uint32_t kv = 0; kv < 2; ++kv) {
        const uint32_t i = kv * layers + l;
        if (!bufs[i] || !blk_bytes[i]) continue;
        memmove(bufs[i] + (uint64_t)dst * blk_bytes[i], bufs[i] + (uint64_t)src * blk_bytes[i],
                blk_bytes[i]);
      }
  }
}
