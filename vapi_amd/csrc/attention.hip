// Paged attention over the block pool for gfx950: one varlen call covers
// decode rows (len_q == 1) and chunked-prefill rows (len_q > 1).
//
// Numerical contract: paged_attention_cpu (vapi
// crates/vapi-backend-candle/src/attention.rs:90-163): f32 scores
// q.k*scale, bottom-right-aligned causal mask (query j of a sequence sits at
// p = len_k - len_q + j), optional left window, softmax, times V, output cast
// to the input dtype. Masking follows the flash convention the reference's
// CUDA path passes (attention.rs:179-194): key k is visible iff
//   (window_right < 0 || k <= p + window_right) &&
//   (window_left  < 0 || k >= p - window_left).
//
// Kernels:
//  * paged_attn_generic  — VALU, any dtype/head_dim/GQA; one wave per
//    (query, head). Used for f32 pools and shapes the MFMA kernels skip.
//  * paged_decode_mfma   — 16-bit pools, split-K flash decoding. One
//    workgroup per (context partition, kv head, sequence); all G query heads
//    of a kv head ride one MFMA tile, so each K/V byte is read from HBM once.
//  * paged_decode_reduce — merges the per-partition (m, l, o) partials.
//  * paged_prefill_mfma  — 16-bit pools, rows = (query token, head) pairs of
//    one kv head, 16-row MFMA tiles, online softmax over 32-key steps.
//
// MFMA scheme (v_mfma_f32_16x16x32_{bf16,f16}; lane l: row/col = l%16,
// k-group g = l/16 holding 8 consecutive k):
//  * S^T = K Q^T: A = K tile (16 keys x 32 d, a lane loads 16 B of one key
//    row straight from HBM), B = Q^T (16 query rows). Result: lane holds
//    keys 4g..4g+3 of one query row (column l%16).
//  * O = P V: A = P, which is exactly the S^T lane layout reinterpreted with
//    the k-slots ordered as the 8 keys that lane already holds (4 from each
//    of two 16-key tiles). B = V: lane (g, n) loads the V rows of those same
//    8 keys at d = n*DPL .. n*DPL+DPL-1 and transposes the 8 x DPL tile in
//    registers, giving DPL B fragments; MFMA number k produces output
//    column n <-> d = n*DPL + k. No LDS round trip and no cross-lane moves
//    are needed for either operand.
#include "common.hpp"

namespace vk {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;  // running-max start: finite, so exp2 never sees inf-inf

struct AttnArgs {
  const char* k;  // layer K base
  const char* v;  // layer V base
  const char* q;
  char* out;
  const uint32_t* cu_q;
  const uint32_t* cu_k;
  const uint32_t* table;
  float* ws;  // split-K partials
  uint64_t blk_e, head_e, tok_e;  // element strides in the pool
  uint32_t max_blocks, batch, num_heads, kvh, group, block_size;
  uint32_t part_tokens, max_parts;
  float scale_log2;  // scale * log2(e)
  float scale;
  int32_t wl, wr;
};

__device__ __forceinline__ void key_range(int32_t p, int32_t len_k, int32_t wl,
                                          int32_t wr, int32_t& lo, int32_t& hi) {
  lo = wl >= 0 ? max(0, p - wl) : 0;
  hi = wr >= 0 ? min(len_k - 1, p + wr) : len_k - 1;
}

// ---------------------------------------------------------------------------
// Generic VALU kernel: one wave per (query token, query head).
// ---------------------------------------------------------------------------

template <typename T, int DPL>  // DPL = ceil(head_dim / 64)
__global__ __launch_bounds__(64) void paged_attn_generic(AttnArgs a,
                                                         uint32_t head_dim) {
  const uint32_t seq = blockIdx.z, h = blockIdx.y, j = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  const uint32_t q0 = a.cu_q[seq], len_q = a.cu_q[seq + 1] - q0;
  if (j >= len_q) return;
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const int32_t p = len_k - (int32_t)len_q + (int32_t)j;
  int32_t lo, hi;
  key_range(p, len_k, a.wl, a.wr, lo, hi);
  const uint32_t kh = h / a.group;

  __shared__ float qs[64 * DPL];
  __shared__ float ps[64];
  const T* qrow = (const T*)a.q + ((uint64_t)(q0 + j) * a.num_heads + h) * head_dim;
  for (uint32_t d = lane; d < 64 * DPL; d += 64)
    qs[d] = d < head_dim ? to_f32(qrow[d]) : 0.f;
  __syncthreads();

  const uint32_t* table = a.table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;

  float m = kNegBig, l = 0.f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;

  for (int32_t c0 = lo; c0 <= hi; c0 += 64) {
    const int32_t key = c0 + (int32_t)lane;
    float s = -INFINITY;
    if (key <= hi) {
      const uint32_t blk = table[key / a.block_size];
      const uint32_t off = key % a.block_size;
      const T* krow = kb + blk * a.blk_e + off * a.tok_e;
      float dot = 0.f;
      for (uint32_t d = 0; d < head_dim; ++d) dot += qs[d] * to_f32(krow[d]);
      s = dot * a.scale;
    }
    float cm = s;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
    const float mn = fmaxf(m, cm);
    const float alpha = __expf(m - mn);
    const float pv = key <= hi ? __expf(s - mn) : 0.f;
    float cs = pv;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cs += __shfl_xor(cs, o);
    l = l * alpha + cs;
    m = mn;
    ps[lane] = pv;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
    const int32_t nk = min(64, hi - c0 + 1);
    for (int32_t kk = 0; kk < nk; ++kk) {
      const int32_t key2 = c0 + kk;
      const uint32_t blk = table[key2 / a.block_size];
      const uint32_t off = key2 % a.block_size;
      const T* vrow = vb + blk * a.blk_e + off * a.tok_e;
      const float pk = ps[kk];
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const uint32_t d = lane + 64 * i;
        if (d < head_dim) acc[i] += pk * to_f32(vrow[d]);
      }
    }
    __syncthreads();
  }
  T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + h) * head_dim;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const uint32_t d = lane + 64 * i;
    if (d < head_dim) orow[d] = from_f32<T>(acc[i] * inv);
  }
}

// ---------------------------------------------------------------------------
// MFMA helpers
// ---------------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ floatx4 mfma16x16x32(uint4 a, uint4 b, floatx4 c);
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<bf16_t>(uint4 a, uint4 b,
                                                        floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<f16_t>(uint4 a, uint4 b,
                                                       floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(
      __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Pack two f32 into one dword of 16-bit values (lo first), RNE.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// Load DPL 16-bit elements (DPL*2 bytes) as dwords.
template <int DPL>
struct VRow {
  uint32_t w[DPL / 2];
};
template <int DPL>
__device__ __forceinline__ VRow<DPL> load_vrow(const void* p) {
  VRow<DPL> r;
  if constexpr (DPL == 8) {
    const uint4 x = *(const uint4*)p;
    r.w[0] = x.x; r.w[1] = x.y; r.w[2] = x.z; r.w[3] = x.w;
  } else if constexpr (DPL == 4) {
    const uint2 x = *(const uint2*)p;
    r.w[0] = x.x; r.w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < DPL / 8; ++i) {
      const uint4 x = ((const uint4*)p)[i];
      r.w[4 * i] = x.x; r.w[4 * i + 1] = x.y; r.w[4 * i + 2] = x.z; r.w[4 * i + 3] = x.w;
    }
  }
  return r;
}

// Column k (0..DPL-1) of the 8 x DPL tile held as 8 rows: 8 16-bit values,
// row j in slot j.
template <int DPL>
__device__ __forceinline__ uint4 vcol(const VRow<DPL> (&rows)[8], int k) {
  uint32_t w[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t x = rows[2 * m].w[k >> 1], y = rows[2 * m + 1].w[k >> 1];
    w[m] = (k & 1) ? ((x >> 16) | (y & 0xffff0000u))
                   : ((x & 0xffffu) | (y << 16));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float wave_max_g(float x) {  // over lanes l, l^16, l^32, l^48
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
__device__ __forceinline__ float wave_sum_g(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// ---------------------------------------------------------------------------
// Decode: split-K over context partitions, GQA group on the MFMA columns.
// ---------------------------------------------------------------------------

template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) void paged_decode_mfma(AttnArgs a) {
  constexpr int KC = D / 32;   // k-chunks of the QK contraction
  constexpr int DPL = D / 16;  // d values per lane in PV / output columns
  const uint32_t seq = blockIdx.z, kh = blockIdx.y, part = blockIdx.x;
  const uint32_t q0 = a.cu_q[seq];
  if (a.cu_q[seq + 1] - q0 != 1) return;  // prefill rows go elsewhere
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const uint32_t nparts = ((uint32_t)len_k + a.part_tokens - 1) / a.part_tokens;
  if (part >= nparts) return;

  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t col = lane & 15, g = lane >> 4;
  const int32_t p = len_k - 1;
  int32_t lo, hi;
  key_range(p, len_k, a.wl, a.wr, lo, hi);
  const int32_t pstart = (int32_t)(part * a.part_tokens);
  const int32_t pend = min(pstart + (int32_t)a.part_tokens, hi + 1);

  // Q^T operand: column = query head kh*G + col (zero past the group).
  uint4 qf[KC];
  {
    const bool real = col < a.group;
    const T* qrow = (const T*)a.q +
                    ((uint64_t)q0 * a.num_heads + kh * a.group + (real ? col : 0)) * D;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      qf[c] = real ? *(const uint4*)(qrow + 32 * c + 8 * g) : make_uint4(0, 0, 0, 0);
    }
  }

  const uint32_t* table = a.table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;

  float m_run = kNegBig, l_run = 0.f;
  floatx4 o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int32_t first = max(pstart, lo & ~31);
  for (int32_t s0 = first + 32 * (int32_t)wave; s0 < pend; s0 += 32 * NW) {
    // K tiles: this lane's key row in each 16-key tile.
    uint4 kf[2][KC];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int32_t key = min(s0 + 16 * tt + (int32_t)col, len_k - 1);
      const uint32_t blk = table[(uint32_t)key / a.block_size];
      const uint32_t off = (uint32_t)key % a.block_size;
      const T* kr = kb + blk * a.blk_e + off * a.tok_e + 8 * g;
#pragma unroll
      for (int c = 0; c < KC; ++c) kf[tt][c] = *(const uint4*)(kr + 32 * c);
    }
    // V rows of the 8 keys this lane's k-slots stand for.
    VRow<DPL> vr[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int32_t key = min(s0 + 16 * (jj >> 2) + 4 * (int32_t)g + (jj & 3), len_k - 1);
      const uint32_t blk = table[(uint32_t)key / a.block_size];
      const uint32_t off = (uint32_t)key % a.block_size;
      vr[jj] = load_vrow<DPL>(vb + blk * a.blk_e + off * a.tok_e + DPL * col);
    }
    // Scores.
    float s[8];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KC; ++c) acc = mfma16x16x32<T>(kf[tt][c], qf[c], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t key = s0 + 16 * tt + 4 * (int32_t)g + i;
        s[4 * tt + i] = (key >= lo && key <= hi && key < pend) ? acc[i] * a.scale_log2
                                                               : -INFINITY;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int jj = 1; jj < 8; ++jj) mx = fmaxf(mx, s[jj]);
    mx = wave_max_g(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float pr[8], psum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      pr[jj] = exp2f(s[jj] - m_new);
      psum += pr[jj];
    }
    l_run = l_run * alpha + psum;
    const uint4 pf = make_uint4(pack2<T>(pr[0], pr[1]), pack2<T>(pr[2], pr[3]),
                                pack2<T>(pr[4], pr[5]), pack2<T>(pr[6], pr[7]));
    // Output rows held by this lane are heads 4g..4g+3: their alpha lives in
    // columns 4g+i.
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[k][i] *= al[i];
      o[k] = mfma16x16x32<T>(pf, vcol<DPL>(vr, k), o[k]);
    }
  }
  l_run = wave_sum_g(l_run);

  // Merge the NW waves through LDS. Per wave: m[16], l[16], o[16][D].
  __shared__ float sm[NW][16], sl[NW][16];
  __shared__ float so[NW][16][D];
  if (g == 0) {
    sm[wave][col] = m_run;
    sl[wave][col] = l_run;
  }
#pragma unroll
  for (int k = 0; k < DPL; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[wave][4 * g + i][DPL * col + k] = o[k][i];
  __syncthreads();

  const uint32_t G = a.group;
  const bool single = nparts == 1;
  for (uint32_t idx = threadIdx.x; idx < G * D; idx += 64 * NW) {
    const uint32_t hh = idx / D, d = idx % D;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w][hh]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = exp2f(sm[w][hh] - M);
      L += sl[w][hh] * f;
      O += so[w][hh][d] * f;
    }
    const uint32_t hq = kh * G + hh;
    if (single) {
      T* orow = (T*)a.out + ((uint64_t)q0 * a.num_heads + hq) * D;
      orow[d] = from_f32<T>(L > 0.f ? O / L : 0.f);
    } else {
      const uint64_t pi = ((uint64_t)seq * a.num_heads + hq) * a.max_parts + part;
      float* ml = a.ws + pi * 2;
      float* po = a.ws + (uint64_t)a.batch * a.num_heads * a.max_parts * 2 + pi * D;
      po[d] = O;
      if (d == 0) {
        ml[0] = M;
        ml[1] = L;
      }
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(D) void paged_decode_reduce(AttnArgs a) {
  const uint32_t seq = blockIdx.y, hq = blockIdx.x, d = threadIdx.x;
  const uint32_t q0 = a.cu_q[seq];
  if (a.cu_q[seq + 1] - q0 != 1) return;
  const uint32_t len_k = a.cu_k[seq + 1] - a.cu_k[seq];
  const uint32_t nparts = (len_k + a.part_tokens - 1) / a.part_tokens;
  if (nparts <= 1) return;
  const uint64_t base = ((uint64_t)seq * a.num_heads + hq) * a.max_parts;
  const float* ml = a.ws + base * 2;
  const float* po = a.ws + (uint64_t)a.batch * a.num_heads * a.max_parts * 2 + base * D;
  float M = kNegBig;
  for (uint32_t i = 0; i < nparts; ++i) M = fmaxf(M, ml[2 * i]);
  float L = 0.f, O = 0.f;
  for (uint32_t i = 0; i < nparts; ++i) {
    const float f = exp2f(ml[2 * i] - M);
    L += ml[2 * i + 1] * f;
    O += po[(uint64_t)i * D + d] * f;
  }
  T* orow = (T*)a.out + ((uint64_t)q0 * a.num_heads + hq) * D;
  orow[d] = from_f32<T>(L > 0.f ? O / L : 0.f);
}

// ---------------------------------------------------------------------------
// Prefill: rows r = j*G + h_local of one kv head; RT 16-row tiles per wave.
// ---------------------------------------------------------------------------

template <typename T, int D, int RT, int NW>
__global__ __launch_bounds__(64 * NW) void paged_prefill_mfma(AttnArgs a) {
  constexpr int KC = D / 32;
  constexpr int DPL = D / 16;
  const uint32_t seq = blockIdx.z, kh = blockIdx.y;
  const uint32_t q0 = a.cu_q[seq];
  const uint32_t len_q = a.cu_q[seq + 1] - q0;
  if (len_q < 2) return;  // decode rows go to the decode kernel
  const uint32_t G = a.group;
  const uint32_t nrows = len_q * G;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t col = lane & 15, g = lane >> 4;
  const uint32_t row0 = (blockIdx.x * NW + wave) * 16 * RT;
  if (row0 >= nrows) return;
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const int32_t offset = len_k - (int32_t)len_q;

  // Q^T operands and the query position of each column row.
  uint4 qf[RT][KC];
  int32_t pos[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint32_t r = row0 + 16 * t + col;
    const bool real = r < nrows;
    const uint32_t j = real ? r / G : 0, hl = real ? r % G : 0;
    pos[t] = offset + (int32_t)j;
    const T* qrow = (const T*)a.q + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qf[t][c] = real ? *(const uint4*)(qrow + 32 * c + 8 * g) : make_uint4(0, 0, 0, 0);
  }
  // Key range of the whole wave.
  const uint32_t rlast = min(row0 + 16 * RT, nrows) - 1;
  const int32_t pmin = offset + (int32_t)(row0 / G), pmax = offset + (int32_t)(rlast / G);
  const int32_t klo = a.wl >= 0 ? max(0, pmin - a.wl) : 0;
  const int32_t khi = a.wr >= 0 ? min(len_k - 1, pmax + a.wr) : len_k - 1;

  const uint32_t* table = a.table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;

  float m_run[RT], l_run[RT];
  floatx4 o[RT][DPL];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m_run[t] = kNegBig;
    l_run[t] = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) o[t][k] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  for (int32_t s0 = klo & ~31; s0 <= khi; s0 += 32) {
    uint4 kf[2][KC];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int32_t key = min(s0 + 16 * tt + (int32_t)col, len_k - 1);
      const uint32_t blk = table[(uint32_t)key / a.block_size];
      const uint32_t off = (uint32_t)key % a.block_size;
      const T* kr = kb + blk * a.blk_e + off * a.tok_e + 8 * g;
#pragma unroll
      for (int c = 0; c < KC; ++c) kf[tt][c] = *(const uint4*)(kr + 32 * c);
    }
    VRow<DPL> vr[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int32_t key = min(s0 + 16 * (jj >> 2) + 4 * (int32_t)g + (jj & 3), len_k - 1);
      const uint32_t blk = table[(uint32_t)key / a.block_size];
      const uint32_t off = (uint32_t)key % a.block_size;
      vr[jj] = load_vrow<DPL>(vb + blk * a.blk_e + off * a.tok_e + DPL * col);
    }
    uint4 vf[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) vf[k] = vcol<DPL>(vr, k);

#pragma unroll
    for (int t = 0; t < RT; ++t) {
      float s[8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = mfma16x16x32<T>(kf[tt][c], qf[t][c], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int32_t key = s0 + 16 * tt + 4 * (int32_t)g + i;
          const bool vis = key < len_k && (a.wr < 0 || key <= pos[t] + a.wr) &&
                           (a.wl < 0 || key >= pos[t] - a.wl);
          s[4 * tt + i] = vis ? acc[i] * a.scale_log2 : -INFINITY;
        }
      }
      float mx = s[0];
#pragma unroll
      for (int jj = 1; jj < 8; ++jj) mx = fmaxf(mx, s[jj]);
      mx = wave_max_g(mx);
      const float m_new = fmaxf(m_run[t], mx);
      const float alpha = exp2f(m_run[t] - m_new);
      m_run[t] = m_new;
      float pr[8], psum = 0.f;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        pr[jj] = exp2f(s[jj] - m_new);
        psum += pr[jj];
      }
      l_run[t] = l_run[t] * alpha + psum;
      const uint4 pf = make_uint4(pack2<T>(pr[0], pr[1]), pack2<T>(pr[2], pr[3]),
                                  pack2<T>(pr[4], pr[5]), pack2<T>(pr[6], pr[7]));
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[t][k][i] *= al[i];
        o[t][k] = mfma16x16x32<T>(pf, vf[k], o[t][k]);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float lt = wave_sum_g(l_run[t]);
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = __shfl(lt, 4 * g + i);
      inv[i] = li > 0.f ? 1.f / li : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = row0 + 16 * t + 4 * g + i;
      if (r >= nrows) continue;
      const uint32_t j = r / G, hl = r % G;
      T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
      uint32_t w[DPL / 2];
#pragma unroll
      for (int k = 0; k < DPL / 2; ++k)
        w[k] = pack2<T>(o[t][2 * k][i] * inv[i], o[t][2 * k + 1][i] * inv[i]);
      if constexpr (DPL == 8) {
        *(uint4*)(orow + DPL * col) = make_uint4(w[0], w[1], w[2], w[3]);
      } else if constexpr (DPL == 4) {
        *(uint2*)(orow + DPL * col) = make_uint2(w[0], w[1]);
      } else {
#pragma unroll
        for (int k = 0; k < DPL / 8; ++k)
          ((uint4*)(orow + DPL * col))[k] =
              make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

constexpr int kDecodeWaves = 4;
constexpr int kPrefillRT = 2;
constexpr int kPrefillWaves = 4;

static uint32_t decode_part_tokens(uint32_t batch, uint32_t kvh, uint32_t max_k) {
  (void)batch;
  (void)kvh;
  (void)max_k;
  return 512;
}

static bool mfma_ok(const vapi_kv_pool* p, uint32_t num_heads) {
  if (p->dtype != VAPI_KV_BF16 && p->dtype != VAPI_KV_F16) return false;
  if (p->head_dim != 64 && p->head_dim != 128) return false;
  if (p->block_size % 16 != 0) return false;
  const uint32_t G = num_heads / p->num_kv_heads;
  return G >= 1 && G <= 16;
}

static uint32_t max_parts_for(const vapi_kv_pool* p, uint32_t batch,
                              uint32_t max_k) {
  const uint32_t pt = decode_part_tokens(batch, p->num_kv_heads, max_k);
  return (max_k + pt - 1) / pt;
}

template <typename T, int D>
static void launch_fast(const AttnArgs& a, uint32_t max_q, uint32_t max_k,
                        hipStream_t s) {
  const uint32_t parts = (max_k + a.part_tokens - 1) / a.part_tokens;
  if (parts > 0) {
    hipLaunchKernelGGL((paged_decode_mfma<T, D, kDecodeWaves>),
                       dim3(parts, a.kvh, a.batch), dim3(64 * kDecodeWaves), 0, s, a);
    if (parts > 1)
      hipLaunchKernelGGL((paged_decode_reduce<T, D>), dim3(a.num_heads, a.batch),
                         dim3(D), 0, s, a);
  }
  if (max_q > 1) {
    const uint32_t rows_per_wg = 16 * kPrefillRT * kPrefillWaves;
    const uint32_t gx = (max_q * a.group + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL((paged_prefill_mfma<T, D, kPrefillRT, kPrefillWaves>),
                       dim3(gx, a.kvh, a.batch), dim3(64 * kPrefillWaves), 0, s, a);
  }
}

template <typename T>
static void launch_generic(const AttnArgs& a, uint32_t head_dim, uint32_t max_q,
                           hipStream_t s) {
  const dim3 grid(max_q, a.num_heads, a.batch);
  if (head_dim <= 64)
    hipLaunchKernelGGL((paged_attn_generic<T, 1>), grid, dim3(64), 0, s, a, head_dim);
  else if (head_dim <= 128)
    hipLaunchKernelGGL((paged_attn_generic<T, 2>), grid, dim3(64), 0, s, a, head_dim);
  else
    hipLaunchKernelGGL((paged_attn_generic<T, 4>), grid, dim3(64), 0, s, a, head_dim);
}

}  // namespace vk

using namespace vk;

extern "C" {

size_t vapi_paged_attention_workspace_size(const vapi_kv_pool* pool,
                                           uint32_t batch, uint32_t num_heads,
                                           uint32_t max_seqlen_q,
                                           uint32_t max_seqlen_k) {
  (void)max_seqlen_q;
  if (!pool || pool->num_kv_heads == 0 || !mfma_ok(pool, num_heads)) return 0;
  const uint32_t mp = max_parts_for(pool, batch, max_seqlen_k);
  if (mp <= 1) return 0;
  return (size_t)batch * num_heads * mp * (pool->head_dim + 2) * sizeof(float);
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
  if (int rc = check_pool(pool, "vapi_paged_attention")) return rc;
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
  if (max_blocks == 0)
    VK_FAIL(VAPI_KV_EINVAL, "vapi_paged_attention: block table width 0");
  if (batch > 65535 || num_heads > 65535)
    VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: batch %u / heads %u too large",
            batch, num_heads);
  const size_t need = vapi_paged_attention_workspace_size(pool, batch, num_heads,
                                                          max_seqlen_q, max_seqlen_k);
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
  a.ws = (float*)workspace;
  a.blk_e = g.blk;
  a.head_e = g.head;
  a.tok_e = g.tok;
  a.max_blocks = max_blocks;
  a.batch = batch;
  a.num_heads = num_heads;
  a.kvh = g.kvh;
  a.group = num_heads / g.kvh;
  a.block_size = g.block_size;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.wl = window_left < 0 ? -1 : window_left;
  a.wr = window_right < 0 ? -1 : window_right;
  const hipStream_t s = hs(stream);

  if (mfma_ok(pool, num_heads)) {
    a.part_tokens = decode_part_tokens(batch, g.kvh, max_seqlen_k);
    a.max_parts = max_parts_for(pool, batch, max_seqlen_k);
    if (pool->dtype == VAPI_KV_BF16) {
      if (g.d == 128) launch_fast<bf16_t, 128>(a, max_seqlen_q, max_seqlen_k, s);
      else launch_fast<bf16_t, 64>(a, max_seqlen_q, max_seqlen_k, s);
    } else {
      if (g.d == 128) launch_fast<f16_t, 128>(a, max_seqlen_q, max_seqlen_k, s);
      else launch_fast<f16_t, 64>(a, max_seqlen_q, max_seqlen_k, s);
    }
  } else {
    if (g.d > 256)
      VK_FAIL(VAPI_KV_EUNSUP, "vapi_paged_attention: head_dim %u > 256", g.d);
    a.part_tokens = 0;
    a.max_parts = 0;
    switch (pool->dtype) {
      case VAPI_KV_F32: launch_generic<float>(a, g.d, max_seqlen_q, s); break;
      case VAPI_KV_BF16: launch_generic<bf16_t>(a, g.d, max_seqlen_q, s); break;
      default: launch_generic<f16_t>(a, g.d, max_seqlen_q, s); break;
    }
  }
  VK_LAUNCHED("paged_attention");
  return 0;
}

}  // extern "C"
