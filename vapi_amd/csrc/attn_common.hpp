// Shared pieces of the gfx950 paged-attention kernels: argument block, MFMA
// operand helpers and the 32-key online-softmax step used by both the decode
// and the prefill kernels.
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
// MFMA scheme (v_mfma_f32_16x16x32_{bf16,f16}; lane l: row/col = l%16,
// k-group g = l/16 holding 8 consecutive k):
//  * S^T = K Q^T: A = K tile (16 keys x 32 d, a lane loads 16 B of one key
//    row straight from HBM), B = Q^T (16 query rows). Result: lane holds
//    keys 4g..4g+3 of one query row (column l%16).
//  * O = P V: A = P, which is exactly the S^T lane layout reinterpreted with
//    the k-slots ordered as the 8 keys that lane already holds (4 from each
//    of two 16-key tiles). B = V: lane (g, n) loads the V rows of those same
//    8 keys at d = n*DPL .. n*DPL+DPL-1 and transposes the 8 x DPL tile in
//    registers (v_perm_b32), giving DPL B fragments; MFMA number k produces
//    output column n <-> d = n*DPL + k. No LDS round trip and no cross-lane
//    moves are needed for either operand.
#pragma once

#include "common.hpp"

namespace vk {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;  // running-max start: finite, so exp2 never sees inf-inf
constexpr float kRescaleSlack = 8.0f;  // log2 units the running max may lag by

struct AttnArgs {
  const char* k;  // layer K base
  const char* v;  // layer V base
  const char* q;
  char* out;
  const uint32_t* cu_q;
  const uint32_t* cu_k;
  const uint32_t* table;
  uint32_t* seg_ranges;  // decode: first and last range of each (sequence, kv head) segment
  float* ws_ml;        // decode: partial (m, l) per slot and head
  float* ws_o;         // decode: partial outputs per slot and head
  uint32_t* bal;       // decode: XCD shares and per-wave timings, kept across launches
  // Fused append (decode only; null otherwise): the step's new K/V rows
  // [n_new, kvh, D] and their slots.
  const char* k_new;
  const char* v_new;
  const uint32_t* slots;
  uint32_t n_new, num_slots;
  uint32_t last_blk;  // num_blocks - 1: table entries are clamped to it
  uint64_t blk_e, head_e;  // element strides in the pool
  uint32_t tok_e;
  uint32_t max_blocks, batch, num_heads, kvh, group, block_size, bs_shift;
  uint32_t num_waves;  // decode: persistent waves in the grid
  float scale_log2;    // |scale| * log2(e) (MFMA paths: Q is negated when scale < 0)
  float scale;
  uint32_t q_sign;     // 0x80008000 when scale < 0: XOR into packed 16-bit Q words
  int32_t wl, wr;
  uint32_t deterministic;  // decode: fixed equal XCD shares, no share update
  uint32_t pf_min_q;       // prefill: rows with len_q >= this (2, or 1 when no decode launch)
  // prefill: the sequences its grid covers, u32[pf_seqs_n] (null: 0 ..
  // batch - 1); the host names the sequences with prefill rows.
  const uint32_t* pf_seqs;
  uint32_t pf_seqs_n;
  // decode: a group of G > 16 query heads per kv head runs as n = kv_parts
  // virtual kv heads of P = group = ceil(G / n) query heads each (kvh and
  // group then count the virtual ones; the last part of a group may hold
  // fewer): virtual head v reads the K/V of pool head v / n and serves query
  // heads (v / n) G + (v % n) P + c for c < min(P, G - (v % n) P). g_real
  // is G (n = 1: group).
  FastDiv kv_parts;
  uint32_t g_real;
  // The pool's head_dim. The decode also runs head dims that are not a
  // kernel's D (a multiple of 8 up to 256) at the next of 64, 128 or 256:
  // elements d >= hd are loaded as zeros and not stored.
  uint32_t hd;
};

__device__ __forceinline__ void key_range(int32_t p, int32_t len_k, int32_t wl,
                                          int32_t wr, int32_t& lo, int32_t& hi) {
  lo = wl >= 0 ? max(0, p - wl) : 0;
  hi = wr >= 0 ? min(len_k - 1, p + wr) : len_k - 1;
}

// Workgroup -> work item. The hardware deals workgroups round-robin to the
// 8 XCDs (linear id % 8); each XCD here gets a contiguous range of work
// items, so the q-tiles of one (sequence, kv head), which read the same K/V,
// run at the same time under one L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t lin, uint32_t n) {
  constexpr uint32_t kXcds = 8;
  const uint32_t x = lin % kXcds, i = lin / kXcds;
  const uint32_t per = n / kXcds, extra = n % kXcds;  // XCD x gets per + (x < extra)
  return x * per + min(x, extra) + i;
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

typedef float float2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Pack two f32 into one dword of 16-bit values (lo first), round to nearest
// even (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 style conversions).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{lo, hi}, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{lo, hi}, f16x2));
}

template <typename T>
__device__ __forceinline__ uint4 pack8(const float (&p)[8]) {
  return make_uint4(pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]),
                    pack2<T>(p[6], p[7]));
}

// DPL 16-bit elements (DPL*2 bytes) of one row, as dwords.
template <int DPL>
struct VRow {
  uint32_t w[DPL / 2];
};
template <int DPL, bool kNt = true>
__device__ __forceinline__ VRow<DPL> load_vrow(const void* p) {
  VRow<DPL> r;
  if constexpr (DPL == 4) {
    const uint2 x = load_kv<kNt>((const uint2*)p);
    r.w[0] = x.x; r.w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < DPL / 8; ++i) {
      const uint4 x = load_kv<kNt>((const uint4*)p + i);
      r.w[4 * i] = x.x; r.w[4 * i + 1] = x.y; r.w[4 * i + 2] = x.z; r.w[4 * i + 3] = x.w;
    }
  }
  return r;
}

// Column k (0..DPL-1) of the 8 x DPL tile held as 8 rows: 8 16-bit values,
// row j in slot j. One v_perm_b32 per output dword.
template <int DPL>
__device__ __forceinline__ uint4 vcol(const VRow<DPL> (&rows)[8], int k) {
  const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
  uint32_t w[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    w[m] = __builtin_amdgcn_perm(rows[2 * m + 1].w[k >> 1], rows[2 * m].w[k >> 1], sel);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Reductions over the four lane groups l, l^16, l^32, l^48 with the gfx950
// lane-swap instructions (no LDS round trip): permlane32_swap of x with
// itself leaves (lower half, lower half) in one result and (upper, upper)
// in the other, permlane16_swap does the same for odd/even 16-lane rows.
// Kernels run with the IEEE mode bit clear and no NaN inputs, so fmaxf
// needs no quieting of its operands (see the build flags).
__device__ __forceinline__ float max_nc(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float max3_nc(float a, float b, float c) {
  return fmaxf(fmaxf(a, b), c);
}
__device__ __forceinline__ float wave_max_g(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nc(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float wave_sum_g(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K and V of one 32-key step (two 16-key tiles) in MFMA operand order.
//  KTile::k[tt][c]: this lane's key row (tile tt, key col) at d = 32c + 8g .. +8.
//  VTile::v[j]: the V row of key slot j (tile j/4, key 4g + j%4) at
//  d = v_d(col, 0 .. DPL - 1) (DPL*col .. +DPL below head_dim 256).
template <int D>
struct KTile {
  uint4 k[2][D / 32];
};
template <int D>
struct VTile {
  VRow<D / 16> v[8];
};
template <int D>
struct KVStep {
  KTile<D> k;
  VTile<D> v;
};

// Loads of a step whose first key s0 is a multiple of 32. Every load stays
// inside a block the table names: a tile past the sequence's final key
// `last` re-reads the tile holding `last`, and keys past `last` read `last`
// itself (all of them are masked out of the softmax, and V rows are finite
// data, so p = 0 removes them exactly). Loads are unconditional, so the
// tiles need no zero-fill. The block id of a 16-key tile is wave-uniform
// (block_size is a power of two >= 16) and comes through the scalar cache;
// per-lane addresses are 32-bit byte offsets from that uniform base.
template <typename T>
__device__ __forceinline__ const char* tile_base(const uint32_t* __restrict__ tab, const T* base,
                                                 const AttnArgs& a, int32_t ts) {
  // Read through the constant address space: the block table is never
  // written by a kernel, and this keeps the load scalar wherever it is
  // inlined (a restrict qualifier does not survive every inlining).
  using ConstU32 = const __attribute__((address_space(4))) uint32_t;
  // Clamped: a table entry past the pool reads the last block, and keys
  // past the table's row (len_k beyond max_blocks * block_size) its last
  // entry, instead of faulting (ForwardBatch::validate is where bad tables
  // are refused).
  const uint32_t col = min((uint32_t)ts >> a.bs_shift, a.max_blocks - 1);
  const uint32_t blk = min(((ConstU32*)tab)[col], a.last_blk);
  const uint32_t off0 = (uint32_t)ts & (a.block_size - 1);
  return (const char*)(base + (uint64_t)blk * a.blk_e + (uint64_t)off0 * a.tok_e);
}

// K and V tiles of the 32-key step at s0 (keys past `last` re-read it). With
// `knew` / `vnew` (the row's new key, D contiguous elements) key `last` is
// read from there instead of the pool: a per-lane address select, no branch.
// KCL: the 32-column chunks of K that are loaded (the rest, padding, are
// left as they were; fewer than D / 32 only with kPad).
// kNt: streaming loads (each tile is read once per call); ordinary ones
// when the virtual kv heads of a split group read the same tiles.
template <typename T, int D, bool kPad = false, int KCL = D / 32, bool kNt = true>
__device__ __forceinline__ void load_k(KTile<D>& st, const uint32_t* __restrict__ tab,
                                       const T* kb, const AttnArgs& a, int32_t s0, int32_t last,
                                       uint32_t col, uint32_t g, const char* knew = nullptr) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int32_t ts = min(s0 + 16 * tt, last & ~15);
    const char* kt = tile_base(tab, kb, a, ts);
    const uint32_t kr = ((uint32_t)min((int32_t)col, last - ts) * a.tok_e + 8 * g) * sizeof(T);
    const char* src = kt + kr;
    if (knew != nullptr && (int32_t)col >= last - ts) src = knew + 8 * g * sizeof(T);
#pragma unroll
    for (int c = 0; c < KCL; ++c) {
      if constexpr (kPad)
        st.k[tt][c] = 32 * c + 8 * g < a.hd ? load_kv<kNt>((const uint4*)(src + 64u * c))
                                             : make_uint4(0u, 0u, 0u, 0u);
      else
        st.k[tt][c] = load_kv<kNt>((const uint4*)(src + 64u * c));
    }
  }
}

// The d index of V value k (0..D/16-1) that lane column m holds: DPL
// consecutive values from DPL m, or at head_dim 256 two runs of 8, d = 8 m +
// k and 128 + 8 m + k - 8 (so that every V load reads whole rows).
template <int D>
__host__ __device__ constexpr uint32_t v_d(uint32_t m, int k) {
  return D == 256 ? (uint32_t)(k >> 3) * 128 + 8 * m + (uint32_t)(k & 7)
                  : (uint32_t)(D / 16) * m + (uint32_t)k;
}
template <int D>
__host__ __device__ constexpr uint32_t v_col0(uint32_t m) { return v_d<D>(m, 0); }

template <typename T, int D, bool kPad = false, bool kNt = true>
__device__ __forceinline__ void load_v(VTile<D>& st, const uint32_t* __restrict__ tab,
                                       const T* vb, const AttnArgs& a, int32_t s0, int32_t last,
                                       uint32_t col, uint32_t g, const char* vnew = nullptr) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int32_t ts = min(s0 + 16 * tt, last & ~15);
    const char* vt = tile_base(tab, vb, a, ts);
    const int32_t lim = last - ts;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t vr =
          ((uint32_t)min((int32_t)(4 * g + i), lim) * a.tok_e + v_col0<D>(col)) * sizeof(T);
      const char* src = vt + vr;
      if (vnew != nullptr && (int32_t)(4 * g + i) >= lim) src = vnew + v_col0<D>(col) * sizeof(T);
      if constexpr (D == 256) {
        // Two 16-byte runs, d = 8 col .. +7 and 128 + 8 col .. +7: each load
        // instruction then reads whole 256-byte rows across the 16 lanes.
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        const uint4 x0 = !kPad || v_d<D>(col, 0) < a.hd ? load_kv<kNt>((const uint4*)src) : z;
        const uint4 x1 = !kPad || v_d<D>(col, 8) < a.hd
                             ? load_kv<kNt>((const uint4*)(src + 128 * sizeof(T))) : z;
        VRow<DPL>& w = st.v[4 * tt + i];
        w.w[0] = x0.x, w.w[1] = x0.y, w.w[2] = x0.z, w.w[3] = x0.w;
        w.w[4] = x1.x, w.w[5] = x1.y, w.w[6] = x1.z, w.w[7] = x1.w;
      } else if constexpr (kPad) {
        if (v_col0<D>(col) < a.hd) {
          st.v[4 * tt + i] = load_vrow<DPL, kNt>(src);
        } else {
#pragma unroll
          for (int w = 0; w < DPL / 2; ++w) st.v[4 * tt + i].w[w] = 0u;
        }
      } else {
        st.v[4 * tt + i] = load_vrow<DPL, kNt>(src);
      }
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ void load_kv_step(KVStep<D>& st, const uint32_t* __restrict__ tab,
                                             const T* kb, const T* vb, const AttnArgs& a,
                                             int32_t s0, int32_t last, uint32_t col,
                                             uint32_t g) {
  load_k<T, D>(st.k, tab, kb, a, s0, last, col, g);
  load_v<T, D>(st.v, tab, vb, a, s0, last, col, g);
}

// Scores S^T = K Q^T of a 32-key step for 16 query rows: acc[tt][i] is key
// 16 tt + 4 g + i of this lane's row.
// KC: the 32-column chunks of d that take part (fewer than D / 32 when the
// rest are padding).
template <typename T, int D, int KC = D / 32>
__device__ __forceinline__ void qk_scores(const KTile<D>& kt, const uint4 (&qf)[D / 32],
                                          floatx4 (&acc)[2]) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    acc[tt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KC; ++c) acc[tt] = mfma16x16x32<T>(kt.k[tt][c], qf[c], acc[tt]);
  }
}

// Lazy rescale of 16 rows given each lane's max mx over its keys (scaled
// log2 units): rows whose max grew by more than 2^kRescaleSlack take the row
// max across the four lane groups and rescale O and l to it.
// DPL: the 16-column d tiles of O that are live (fewer than D / 16 when the
// rest are padding).
template <int D, int DPL = D / 16>
__device__ __forceinline__ void rescale_rows(float mx, floatx4 (&o)[D / 16], float& m_run,
                                             float& l_run) {
  if (__any(mx > m_run + kRescaleSlack)) {
    const float m_new = fmaxf(m_run, wave_max_g(mx));
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int k = 0; k < DPL; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[k][i] *= alpha;
  }
}

// P = exp2(s * c - m) for a lane's 8 scores, added to l and packed in the
// input dtype.
template <typename T>
__device__ __forceinline__ uint4 exp_pack(const float (&s)[8], float m_run, float& l_run,
                                          float scale_log2) {
  float p[8];
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = fast_exp2(__builtin_fmaf(s[j], scale_log2, -m_run));
    ps += p[j];
  }
  l_run += ps;
  return pack8<T>(p);
}

// First half of an online-softmax step for 16 query rows (the MFMA
// columns): scores S^T = K Q^T, lazy rescale of the running max (and of O),
// returns P packed in the input dtype as the PV A operand.
// `visible(i_tile, i)` masks key slot (tt, 4g+i). m_run is kept in scaled
// log2 units; scale_log2 >= 0, so the max is taken on the raw scores and the
// scale folds into one FMA per score: p = exp2(s * c - m).
// KC: the 32-column chunks of d in the scores (fewer than D / 32 when the
// rest are padding).
template <typename T, int D, int KC = D / 32, typename Mask>
__device__ __forceinline__ uint4 attend_qk(const KTile<D>& kt, const uint4 (&qf)[D / 32],
                                           floatx4 (&o)[D / 16], float& m_run, float& l_run,
                                           float scale_log2, uint32_t g, Mask visible) {
  constexpr int DPL = D / 16;
  float s[8];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KC; ++c) acc = mfma16x16x32<T>(kt.k[tt][c], qf[c], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[4 * tt + i] = visible(tt, i) ? acc[i] : -INFINITY;
  }
  // This lane's max over its 8 keys. m_run is the same in the four lane
  // groups that hold a row, so comparing each lane's own max with it finds
  // every row whose max grew by more than 2^kRescaleSlack; only then is the
  // row max reduced across the groups and the row rescaled (the same
  // softmax; P stays below 2^kRescaleSlack).
  const float mx = max3_nc(max3_nc(s[0], s[1], s[2]), max3_nc(s[3], s[4], s[5]),
                           max_nc(s[6], s[7])) * scale_log2;
  if (__any(mx > m_run + kRescaleSlack)) {
    const float m_new = fmaxf(m_run, wave_max_g(mx));
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int k = 0; k < DPL; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[k][i] *= alpha;
  }
  float p[8];
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = fast_exp2(__builtin_fmaf(s[j], scale_log2, -m_run));
    ps += p[j];
  }
  l_run += ps;
  return pack8<T>(p);
}

// Second half: O^T += V^T P^T. The V fragments are the A operand (MFMA k's
// row m <-> d = v_d(m, k), DPL*m + k below head_dim 256) and P^T is the B
// operand exactly as the score layout left it, so the result lands as lane
// (g, col) holding query row col at d = v_d(4g + i, k) (i = 0..3, k =
// 0..DPL-1): every lane's accumulators
// belong to its own row, and rescaling needs no cross-lane traffic.
template <typename T, int D>
__device__ __forceinline__ void attend_pv(const VTile<D>& vt, uint4 pf, floatx4 (&o)[D / 16]) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = mfma16x16x32<T>(vcol<DPL>(vt.v, k), pf, o[k]);
}

// Store row `col`'s outputs d = v_d(4g + i, k) of o, scaled, to `row`
// (16-bit output; DPL-wide runs, or two runs of 8 at head_dim 256).
template <typename T, int D, bool kPad = false>
__device__ __forceinline__ void store_row(T* row, const floatx4 (&o)[D / 16], float scale,
                                          uint32_t g, uint32_t hd = D) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w[DPL / 2];
#pragma unroll
    for (int k = 0; k < DPL / 2; ++k)
      w[k] = pack2<T>(o[2 * k][i] * scale, o[2 * k + 1][i] * scale);
    if constexpr (D == 256) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (!kPad || v_d<D>(4 * g + i, 8 * h) < hd)
          *(uint4*)(row + v_d<D>(4 * g + i, 8 * h)) =
              make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]);
      continue;
    }
    if (kPad && DPL * (4 * g + i) >= hd) continue;  // padding columns
    T* dst = row + DPL * (4 * g + i);
    if constexpr (DPL == 4) {
      *(uint2*)dst = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int k = 0; k < DPL / 8; ++k)
        ((uint4*)dst)[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
    }
  }
}

template <typename T, int D, typename Mask>
__device__ __forceinline__ void attend_step(const KVStep<D>& st, const uint4 (&qf)[D / 32],
                                            floatx4 (&o)[D / 16], float& m_run, float& l_run,
                                            float scale_log2, uint32_t g, Mask visible) {
  const uint4 pf = attend_qk<T, D>(st.k, qf, o, m_run, l_run, scale_log2, g, visible);
  attend_pv<T, D>(st.v, pf, o);
}

// ---- f32 pools: v_mfma_f32_16x16x4_f32 --------------------------------------
//
// The same operand scheme at K = 4 per MFMA, one 16-key tile (a half step)
// at a time. S^T = K Q^T: lane (key r, g) loads K[r][16c + 4g .. +3] as one
// float4 per c, element j feeding MFMA (c, j), whose k-slot g is d = 16c +
// 4g + j; lane (col, g) supplies Q[col] at the same d. The result is the
// 16-bit path's score layout: lane (col, g) holds keys 4g .. 4g + 3 of the
// tile for query column col. O^T += V^T P^T: MFMA (i) takes key 4g + i in
// k-slot g, so its B operand is the lane's own score p[i]; its A operand is
// V[4g + i][d] with output row m <-> d = 64h + 4m + j for d tile t = 4h + j,
// from one float4 V[4g + i][64h + 4m .. +3] per (i, h). Lane (col, g) then
// holds output d = 64h + 16g + 4i + j in o[4h + j][i]. P stays f32.
template <int D>
struct KHalfF32 {
  float4 k[D / 16];
};
template <int D>
struct VHalfF32 {
  float4 v[4][D / 64];
};
template <int D>
struct KTileF32 {
  KHalfF32<D> h[2];
};
template <int D>
struct VTileF32 {
  VHalfF32<D> h[2];
};

__device__ __forceinline__ floatx4 mfma16x16x4f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// K and V of the 16-key tile at s0 + 16 tt (keys past `last` re-read it).
// kStream: streaming loads (the decode reads each byte once); the prefill's
// waves share a kv head's K/V through L2 and load them the ordinary way.
// CL: the 16-column chunks of K that are loaded (fewer than D / 16 when the
// rest are padding; those stay as they were).
template <int D, bool kStream = true, bool kPad = false, int CL = D / 16>
__device__ __forceinline__ void load_half_f32(KHalfF32<D>& kt, VHalfF32<D>& vt,
                                              const uint32_t* __restrict__ tab, const float* kb,
                                              const float* vb, const AttnArgs& a, int32_t s0,
                                              int tt, int32_t last, uint32_t col, uint32_t g) {
  const int32_t ts = min(s0 + 16 * tt, last & ~15);
  const int32_t lim = last - ts;
  const char* kp = tile_base(tab, kb, a, ts) +
                   ((uint32_t)min((int32_t)col, lim) * a.tok_e + 4 * g) * sizeof(float);
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int c = 0; c < CL; ++c)
    kt.k[c] = kPad && 16 * c + 4 * g >= a.hd ? z
              : kStream ? load_stream((const float4*)(kp + 64u * c))
                        : *(const float4*)(kp + 64u * c);
  const char* vp = tile_base(tab, vb, a, ts);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const char* row =
        vp + ((uint32_t)min((int32_t)(4 * g + i), lim) * a.tok_e + 4 * col) * sizeof(float);
#pragma unroll
    for (int h = 0; h < D / 64; ++h)
      vt.v[i][h] = kPad && 64 * h + 4 * col >= a.hd ? z
                   : kStream ? load_stream((const float4*)(row + 256u * h))
                             : *(const float4*)(row + 256u * h);
  }
}

__device__ __forceinline__ float f4(const float4& x, int j) {
  return j == 0 ? x.x : j == 1 ? x.y : j == 2 ? x.z : x.w;
}

// Online softmax over one 16-key tile for 16 query columns: S^T, lazy
// rescale, P = exp2(s c - m) in f32, O^T += V^T P^T. visible(i): key 4g + i
// of the tile. CL: the 16-column chunks of d in the scores (fewer than
// D / 16 when the rest are padding).
template <int D, int CL = D / 16, typename Mask>
__device__ __forceinline__ void attend_half_f32(const KHalfF32<D>& kt, const VHalfF32<D>& vt,
                                                const float4 (&qf)[D / 16],
                                                floatx4 (&o)[D / 16], float& m_run,
                                                float& l_run, float scale_log2, Mask visible) {
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CL; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma16x16x4f32(f4(kt.k[c], j), f4(qf[c], j), acc);
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = visible(i) ? acc[i] : -INFINITY;
  const float mx = max_nc(max_nc(s[0], s[1]), max_nc(s[2], s[3])) * scale_log2;
  rescale_rows<D>(mx, o, m_run, l_run);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(__builtin_fmaf(s[i], scale_log2, -m_run));
  l_run += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int h = 0; h < D / 64; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[4 * h + j] = mfma16x16x4f32(f4(vt.v[i][h], j), p[i], o[4 * h + j]);
}

// Row `col`'s outputs of o (the f32 layout above), scaled, as float4 runs
// d = 64h + 16g + 4i .. +3, to `row` (f32 output or partial).
template <int D, bool kPad = false>
__device__ __forceinline__ void store_row_f32(float* row, const floatx4 (&o)[D / 16],
                                              float scale, uint32_t g, uint32_t hd = D) {
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (!kPad || 64 * h + 16 * g + 4 * i < hd)
        *(float4*)(row + 64 * h + 16 * g + 4 * i) =
          make_float4(o[4 * h][i] * scale, o[4 * h + 1][i] * scale, o[4 * h + 2][i] * scale,
                      o[4 * h + 3][i] * scale);
}

// Bytes of one (item, split) partial block of a prefill key split: (m, l)
// f32 per row, then o / l per row in f32 (the split adds no rounding before
// the merge).
__host__ __device__ constexpr uint64_t pf_part_bytes(uint32_t rows, uint32_t d) {
  return (uint64_t)rows * (8 + 4 * d);
}

// ---- launchers (one per translation unit) ----------------------------------


// Decode rows (len_q == 1) of the batch; bf16/f16 with head_dim 64, 128 or
// 256, f32 with head_dim 64 or 128 (f32: no fused append).
size_t decode_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group,
                              uint32_t head_dim, uint32_t num_waves);
void launch_decode(AttnArgs a, void* workspace, uint32_t head_dim, uint32_t dtype,
                   hipStream_t s);
// Prefill rows (len_q > 1); bf16/f16, head_dim 64, 128 or 256.
// Workgroups of the prefill launch (query tiles x kv heads x sequences); a
// launch needs it below 2^32.
uint64_t prefill_grid(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t max_q,
                      uint32_t head_dim);
// The prefill launch over a.pf_seqs_n sequences (those a.pf_seqs names, or
// all a.batch); with a workspace (`split_ws`, `split_ws_bytes`) a batch too
// small to fill the GPU splits its keys over more workgroups.
void launch_prefill(const AttnArgs& a, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                    bool bf16, void* split_ws, size_t split_ws_bytes, hipStream_t s);
// A step with decode rows and prefill rows (at most kMaxPlanSeqs sequences,
// no fused append) in one launch of both kernels' workgroups side by side,
// then the decode's merge and, when the prefill split its keys, the
// prefill's merge. `workspace` is the decode's; split_ws the prefill's part.
void launch_mixed(const AttnArgs& a, void* workspace, uint32_t max_q, uint32_t max_k,
                  uint32_t head_dim, bool bf16, void* split_ws, size_t split_ws_bytes,
                  hipStream_t s);
// Prefill workgroups (before any key split) of a mixed launch.
uint64_t mixed_prefill_items(uint32_t n_seqs, uint32_t kvh, uint32_t group, uint32_t max_q);
// Sequences one decode launch plans for (larger batches are cut into launches).
uint32_t decode_max_plan_seqs();
// Workspace the prefill's key split wants for this shape (0: no split).
size_t prefill_split_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                           uint32_t max_q, uint32_t max_k);
// Prefill rows of an f32 pool (head_dim 64 or 128) on f32 MFMAs, over
// a.pf_seqs_n sequences; waves of the launch (a launch needs it below 2^32).
uint64_t prefill_f32_items(uint32_t n_seqs, uint32_t kvh, uint32_t group, uint32_t max_q);
// With a workspace (`split_ws`), a batch of fewer waves than the GPU holds
// splits its keys; the merge runs as a second launch.
void launch_prefill_f32(const AttnArgs& a, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                        void* split_ws, size_t split_ws_bytes, hipStream_t s);
// Workspace the f32 prefill's key split wants for this shape (0: no split).
size_t prefill_f32_split_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                               uint32_t max_q, uint32_t max_k);
void launch_prefill_merge_f32(const AttnArgs& a, uint32_t qtiles, uint32_t rows_per_item,
                              uint32_t n_split, const float* part, uint64_t base,
                              uint32_t head_dim, hipStream_t s);
// Any row, any dtype, head_dim <= 256 (VALU); split contexts combine their
// partials through `workspace` (generic_workspace_bytes).
void launch_generic(const AttnArgs& a, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                    uint32_t dtype, void* workspace, hipStream_t s);
// Workgroups of the VALU kernel's launch (row tiles x kv heads x sequences
// x key chunks); a launch needs it below 2^32.
uint64_t generic_grid(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t max_q,
                      uint32_t max_k);
size_t generic_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                               uint32_t max_q, uint32_t max_k);
// Persistent decode waves for the current device (CUs x 8).
uint32_t decode_num_waves();
// Bytes at the start of a decode workspace that carry over between calls
// (the balance block: XCD shares and per-wave timings); zero = equal shares.
extern const size_t kDecodeBalanceBytes;

}  // namespace vk
