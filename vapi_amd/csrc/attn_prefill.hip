// Chunked-prefill paged attention on MFMA (bf16/f16, head_dim 64 or 128).
//
// Rows are the (query token, head) pairs of one kv head, r = j*G + h_local,
// so the G query heads of a group share every K/V byte. A workgroup owns 256
// rows (8 waves x 2 tiles of 16; one workgroup per CU, two waves per SIMD,
// measured 5% faster than two workgroups of 4 waves) and walks the keys they
// can see in 32-key steps. Each step's K and V are loaded once per workgroup into LDS (double
// buffered in LDS, with the global loads issued two steps ahead into
// registers) and every K/V fragment read from LDS feeds both row tiles of a
// wave. V is written to LDS transposed, with the keys of a step permuted so
// that the 8 keys one lane group feeds to an MFMA are contiguous (each V^T
// fragment is a single ds_read_b128), and with its rows and the staging
// threads arranged so that neither the writes nor the reads collide on LDS
// banks (measured with SQ_LDS_BANK_CONFLICT: 20% -> 28% MFMA utilisation). The math per row
// tile is attend_qk / attend_pv (S^T = K Q^T, online softmax, O^T += V^T P^T)
// with the bottom-right causal mask and left window per row; row tiles
// whose rows cannot see any key of a step skip it. Rows with len_q < 2 are
// left to the decode kernel.
#include <type_traits>

#include "attn_common.hpp"

namespace vk {

#ifndef VK_PF_WAVES
#define VK_PF_WAVES 8
#endif
constexpr int kPfWaves = VK_PF_WAVES;
constexpr int kPfThreads = 64 * kPfWaves;
// 16-byte K chunks of one 32-key step per thread.
template <int D>
constexpr int kKIter = (32 * D / 8 + kPfThreads - 1) / kPfThreads;
constexpr int kKPad = 8;  // elements of padding per K row in LDS
constexpr int kVPad = 8;  // elements of padding per V^T row in LDS

// Column of key k (0..31 within a step) in a V^T row: keys 4g..4g+3 of both
// 16-key tiles (one lane group's MFMA k-slots) land in 8 contiguous columns.
__device__ __forceinline__ uint32_t vt_col(uint32_t k) {
  const uint32_t tt = k >> 4, r = k & 15;
  return 8 * (r >> 2) + 4 * tt + (r & 3);
}

// V staging: thread -> (key pair kp, 16-byte d chunk c). Key pairs run
// fastest across the lanes, so the 16 lanes of a group write 16 different
// columns of one V^T row (d chunks fastest put them on rows 8 apart, which
// share LDS banks).
__device__ __forceinline__ uint32_t vkp(uint32_t tid, uint32_t cpk) {
  return (tid % 16) + 16 * (tid / (16 * cpk));
}
__device__ __forceinline__ uint32_t vchunk(uint32_t tid, uint32_t cpk) { return (tid / 16) % cpk; }

// LDS row of V^T row d: the rows the 16 lanes of a lane group read together
// (d = DPL*col + k, col = 0..15) are stored consecutively, which the 80-byte
// row pitch spreads over the banks (rows DPL apart would share two).
template <int D>
__device__ __forceinline__ uint32_t vrow(uint32_t d) {
  constexpr uint32_t DPL = D / 16;
  return (d % DPL) * 16 + d / DPL;
}

template <int D>
struct alignas(16) PfSmem {
  uint16_t k[2][32][D + kKPad];
  uint16_t vt[2][D][32 + kVPad];
};

// One step's global loads, held in registers between issue and LDS store.
// Plain members rather than arrays: a register copy between stages must not
// turn the stage into a stack object.
template <int D>
struct PfStage {
  uint4 k0, k1;  // K chunks (16 B) tid and tid + 256 of the step's 32 x D tile (k1: D = 128)
  uint4 v0, v1;  // V of keys 2kp and 2kp+1 at d = 8c .. 8c+7 (tid < 2*D)
};

template <typename T, int D>
__device__ __forceinline__ void pf_load(PfStage<D>& st, const uint32_t* __restrict__ tab,
                                        const T* kb, const T* vb, const AttnArgs& a, int32_t s0,
                                        int32_t last, uint32_t tid) {
  constexpr uint32_t CPK = D / 8;  // 16-byte chunks per key row
  // The step's two 16-key tiles (a tile past the last key re-reads the
  // tile holding it): both block-table entries are read once, back to back,
  // for K and V alike, through the scalar cache (the table is never written
  // by a kernel).
  using ConstU32 = const __attribute__((address_space(4))) uint32_t;
  const int32_t ts0 = min(s0, last & ~15), ts1 = min(s0 + 16, last & ~15);
  const uint32_t c0 = min((uint32_t)ts0 >> a.bs_shift, a.max_blocks - 1);
  const uint32_t c1 = min((uint32_t)ts1 >> a.bs_shift, a.max_blocks - 1);
  const uint32_t blk0 = min(((ConstU32*)tab)[c0], a.last_blk);
  const uint32_t blk1 = min(((ConstU32*)tab)[c1], a.last_blk);
  const uint64_t off0 = (uint64_t)blk0 * a.blk_e + (uint64_t)((uint32_t)ts0 & (a.block_size - 1)) * a.tok_e;
  const uint64_t off1 = (uint64_t)blk1 * a.blk_e + (uint64_t)((uint32_t)ts1 & (a.block_size - 1)) * a.tok_e;
#pragma unroll
  for (int j = 0; j < kKIter<D>; ++j) {
    const uint32_t ci = min(tid + kPfThreads * j, 32 * CPK - 1);
    const uint32_t key = ci / CPK, part = ci % CPK;
    // Uniform per wave: the 64 lanes cover 64 / CPK keys of one tile.
    const bool second = __builtin_amdgcn_readfirstlane(key >> 4) != 0;
    const T* base = kb + (second ? off1 : off0);
    const int32_t lim = last - (second ? ts1 : ts0);
    const uint32_t kk = (uint32_t)min((int32_t)(key & 15), lim);
    const uint4 x = *(const uint4*)(base + kk * a.tok_e + 8 * part);
    if (j == 0) st.k0 = x; else st.k1 = x;
  }
  if (tid < 2 * D) {
    const uint32_t kp = vkp(tid, CPK), c = vchunk(tid, CPK);
    // Key pairs 0..7 sit in the first tile, 8..15 in the second: selected
    // per lane.
    const bool second = kp >= 8;
    const T* base = vb + (second ? off1 : off0);
    const int32_t lim = last - (second ? ts1 : ts0);
    const uint32_t k0 = (uint32_t)min((int32_t)((2 * kp) & 15), lim);
    const uint32_t k1 = (uint32_t)min((int32_t)((2 * kp + 1) & 15), lim);
    st.v0 = *(const uint4*)(base + k0 * a.tok_e + 8 * c);
    st.v1 = *(const uint4*)(base + k1 * a.tok_e + 8 * c);
  }
}

template <int D>
__device__ __forceinline__ void pf_store(PfSmem<D>& sm, int buf, const PfStage<D>& st,
                                         uint32_t tid) {
  constexpr uint32_t CPK = D / 8;
#pragma unroll
  for (int j = 0; j < kKIter<D>; ++j) {
    const uint32_t ci = tid + kPfThreads * j;
    if (ci < 32 * CPK) *(uint4*)&sm.k[buf][ci / CPK][8 * (ci % CPK)] = j == 0 ? st.k0 : st.k1;
  }
  if (tid < 2 * D) {
    const uint32_t kp = vkp(tid, CPK), c = vchunk(tid, CPK);
    const uint32_t col = vt_col(2 * kp);  // even; key 2kp+1 sits next to it
    const uint32_t x[4] = {st.v0.x, st.v0.y, st.v0.z, st.v0.w};
    const uint32_t y[4] = {st.v1.x, st.v1.y, st.v1.z, st.v1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t w =
          __builtin_amdgcn_perm(y[e >> 1], x[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
      *(uint32_t*)&sm.vt[buf][vrow<D>(8 * c + e)][col] = w;
    }
  }
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

template <typename T, int D, int RT, int OCC>
__global__ __launch_bounds__(kPfThreads, OCC) void paged_prefill_tiled(
    AttnArgs a, const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ cu_k,
    const uint32_t* __restrict__ table, uint32_t qtiles) {
  constexpr int KC = D / 32;
  constexpr int DPL = D / 16;
  constexpr int kPfRT = RT;
  constexpr uint32_t kPfRows = 16 * RT * kPfWaves;
  __shared__ PfSmem<D> sm;
  const uint32_t n_items = gridDim.x;
  const uint32_t item = xcd_remap(blockIdx.x, n_items);
  const uint32_t qt = item % qtiles, rest = item / qtiles;
  const uint32_t kh = rest % a.kvh, seq = rest / a.kvh;
  const uint32_t q0 = cu_q[seq];
  const uint32_t len_q = cu_q[seq + 1] - q0;
  if (len_q < 2) return;
  const uint32_t G = a.group;
  const uint32_t nrows = len_q * G;
  const uint32_t row_base = qt * kPfRows;
  if (row_base >= nrows) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t col = lane & 15, g = lane >> 4;
  const int32_t len_k = (int32_t)(cu_k[seq + 1] - cu_k[seq]);
  const int32_t offset = len_k - (int32_t)len_q;
  const int32_t last = len_k - 1;

  // Keys the whole workgroup can see.
  const uint32_t wg_last = min(row_base + kPfRows, nrows) - 1;
  const int32_t wg_pmin = offset + (int32_t)(row_base / G);
  const int32_t wg_pmax = offset + (int32_t)(wg_last / G);
  const int32_t klo = a.wl >= 0 ? max(0, wg_pmin - a.wl) : 0;
  const int32_t khi = a.wr >= 0 ? min(last, wg_pmax + a.wr) : last;

  // This wave's rows: Q^T operands, per-lane query position, per-tile range.
  const uint32_t row0 = row_base + wave * 16 * kPfRT;
  uint4 qf[kPfRT][KC];
  // Per lane: visible keys lo..hi of its row, as key - lo < cnt (unsigned).
  int32_t lo[kPfRT], cnt[kPfRT];
#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    const uint32_t r = row0 + 16 * t + col;
    const uint32_t rr = r < nrows ? r : 0;  // padding rows copy row 0, never stored
    const uint32_t j = rr / G, hl = rr % G;
    int32_t hi;
    key_range(offset + (int32_t)j, len_k, a.wl, a.wr, lo[t], hi);
    cnt[t] = max(hi - lo[t] + 1, 0);
    const T* qrow = (const T*)a.q + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      uint4 x = *(const uint4*)(qrow + 32 * c + 8 * g);
      x.x ^= a.q_sign, x.y ^= a.q_sign, x.z ^= a.q_sign, x.w ^= a.q_sign;
      qf[t][c] = x;
    }
  }

  const uint32_t* __restrict__ tab = table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;

  float m_run[kPfRT], l_run[kPfRT];
  floatx4 o[kPfRT][DPL];
#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    m_run[t] = kNegBig;
    l_run[t] = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) o[t][k] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Keys every row of the workgroup sees (ranges move right with the row):
  // steps inside [full_lo, full_hi] need no mask.
  int32_t full_lo, full_hi, unused;
  key_range(wg_pmax, len_k, a.wl, a.wr, full_lo, unused);
  key_range(wg_pmin, len_k, a.wl, a.wr, unused, full_hi);

  // Two register stages: the global loads of step s+2 are issued before
  // step s is computed from LDS, and those of step s+1 (issued a whole step
  // earlier) are stored to the other LDS buffer after it, so a step's global
  // latency hides behind two steps of compute. Loads are unconditional
  // (steps past the last re-read it).
  PfStage<D> stA, stB;
  int32_t s0_ = klo & ~31;
  const int32_t s_last = khi & ~31;
  pf_load<T, D>(stA, tab, kb, vb, a, s0_, last, tid);
  pf_store<D>(sm, 0, stA, tid);
  pf_load<T, D>(stA, tab, kb, vb, a, min(s0_ + 32, s_last), last, tid);
  __syncthreads();
  int buf = 0;
  // `ready` holds step s+1 (in flight since the previous step), `next`
  // receives step s+2.
  auto step = [&](auto masked, PfStage<D>& ready, PfStage<D>& next) __attribute__((always_inline)) {
    // s0 is uniform; saying so keeps the table reads on the scalar unit.
    const int32_t s0 = __builtin_amdgcn_readfirstlane(s0_);
    pf_load<T, D>(next, tab, kb, vb, a, min(s0 + 64, s_last), last, tid);
    KTile<D> kt;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int c = 0; c < KC; ++c)
        kt.k[tt][c] = *(const uint4*)&sm.k[buf][16 * tt + col][32 * c + 8 * g];
    // Every row tile runs every step: a tile whose rows see no key of the
    // step gets P = 0 (all scores -inf). The scores of all row tiles are
    // issued first (independent MFMA chains), then their maxima share one
    // rescale branch, so no branch sits between a tile's MFMAs and the
    // next tile's.
    float sc[kPfRT][8];
    {
      floatx4 acc[kPfRT][2];
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) qk_scores<T, D>(kt, qf[t], acc[t]);
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) {
        const uint32_t base = (uint32_t)(s0 + 4 * (int32_t)g - lo[t]), n = (uint32_t)cnt[t];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool vis = !decltype(masked)::value || base + 16 * tt + i < n;
            sc[t][4 * tt + i] = vis ? acc[t][tt][i] : -INFINITY;
          }
      }
    }
    float mx[kPfRT];
    bool grow = false;
#pragma unroll
    for (int t = 0; t < kPfRT; ++t) {
      mx[t] = max3_nc(max3_nc(sc[t][0], sc[t][1], sc[t][2]), max3_nc(sc[t][3], sc[t][4], sc[t][5]),
                      max_nc(sc[t][6], sc[t][7])) * a.scale_log2;
      grow |= mx[t] > m_run[t] + kRescaleSlack;
    }
    if (__any(grow)) {
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) rescale_rows<D>(mx[t], o[t], m_run[t], l_run[t]);
    }
    uint4 pf[kPfRT];
#pragma unroll
    for (int t = 0; t < kPfRT; ++t) pf[t] = exp_pack<T>(sc[t], m_run[t], l_run[t], a.scale_log2);
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const uint4 vf = *(const uint4*)&sm.vt[buf][vrow<D>(DPL * col + k)][8 * g];
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) o[t][k] = mfma16x16x32<T>(vf, pf[t], o[t][k]);
    }
    pf_store<D>(sm, buf ^ 1, ready, tid);
    __syncthreads();
    buf ^= 1;
    s0_ += 32;
  };
  using Masked = std::integral_constant<bool, true>;
  using Full = std::integral_constant<bool, false>;
  // Steps alternate the stage roles (unrolled by two); a loop that ends on
  // an odd step moves the in-flight stage back to stA, the invariant between
  // loops.
  auto loop = [&](auto masked, auto more) __attribute__((always_inline)) {
    while (more()) {
      step(masked, stA, stB);
      if (!more()) {
        stA = stB;
        return;
      }
      step(masked, stB, stA);
    }
  };
  loop(Masked{}, [&] { return s0_ <= khi && s0_ < full_lo; });
  loop(Full{}, [&] { return s0_ <= khi && s0_ + 31 <= full_hi; });
  loop(Masked{}, [&] { return s0_ <= khi; });

#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    const float lt = wave_sum_g(l_run[t]);
    const uint32_t r = row0 + 16 * t + col;  // this lane's query row
    if (r >= nrows) continue;
    const uint32_t j = r / G, hl = r % G;
    T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
    store_row<T, D>(orow, o[t], lt > 0.f ? 1.f / lt : 0.f, g);
  }
}

#ifndef VK_PF_RT
#define VK_PF_RT 2
#endif
#ifndef VK_PF_OCC
#define VK_PF_OCC 1
#endif

void launch_prefill(const AttnArgs& a, uint32_t max_q, uint32_t head_dim, bool bf16,
                    hipStream_t s) {
  constexpr uint32_t rows = 16 * VK_PF_RT * kPfWaves;
  const uint32_t qtiles = (max_q * a.group + rows - 1) / rows;
  const uint64_t n = (uint64_t)qtiles * a.kvh * a.batch;
  const dim3 grid((uint32_t)n), block(kPfThreads);
#define VK_PF(T, DD)                                                                    \
  hipLaunchKernelGGL((paged_prefill_tiled<T, DD, VK_PF_RT, VK_PF_OCC>), grid, block, 0, s, a, \
                     a.cu_q, a.cu_k, a.table, qtiles)
  if (bf16) {
    if (head_dim == 128) VK_PF(bf16_t, 128);
    else VK_PF(bf16_t, 64);
  } else {
    if (head_dim == 128) VK_PF(f16_t, 128);
    else VK_PF(f16_t, 64);
  }
#undef VK_PF
}

}  // namespace vk
