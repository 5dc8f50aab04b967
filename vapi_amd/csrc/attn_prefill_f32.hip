// Chunked-prefill paged attention for f32 pools on v_mfma_f32_16x16x4_f32.
//
// Rows are the (query token, head) pairs of one kv head, r = j*G + h_local,
// as in the 16-bit prefill. Each wave owns RT tiles of 16 rows of one
// (sequence, kv head) and walks the keys they can see in 32-key steps, each
// step as two 16-key halves in the f32 operand scheme of the decode
// (attend_half_f32: S^T = K Q^T at K = 4 per MFMA, lazy-rescaled online
// softmax with P kept in f32, O^T += V^T P^T). A half is computed for every
// row tile of the wave, then reloaded with the next step's half while the
// other half is computed, so 16 KiB of K/V stay in flight per wave.
//
// K and V come straight from memory into registers, with ordinary (cached)
// loads: the waves of one (sequence, kv head) read the same K/V, and the
// workgroup -> work-item map gives each XCD a contiguous range of items, so
// those waves run together under one L2. Four waves per workgroup, one per
// SIMD: f32 MFMAs are long (a 16x16x4 takes 32 cycles), so a wave's softmax
// is small beside its MFMAs and a second wave per SIMD buys little.
//
// Rows with len_q < a.pf_min_q are left to the decode stream (pf_min_q 1:
// every row here). kPad: a head_dim a.hd below D (a multiple of 4); Q, K
// and V elements past it load as zeros, output rows are a.hd apart and
// their columns past it are not stored. Numerical contract: paged_attention_cpu (vapi
// crates/vapi-backend-candle/src/attention.rs:90-163), f32 throughout.
#include "attn_common.hpp"

namespace vk {

constexpr int kPf32Waves = 4;

// kSplit: the keys a wave would walk are cut into n_split contiguous runs
// of steps, one wave each (a batch too small to fill the GPU with query
// tiles alone); each writes its rows' (m, l, o / l) to `part`
// (pf_part_bytes of 16 * RT rows per (item, split)) for the merge.
// CL: the 16-column chunks of d that hold head_dim (kPad; D / 16
// otherwise): K chunks past them are neither loaded nor multiplied.
template <int D, int RT, bool kSplit, bool kPad, int CL = D / 16>
__global__ __launch_bounds__(64 * kPf32Waves, 1) void paged_prefill_f32(
    AttnArgs a, uint32_t qtiles, uint32_t n_items, uint32_t n_split_arg,
    float* __restrict__ part) {
  const uint32_t n_split = kSplit ? n_split_arg : 1u;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t item = xcd_remap(blockIdx.x, gridDim.x) * kPf32Waves + wave;
  if (item >= n_items) return;
  // Item order: query tile fastest, then key split, kv head, sequence.
  const uint32_t qt = item % qtiles, rest_s = item / qtiles;
  const uint32_t split = rest_s % n_split, rest = rest_s / n_split;
  const uint32_t kh = rest % a.kvh;
  const uint32_t seq = a.pf_seqs ? a.pf_seqs[rest / a.kvh] : rest / a.kvh;
  if (seq >= a.batch) return;
  const uint32_t q0 = a.cu_q[seq];
  const uint32_t len_q = a.cu_q[seq + 1] - q0;
  if (len_q < a.pf_min_q || len_q == 0) return;
  const uint32_t G = a.group;
  const uint32_t nrows = len_q * G;
  const uint32_t row0 = qt * 16 * RT;
  if (row0 >= nrows) return;
  const uint32_t col = lane & 15, g = lane >> 4;
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const int32_t offset = len_k - (int32_t)len_q;

  // This wave's rows: Q^T operands and visible key ranges.
  float4 qf[RT][D / 16];
  int32_t lo[RT];
  uint32_t cnt[RT];
  const uint32_t sg = a.q_sign ? 0x80000000u : 0u;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint32_t r = row0 + 16 * t + col;
    const uint32_t rr = r < nrows ? r : 0;
    const uint32_t j = rr / G, hl = rr % G;
    int32_t hi;
    key_range(offset + (int32_t)j, len_k, a.wl, a.wr, lo[t], hi);
    cnt[t] = (uint32_t)max(hi - lo[t] + 1, 0);
    const float* qrow =
        (const float*)a.q + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * (kPad ? a.hd : D);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      uint4 x = make_uint4(0, 0, 0, 0);
      if (!kPad || 16 * c + 4 * g < a.hd) x = *(const uint4*)(qrow + 16 * c + 4 * g);
      x.x ^= sg, x.y ^= sg, x.z ^= sg, x.w ^= sg;
      qf[t][c] = make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                             __uint_as_float(x.w));
    }
  }
  // The keys any row of the wave sees: from the first row's window start to
  // the last row's last key.
  const uint32_t r_last = min(row0 + 16 * RT, nrows) - 1;
  int32_t klo, khi, unused;
  key_range(offset + (int32_t)(row0 / G), len_k, a.wl, a.wr, klo, unused);
  key_range(offset + (int32_t)(r_last / G), len_k, a.wl, a.wr, unused, khi);
  if (kSplit) {
    // This split's share of the wave's 32-key steps (empty: khi < klo).
    const int32_t first = klo & ~31;
    const uint32_t steps = khi >= klo ? (uint32_t)(((khi & ~31) - first) / 32 + 1) : 0u;
    const uint32_t a0 = split * steps / n_split, a1 = (split + 1) * steps / n_split;
    klo = max(klo, first + 32 * (int32_t)a0);
    khi = min(khi, first + 32 * (int32_t)a1 - 1);
  }

  float m_run[RT], l_run[RT];
  floatx4 o[RT][D / 16];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m_run[t] = kNegBig;
    l_run[t] = 0.f;
#pragma unroll
    for (int k = 0; k < D / 16; ++k) o[t][k] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  if (khi >= klo) {
    const uint32_t* __restrict__ tab = a.table + (uint64_t)seq * a.max_blocks;
    const float* kb = (const float*)a.k + kh * a.head_e;
    const float* vb = (const float*)a.v + kh * a.head_e;
    const int32_t s_last = khi & ~31;
    int32_t s0 = klo & ~31;
    KTileF32<D> kt;
    VTileF32<D> vt;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
      load_half_f32<D, false, kPad, CL>(kt.h[tt], vt.h[tt], tab, kb, vb, a, s0, tt, khi, col, g);
    while (true) {
      // The next step's halves are loaded unconditionally (the last step
      // re-reads its own keys, from L2): a load inside a branch would make
      // the compiler wait for it before this step's MFMAs.
      const int32_t s_next = min(s0 + 32, s_last);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const uint32_t base = (uint32_t)(s0 + 16 * tt + 4 * (int32_t)g - lo[t]);
          const uint32_t n = cnt[t];
          attend_half_f32<D, CL>(kt.h[tt], vt.h[tt], qf[t], o[t], m_run[t], l_run[t], a.scale_log2,
                             [&](int i) { return base + (uint32_t)i < n; });
        }
        load_half_f32<D, false, kPad, CL>(kt.h[tt], vt.h[tt], tab, kb, vb, a, s_next, tt, khi, col, g);
      }
      if (s0 >= s_last) break;
      s0 += 32;
    }
  }

  if constexpr (kSplit) {
    char* pb = (char*)part + ((uint64_t)(rest * qtiles + qt) * n_split + split) *
                                 pf_part_bytes(16 * RT, D);
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const float lt = wave_sum_g(l_run[t]);
      const uint32_t row = 16 * t + col;
      if (g == 0) *(float2*)(pb + (uint64_t)row * 8) = make_float2(m_run[t], lt);
      float* po = (float*)(pb + (uint64_t)16 * RT * 8) + (uint64_t)row * D;
      store_row_f32<D>(po, o[t], lt > 0.f ? 1.f / lt : 0.f, g);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float lt = wave_sum_g(l_run[t]);
    const uint32_t r = row0 + 16 * t + col;
    if (r >= nrows) continue;
    const uint32_t j = r / G, hl = r % G;
    float* orow =
        (float*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * (kPad ? a.hd : D);
    store_row_f32<D, kPad>(orow, o[t], lt > 0.f ? 1.f / lt : 0.f, g, a.hd);
  }
}

constexpr int kPf32RowTiles = 2;
constexpr uint32_t kPf32Rows = 16 * kPf32RowTiles;

uint64_t prefill_f32_items(uint32_t n_seqs, uint32_t kvh, uint32_t group, uint32_t max_q) {
  return ((uint64_t)max_q * group + kPf32Rows - 1) / kPf32Rows * kvh * n_seqs;
}

// Key splits for `base` waves over at most max_k keys: enough for about one
// wave per SIMD of a 256-CU GPU (one wave each is the kernel's occupancy),
// each split keeping at least 8 steps of 32 keys, at most 64; fewer when
// the workspace given holds fewer partials (at most 256 MiB of them).
static uint32_t pf32_splits(uint64_t base, uint32_t max_k, uint32_t head_dim, uint64_t bytes) {
  constexpr uint64_t kTarget = 1024;
  if (base == 0 || base >= kTarget) return 1;
  uint64_t n = std::min<uint64_t>((kTarget + base - 1) / base, std::max<uint32_t>(1u, max_k / 256));
  n = std::min<uint64_t>(n, 64);
  const uint64_t cap = std::min<uint64_t>(bytes, 256ull << 20);
  while (n > 1 && base * n * pf_part_bytes(kPf32Rows, head_dim) > cap) --n;
  return (uint32_t)n;
}

size_t prefill_f32_split_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                               uint32_t max_q, uint32_t max_k) {
  if (max_q <= 1) return 0;
  const uint64_t base = prefill_f32_items(batch, kvh, group, max_q);
  const uint32_t n = pf32_splits(base, max_k, head_dim, ~0ull);
  return n > 1 ? (size_t)(base * n * pf_part_bytes(kPf32Rows, head_dim)) : 0;
}

void launch_prefill_f32(const AttnArgs& a, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                        void* split_ws, size_t split_ws_bytes, hipStream_t s) {
  const uint32_t qtiles = (uint32_t)(((uint64_t)max_q * a.group + kPf32Rows - 1) / kPf32Rows);
  const uint64_t base = (uint64_t)qtiles * a.kvh * a.pf_seqs_n;
  // No split without a workspace, nor for a deterministic call (its output
  // must not depend on the workspace it is given).
  const uint32_t n_split =
      split_ws && !a.deterministic ? pf32_splits(base, max_k, head_dim, split_ws_bytes) : 1;
  const uint64_t items = base * n_split;
  const uint32_t wgs = (uint32_t)((items + kPf32Waves - 1) / kPf32Waves);
  float* part = n_split > 1 ? (float*)split_ws : nullptr;
#define VK_PF32(DD, PAD, CL)                                                                    \
  do {                                                                                          \
    if (n_split > 1) {                                                                          \
      hipLaunchKernelGGL((paged_prefill_f32<DD, kPf32RowTiles, true, PAD, CL>), dim3(wgs),      \
                         dim3(64 * kPf32Waves), 0, s, a, qtiles, (uint32_t)items, n_split, part); \
      launch_prefill_merge_f32(a, qtiles, kPf32Rows, n_split, part, base, DD, s);               \
    } else {                                                                                    \
      hipLaunchKernelGGL((paged_prefill_f32<DD, kPf32RowTiles, false, PAD, CL>), dim3(wgs),     \
                         dim3(64 * kPf32Waves), 0, s, a, qtiles, (uint32_t)items, 1u, nullptr); \
    }                                                                                           \
  } while (0)
  // A head_dim below the kernel's D runs the padded variant, which skips the
  // K chunks wholly past it where the launch has a variant that stops there
  // (64: 32 columns; 128: 80 or 96).
  const uint32_t live = (a.hd + 15) / 16;
  if (head_dim == 128) {
    if (a.hd == 128) VK_PF32(128, false, 8);
    else if (live <= 5) VK_PF32(128, true, 5);
    else if (live <= 6) VK_PF32(128, true, 6);
    else VK_PF32(128, true, 8);
  } else {
    if (a.hd == 64) VK_PF32(64, false, 4);
    else if (live <= 2) VK_PF32(64, true, 2);
    else VK_PF32(64, true, 4);
  }
#undef VK_PF32
}

}  // namespace vk
