// Chunked-prefill paged attention on MFMA (bf16/f16, head_dim 64 or 128).
// Rows are the (query token, head) pairs of one kv head, r = j*G + h_local,
// so all G query heads of a group share every K/V load; each wave owns RT
// 16-row tiles and walks the visible keys in 32-key steps with an online
// softmax (attend_step). Rows with len_q < 2 are left to the decode kernel.
#include "attn_common.hpp"

namespace vk {

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
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

  const uint32_t* __restrict__ tab = a.table + (uint64_t)seq * a.max_blocks;
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

  KVStep<D> st;
  for (int32_t s0 = klo & ~31; s0 <= khi; s0 += 32) {
    load_kv_step<T, D>(st, tab, kb, vb, a, s0, len_k - 1, col, g);
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int32_t pt = pos[t];
      attend_step<T, D>(st, qf[t], o[t], m_run[t], l_run[t], a.scale_log2, g,
                        [&](int tt, int i) {
                          const int32_t key = s0 + 16 * tt + 4 * (int32_t)g + i;
                          return key < len_k && (a.wr < 0 || key <= pt + a.wr) &&
                                 (a.wl < 0 || key >= pt - a.wl);
                        });
    }
  }

#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float lt = wave_sum_g(l_run[t]);
    const uint32_t r = row0 + 16 * t + col;  // this lane's query row
    if (r >= nrows) continue;
    const uint32_t j = r / G, hl = r % G;
    T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
    store_row<T, D>(orow, o[t], lt > 0.f ? 1.f / lt : 0.f, g);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch

constexpr int kPrefillRT = 2;
constexpr int kPrefillWaves = 4;

void launch_prefill(const AttnArgs& a, uint32_t max_q, uint32_t head_dim, bool bf16,
                    hipStream_t s) {
  const uint32_t rows_per_wg = 16 * kPrefillRT * kPrefillWaves;
  const dim3 grid((max_q * a.group + rows_per_wg - 1) / rows_per_wg, a.kvh, a.batch);
  const dim3 block(64 * kPrefillWaves);
  if (bf16) {
    if (head_dim == 128)
      hipLaunchKernelGGL((paged_prefill_mfma<bf16_t, 128, kPrefillRT, kPrefillWaves>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((paged_prefill_mfma<bf16_t, 64, kPrefillRT, kPrefillWaves>), grid, block, 0, s, a);
  } else {
    if (head_dim == 128)
      hipLaunchKernelGGL((paged_prefill_mfma<f16_t, 128, kPrefillRT, kPrefillWaves>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((paged_prefill_mfma<f16_t, 64, kPrefillRT, kPrefillWaves>), grid, block, 0, s, a);
  }
}

}  // namespace vk
