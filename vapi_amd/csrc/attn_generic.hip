// Generic VALU paged attention: any dtype (f32 included), any head_dim up
// to 256 and any GQA ratio. One wave per (query token, query head); K rows
// are dotted one key per lane, V rows are accumulated one d per lane.
#include "attn_common.hpp"

namespace vk {

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
      const uint32_t blk = min(table[min((uint32_t)key / a.block_size, a.max_blocks - 1)], a.last_blk);
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
      const uint32_t blk = min(table[min((uint32_t)key2 / a.block_size, a.max_blocks - 1)], a.last_blk);
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

void launch_generic(const AttnArgs& a, uint32_t max_q, uint32_t head_dim, uint32_t dtype,
                    hipStream_t s) {
  const dim3 grid(max_q, a.num_heads, a.batch);
#define VK_GEN(T)                                                                         \
  do {                                                                                    \
    if (head_dim <= 64)                                                                   \
      hipLaunchKernelGGL((paged_attn_generic<T, 1>), grid, dim3(64), 0, s, a, head_dim); \
    else if (head_dim <= 128)                                                             \
      hipLaunchKernelGGL((paged_attn_generic<T, 2>), grid, dim3(64), 0, s, a, head_dim); \
    else                                                                                  \
      hipLaunchKernelGGL((paged_attn_generic<T, 4>), grid, dim3(64), 0, s, a, head_dim); \
  } while (0)
  switch (dtype) {
    case VAPI_KV_F32: VK_GEN(float); break;
    case VAPI_KV_BF16: VK_GEN(bf16_t); break;
    default: VK_GEN(f16_t); break;
  }
#undef VK_GEN
}

}  // namespace vk
