// Decode (len_q == 1) paged attention as one persistent, evenly split stream.
//
// The work of a decode batch is the sequence of 32-key steps over every
// (sequence, kv head) segment: segment (s, h) has ceil((len_k - lo32)/32)
// steps, where lo32 is the window start rounded down to 32. The grid holds
// exactly as many waves as the chip runs at once (CUs x 8); wave w takes the
// contiguous slice [w*S/W, (w+1)*S/W) of the S steps, so every wave moves the
// same number of K/V bytes (+-1 step) and no workgroup ramps up or drains
// while others still run. A wave keeps the next step's K/V in flight while it
// computes the current one, including across segment boundaries.
//
// A slice that covers a whole segment writes the normalised output directly.
// Otherwise the wave writes its piece's (m, l, o) to slot w + segment (slots
// are unique because slices and segments are both increasing), and
// paged_decode_merge combines the pieces of each split segment. All G query
// heads of a kv head ride one MFMA tile, so K/V bytes are read exactly once.
#include "attn_common.hpp"

namespace vk {

constexpr int kDecodeWavesPerWG = 4;
constexpr uint32_t kMaxPlanSeqs = 4096;  // sequences per launch (host chunks beyond)

// Steps of sequence s (0 for rows that are not decode rows) and its first key.
__device__ __forceinline__ uint32_t decode_steps(const AttnArgs& a, uint32_t s, int32_t& lo) {
  lo = 0;
  if (a.cu_q[s + 1] - a.cu_q[s] != 1) return 0;
  const int32_t len_k = (int32_t)(a.cu_k[s + 1] - a.cu_k[s]);
  if (len_k <= 0) return 0;
  lo = a.wl >= 0 ? max(0, len_k - 1 - a.wl) : 0;
  return (uint32_t)(len_k - (lo & ~31) + 31) >> 5;
}

// Where global step t lives.
struct DecodePos {
  uint32_t seq, kh, q0;
  int32_t key0, len_k, lo;
  bool seg_first;  // key0 is the segment's first step
};

__device__ __forceinline__ DecodePos locate(const AttnArgs& a, const uint32_t* P, uint32_t t) {
  uint32_t lo_i = 0, hi_i = a.batch;  // P[lo_i] <= t < P[hi_i]
  while (hi_i - lo_i > 1) {
    const uint32_t mid = (lo_i + hi_i) >> 1;
    if (__builtin_amdgcn_readfirstlane(P[mid]) <= t) lo_i = mid;
    else hi_i = mid;
  }
  DecodePos p;
  p.seq = lo_i;
  const uint32_t p0 = __builtin_amdgcn_readfirstlane(P[lo_i]);
  const uint32_t nst = (__builtin_amdgcn_readfirstlane(P[lo_i + 1]) - p0) / a.kvh;
  const uint32_t local = t - p0;
  p.kh = local / nst;
  const uint32_t ks = local - p.kh * nst;
  p.q0 = a.cu_q[p.seq];
  p.len_k = (int32_t)(a.cu_k[p.seq + 1] - a.cu_k[p.seq]);
  p.lo = a.wl >= 0 ? max(0, p.len_k - 1 - a.wl) : 0;
  p.key0 = (p.lo & ~31) + 32 * (int32_t)ks;
  p.seg_first = ks == 0;
  return p;
}

template <typename T, int D>
__device__ __forceinline__ void load_q(uint4 (&qf)[D / 32], const AttnArgs& a, const DecodePos& p,
                                       uint32_t col, uint32_t g) {
  const bool real = col < a.group;
  const T* qrow = (const T*)a.q +
                  ((uint64_t)p.q0 * a.num_heads + p.kh * a.group + (real ? col : 0)) * D;
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
    qf[c] = real ? *(const uint4*)(qrow + 32 * c + 8 * g) : make_uint4(0, 0, 0, 0);
}

template <typename T, int D>
__device__ __forceinline__ void load_step(KVStep<D>& st, const AttnArgs& a, const DecodePos& p,
                                          uint32_t col, uint32_t g) {
  const uint32_t* __restrict__ tab = a.table + (uint64_t)p.seq * a.max_blocks;
  const T* kb = (const T*)a.k + p.kh * a.head_e;
  const T* vb = (const T*)a.v + p.kh * a.head_e;
  load_kv_step<T, D>(st, tab, kb, vb, a, p.key0, p.len_k, p.len_k - 1, col, g);
}

// Write this wave's piece of segment (p.seq, p.kh): the final output if the
// piece is the whole segment, else a partial in slot `slot`.
template <typename T, int D>
__device__ __forceinline__ void flush_piece(const AttnArgs& a, const DecodePos& p, bool whole,
                                            uint32_t slot, const floatx4 (&o)[D / 16],
                                            float m_run, float l_run, uint32_t col, uint32_t g) {
  constexpr int DPL = D / 16;
  const uint32_t G = a.group;
  const float l_tot = wave_sum_g(l_run);
  if (whole) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = __shfl(l_tot, 4 * g + i);
      const uint32_t hh = 4 * g + i;
      if (hh >= G) continue;
      const float inv = li > 0.f ? 1.f / li : 0.f;
      T* orow = (T*)a.out + ((uint64_t)p.q0 * a.num_heads + p.kh * G + hh) * D + DPL * col;
      uint32_t w[DPL / 2];
#pragma unroll
      for (int k = 0; k < DPL / 2; ++k)
        w[k] = pack2<T>(o[2 * k][i] * inv, o[2 * k + 1][i] * inv);
      if constexpr (DPL == 4) {
        *(uint2*)orow = make_uint2(w[0], w[1]);
      } else {
#pragma unroll
        for (int k = 0; k < DPL / 8; ++k)
          ((uint4*)orow)[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hh = 4 * g + i;
      if (hh >= G) continue;
      float* po = a.ws_o + ((uint64_t)slot * G + hh) * D + DPL * col;
#pragma unroll
      for (int k = 0; k < DPL; k += 4)
        *(float4*)(po + k) = make_float4(o[k][i], o[k + 1][i], o[k + 2][i], o[k + 3][i]);
    }
    if (g == 0 && col < G) {
      float* ml = a.ws_ml + ((uint64_t)slot * G + col) * 2;
      ml[0] = m_run;
      ml[1] = l_tot;
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kDecodeWavesPerWG, 2) void paged_decode_stream(AttnArgs a) {
  constexpr int DPL = D / 16;
  __shared__ uint32_t P[kMaxPlanSeqs + 1];
  __shared__ uint32_t wave_tot[kDecodeWavesPerWG];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t B = a.batch;

  // Step prefix sums over sequences (each sequence contributes kvh segments).
  {
    constexpr uint32_t NT = 64 * kDecodeWavesPerWG;
    const uint32_t per = (B + NT - 1) / NT;
    const uint32_t b0 = min(tid * per, B), b1 = min(b0 + per, B);
    uint32_t sum = 0;
    for (uint32_t s = b0; s < b1; ++s) {
      int32_t lo;
      sum += decode_steps(a, s, lo) * a.kvh;
    }
    uint32_t inc = sum;  // inclusive scan within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(inc, o);
      if (lane >= (uint32_t)o) inc += y;
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    uint32_t run = inc - sum;
    for (uint32_t w = 0; w < wave; ++w) run += wave_tot[w];
    for (uint32_t s = b0; s < b1; ++s) {
      P[s] = run;
      int32_t lo;
      run += decode_steps(a, s, lo) * a.kvh;
    }
    if (tid == NT - 1) P[B] = run;
    __syncthreads();
    if (blockIdx.x == 0)
      for (uint32_t s = tid; s <= B; s += NT) a.plan[s] = P[s];
  }

  const uint32_t S = __builtin_amdgcn_readfirstlane(P[B]);
  const uint32_t gw = blockIdx.x * kDecodeWavesPerWG + wave;
  const uint32_t W = a.num_waves;
  uint32_t t = (uint32_t)(((uint64_t)gw * S) / W);
  const uint32_t t_end = (uint32_t)(((uint64_t)(gw + 1) * S) / W);
  if (t >= t_end) return;

  const uint32_t col = lane & 15, g = lane >> 4;
  DecodePos pos = locate(a, P, t);
  uint4 qf[D / 32];
  load_q<T, D>(qf, a, pos, col, g);
  bool piece_first = pos.seg_first;
  float m_run = kNegBig, l_run = 0.f;
  floatx4 o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};

  KVStep<D> bufA, bufB;
  load_step<T, D>(bufA, a, pos, col, g);

  // One step: prefetch the next step into `nb`, attend over `cb`, flush and
  // switch segment when the next step starts a new one. Returns false at the
  // end of the slice.
  auto step = [&](KVStep<D>& cb, KVStep<D>& nb) -> bool {
    const bool more = t + 1 < t_end;
    const bool same_seg = pos.key0 + 32 < pos.len_k;
    DecodePos nxt = pos;
    if (more) {
      if (same_seg) {
        nxt.key0 += 32;
        nxt.seg_first = false;
      } else {
        nxt = locate(a, P, t + 1);
      }
      load_step<T, D>(nb, a, nxt, col, g);
    }
    const int32_t lo = pos.lo, len_k = pos.len_k, key0 = pos.key0;
    attend_step<T, D>(cb, qf, o, m_run, l_run, a.scale_log2, g, [&](int tt, int i) {
      const int32_t key = key0 + 16 * tt + 4 * (int32_t)g + i;
      return key >= lo && key < len_k;
    });
    if (!more || !same_seg) {
      const uint32_t seg = pos.seq * a.kvh + pos.kh;
      flush_piece<T, D>(a, pos, piece_first && !same_seg, gw + seg, o, m_run, l_run, col, g);
      if (!more) return false;
      m_run = kNegBig;
      l_run = 0.f;
#pragma unroll
      for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};
      load_q<T, D>(qf, a, nxt, col, g);
      piece_first = nxt.seg_first;
    }
    pos = nxt;
    ++t;
    return true;
  };
  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
}

// Combine the pieces of each split (sequence, kv head) segment.
template <typename T, int D>
__global__ __launch_bounds__(256) void paged_decode_merge(AttnArgs a) {
  const uint32_t seq = blockIdx.y, kh = blockIdx.x;
  const uint32_t* P = a.plan;
  const uint32_t p0 = P[seq], p1 = P[seq + 1];
  if (p0 == p1) return;  // not a decode row
  const uint32_t S = P[a.batch], W = a.num_waves;
  const uint32_t nst = (p1 - p0) / a.kvh;
  const uint32_t t0 = p0 + kh * nst, t1 = t0 + nst - 1;
  auto wave_of = [&](uint32_t t) {
    return (uint32_t)((((uint64_t)t + 1) * W - 1) / S);
  };
  const uint32_t w0 = wave_of(t0), w1 = wave_of(t1);
  if (w0 == w1) return;  // one wave held the whole segment and wrote the output
  const uint32_t G = a.group, seg = seq * a.kvh + kh;
  __shared__ float sM[16], sInv[16];
  if (threadIdx.x < G) {
    const uint32_t hh = threadIdx.x;
    float M = kNegBig;
    for (uint32_t w = w0; w <= w1; ++w) M = fmaxf(M, a.ws_ml[((uint64_t)(w + seg) * G + hh) * 2]);
    float L = 0.f;
    for (uint32_t w = w0; w <= w1; ++w) {
      const float* ml = a.ws_ml + ((uint64_t)(w + seg) * G + hh) * 2;
      L += ml[1] * fast_exp2(ml[0] - M);
    }
    sM[hh] = M;
    sInv[hh] = L > 0.f ? 1.f / L : 0.f;
  }
  __syncthreads();
  const uint32_t q0 = a.cu_q[seq];
  for (uint32_t idx = threadIdx.x; idx < G * D; idx += 256) {
    const uint32_t hh = idx / D, d = idx % D;
    float O = 0.f;
    for (uint32_t w = w0; w <= w1; ++w) {
      const uint64_t sl = (uint64_t)(w + seg) * G + hh;
      O += a.ws_o[sl * D + d] * fast_exp2(a.ws_ml[sl * 2] - sM[hh]);
    }
    T* orow = (T*)a.out + ((uint64_t)q0 * a.num_heads + kh * G + hh) * D;
    orow[d] = from_f32<T>(O * sInv[hh]);
  }
}

uint32_t decode_num_waves() {
  static uint32_t cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cache[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = (uint32_t)cus * 2 * kDecodeWavesPerWG;  // 2 workgroups of 4 waves per CU
  }
  return cache[dev];
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t decode_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                              uint32_t num_waves) {
  const uint32_t b = std::min(batch, kMaxPlanSeqs);
  const size_t slots = (size_t)num_waves + (size_t)b * kvh;
  return up256((b + 1) * sizeof(uint32_t)) + up256(slots * group * 2 * sizeof(float)) +
         slots * group * head_dim * sizeof(float);
}

void launch_decode(AttnArgs a, void* workspace, uint32_t head_dim, bool bf16, hipStream_t s) {
  const uint32_t W = a.num_waves;
  const uint32_t total = a.batch;
  for (uint32_t b0 = 0; b0 < total; b0 += kMaxPlanSeqs) {
    const uint32_t nb = std::min(kMaxPlanSeqs, total - b0);
    AttnArgs c = a;
    c.batch = nb;
    c.cu_q = a.cu_q + b0;
    c.cu_k = a.cu_k + b0;
    c.table = a.table + (uint64_t)b0 * a.max_blocks;
    const size_t slots = (size_t)W + (size_t)nb * a.kvh;
    char* ws = (char*)workspace;
    c.plan = (uint32_t*)ws;
    c.ws_ml = (float*)(ws + up256((nb + 1) * sizeof(uint32_t)));
    c.ws_o = (float*)((char*)c.ws_ml + up256(slots * a.group * 2 * sizeof(float)));
    const dim3 grid(W / kDecodeWavesPerWG), block(64 * kDecodeWavesPerWG);
    const dim3 mgrid(a.kvh, nb);
#define VK_DEC(T, DD)                                                             \
  do {                                                                            \
    hipLaunchKernelGGL((paged_decode_stream<T, DD>), grid, block, 0, s, c);       \
    hipLaunchKernelGGL((paged_decode_merge<T, DD>), mgrid, dim3(256), 0, s, c);   \
  } while (0)
    if (bf16) {
      if (head_dim == 128) VK_DEC(bf16_t, 128);
      else VK_DEC(bf16_t, 64);
    } else {
      if (head_dim == 128) VK_DEC(f16_t, 128);
      else VK_DEC(f16_t, 64);
    }
#undef VK_DEC
  }
}

}  // namespace vk
