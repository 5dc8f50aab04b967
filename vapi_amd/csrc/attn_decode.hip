// Decode (len_q == 1) paged attention as one persistent stream with guided
// self-scheduling.
//
// The work of a decode batch is the sequence of 32-key steps over every
// (sequence, kv head) segment: segment (s, h) has ceil((len_k - lo32)/32)
// steps, where lo32 is the window start rounded down to 32. The grid holds
// exactly as many waves as the chip runs at once (CUs x 8). The first
// fraction of the S steps is split statically, wave w taking the contiguous
// slice [w*S1/W, (w+1)*S1/W); the rest is cut into chunks of a few steps that
// waves take from an atomic counter as they finish, so waves on faster
// CUs/XCDs (measured: +-25% spread in per-wave throughput) can absorb the
// tail. The static share defaults to 100% (see static_pct()).
// A wave keeps the next step's K/V in flight while it computes the current
// one, across segment and range boundaries, and asks for its next chunk one
// range ahead so the request latency is hidden too. Only the counter value is
// shared between waves, so no memory fence is needed (agent-scope fences on
// gfx950 write back the XCD-private L2s).
//
// Ranges (static slices r < W, chunks r = W + c) are increasing in step
// order, as are segments, so piece slot r + segment is unique. A range that
// covers a whole segment writes the normalised output directly; otherwise
// it writes the piece's (m, l, o) and paged_decode_merge combines the pieces.
// All G query heads of a kv head ride one MFMA tile, so K/V bytes are read
// exactly once.
#include <cstdlib>

#include "attn_common.hpp"

namespace vk {

constexpr int kDecodeWavesPerWG = 4;
constexpr uint32_t kMaxPlanSeqs = 4096;  // sequences per launch (host chunks beyond)

// Steps of sequence s (0 for rows that are not decode rows).
__device__ __forceinline__ uint32_t decode_steps(const AttnArgs& a,
                                                 const uint32_t* __restrict__ cu_q,
                                                 const uint32_t* __restrict__ cu_k, uint32_t s) {
  if (cu_q[s + 1] - cu_q[s] != 1) return 0;
  const int32_t len_k = (int32_t)(cu_k[s + 1] - cu_k[s]);
  if (len_k <= 0) return 0;
  const int32_t lo = a.wl >= 0 ? max(0, len_k - 1 - a.wl) : 0;
  return (uint32_t)(len_k - (lo & ~31) + 31) >> 5;
}

// Static/dynamic split of the S steps (identical in both kernels).
struct Split {
  uint32_t S, S1, C, K, W;
  __device__ __forceinline__ Split(const AttnArgs& a, uint32_t S_) : S(S_) {
    W = a.num_waves;
    K = a.chunk_steps;
    S1 = (uint32_t)(((uint64_t)S * a.static_num) / a.static_den);
    C = (S - S1 + K - 1) / K;
  }
  // Range holding step t.
  __device__ __forceinline__ uint32_t range_of(uint32_t t) const {
    if (t < S1) return (uint32_t)((((uint64_t)t + 1) * W - 1) / S1);
    return W + (t - S1) / K;
  }
};

// Where global step t lives.
struct DecodePos {
  uint32_t seq, kh, q0;
  int32_t key0, len_k, lo;
  uint32_t seg_first;  // key0 is the segment's first step (a word, not a bool: no stack copy)
};

__device__ __forceinline__ DecodePos locate(const AttnArgs& a, const uint32_t* __restrict__ cu_q,
                                            const uint32_t* __restrict__ cu_k, const uint32_t* P,
                                            uint32_t t) {
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
  p.q0 = cu_q[p.seq];
  p.len_k = (int32_t)(cu_k[p.seq + 1] - cu_k[p.seq]);
  p.lo = a.wl >= 0 ? max(0, p.len_k - 1 - a.wl) : 0;
  p.key0 = (p.lo & ~31) + 32 * (int32_t)ks;
  p.seg_first = ks == 0;
  return p;
}

template <typename T, int D>
__device__ __forceinline__ void load_q(uint4* qs, const AttnArgs& a, const DecodePos& p,
                                       uint32_t lane, uint32_t col, uint32_t g) {
  asm volatile("" : "+v"(lane), "+v"(col), "+v"(g));  // see flush_piece
  // MFMA columns past the group carry a copy of the group's first head: their
  // results are computed and never stored.
  const uint32_t h = col < a.group ? col : 0;
  const T* qrow = (const T*)a.q + ((uint64_t)p.q0 * a.num_heads + p.kh * a.group + h) * D;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    uint4 x = *(const uint4*)(qrow + 32 * c + 8 * g);
    x.x ^= a.q_sign, x.y ^= a.q_sign, x.z ^= a.q_sign, x.w ^= a.q_sign;
    qs[c * 64 + lane] = x;
  }
}

template <typename T, int D>
__device__ __forceinline__ void load_step_k(KTile<D>& st, const AttnArgs& a,
                                            const uint32_t* __restrict__ table,
                                            const DecodePos& p, uint32_t col, uint32_t g) {
  const uint32_t* __restrict__ tab = table + (uint64_t)p.seq * a.max_blocks;
  const T* kb = (const T*)a.k + p.kh * a.head_e;
  load_k<T, D>(st, tab, kb, a, p.key0, p.len_k - 1, col, g);
}

template <typename T, int D>
__device__ __forceinline__ void load_step_v(VTile<D>& st, const AttnArgs& a,
                                            const uint32_t* __restrict__ table,
                                            const DecodePos& p, uint32_t col, uint32_t g) {
  const uint32_t* __restrict__ tab = table + (uint64_t)p.seq * a.max_blocks;
  const T* vb = (const T*)a.v + p.kh * a.head_e;
  load_v<T, D>(st, tab, vb, a, p.key0, p.len_k - 1, col, g);
}

// Write a finished piece of segment (p.seq, p.kh): the final output if the
// piece is the whole segment, else a partial in slot `slot`.
template <typename T, int D>
__device__ __forceinline__ void flush_piece(const AttnArgs& a, const DecodePos& p, bool whole,
                                            uint32_t slot, const floatx4 (&o)[D / 16],
                                            float m_run, float l_run, uint32_t col, uint32_t g) {
  constexpr int DPL = D / 16;
  const uint32_t G = a.group;
  const float l_tot = wave_sum_g(l_run);
  // An opaque copy of the lane coordinates: keeps the compiler from hoisting
  // this rarely-taken path's per-lane addresses out of the step loop, where
  // they would pin registers the K/V buffers need.
  asm volatile("" : "+v"(col), "+v"(g));
  if (col >= G) return;  // lanes of padding columns hold no head
  if (whole) {
    T* orow = (T*)a.out + ((uint64_t)p.q0 * a.num_heads + p.kh * G + col) * D;
    store_row<T, D>(orow, o, l_tot > 0.f ? 1.f / l_tot : 0.f, g);
  } else {
    float* po = a.ws_o + ((uint64_t)slot * G + col) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < DPL; k += 4)
        *(float4*)(po + DPL * (4 * g + i) + k) =
            make_float4(o[k][i], o[k + 1][i], o[k + 2][i], o[k + 3][i]);
    if (g == 0) {
      float* ml = a.ws_ml + ((uint64_t)slot * G + col) * 2;
      ml[0] = m_run;
      ml[1] = l_tot;
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kDecodeWavesPerWG, 2) void paged_decode_stream(
    AttnArgs a, const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ cu_k,
    const uint32_t* __restrict__ table) {
  constexpr int DPL = D / 16;
  extern __shared__ uint32_t P[];  // batch + 1 entries (dynamic LDS)
  __shared__ uint32_t wave_tot[kDecodeWavesPerWG];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t B = a.batch;
  uint32_t* counter = a.plan + B + 1;

  // Step prefix sums over sequences (each sequence contributes kvh segments).
  {
    constexpr uint32_t NT = 64 * kDecodeWavesPerWG;
    const uint32_t per = (B + NT - 1) / NT;
    const uint32_t b0 = min(tid * per, B), b1 = min(b0 + per, B);
    uint32_t sum = 0;
    for (uint32_t s = b0; s < b1; ++s) sum += decode_steps(a, cu_q, cu_k, s) * a.kvh;
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
      run += decode_steps(a, cu_q, cu_k, s) * a.kvh;
    }
    if (tid == NT - 1) P[B] = run;
    __syncthreads();
    if (blockIdx.x == 0)
      for (uint32_t s = tid; s <= B; s += NT) a.plan[s] = P[s];
  }

  const Split sp(a, __builtin_amdgcn_readfirstlane(P[B]));
  const uint32_t gw = blockIdx.x * kDecodeWavesPerWG + wave;
  // Next chunk id: requested when the wave starts the second-to-last step of
  // its range (so requests from different waves spread out in time instead
  // of all hitting the counter at once), read at the last step; lane 0 holds
  // it until then.
  // (atomicInc, not atomicAdd: the compiler's atomic optimizer rewrites a
  // uniform-address add into a wave-aggregated form that broadcasts the
  // result at once, i.e. waits for it and for every load in flight.)
  auto request = [&]() -> uint32_t {
    uint32_t v = 0;
    if (lane == 0) v = atomicInc(counter, 0xFFFFFFFFu);
    return v;
  };

  uint32_t t = sp.S1 ? (uint32_t)(((uint64_t)gw * sp.S1) / sp.W) : 0;
  uint32_t t_end = sp.S1 ? (uint32_t)(((uint64_t)(gw + 1) * sp.S1) / sp.W) : 0;
  uint32_t r = gw;
  uint32_t nc_v = 0;
  bool asked = false;
  if (t >= t_end) {  // empty static slice: start on a chunk
    const uint32_t nc = __builtin_amdgcn_readfirstlane(request());
    if (nc >= sp.C) return;
    t = sp.S1 + nc * sp.K;
    t_end = min(t + sp.K, sp.S);
    r = sp.W + nc;
  }
#ifdef VK_DECODE_TRACE
  const uint64_t tr0 = __builtin_amdgcn_s_memrealtime();
  uint32_t nsteps = 0;
#endif

  const uint32_t col = lane & 15, g = lane >> 4;
  DecodePos pos = locate(a, cu_q, cu_k, P, t);
  // The Q^T operand of the current segment lives in LDS (read back every
  // step) to keep the two K/V buffers in registers without spilling.
  __shared__ uint4 q_lds[kDecodeWavesPerWG][D / 32 * 64];
  uint4* qs = q_lds[wave];
  load_q<T, D>(qs, a, pos, lane, col, g);
  bool piece_first = pos.seg_first;
  float m_run = kNegBig, l_run = 0.f;
  floatx4 o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};

  KTile<D> kA, kB;
  VTile<D> vA, vB;
  load_step_k<T, D>(kA, a, table, pos, col, g);
  load_step_v<T, D>(vA, a, table, pos, col, g);

  // One step: find the next step, prefetch its K before QK^T and its V
  // before PV (so at most three of the four tiles are live), flush when the
  // piece ends (segment or range boundary). Returns false when the wave has
  // no more work.
  auto step = [&](KTile<D>& kc, VTile<D>& vc, KTile<D>& kn, VTile<D>& vn) -> bool {
    const bool in_range = t + 1 < t_end;
    if (!asked && t + 2 >= t_end) {
      nc_v = request();
      asked = true;
    }
    bool more = in_range;
    uint32_t tn = t + 1, nc = 0;
    if (!in_range) {
      nc = __builtin_amdgcn_readfirstlane(nc_v);
      more = nc < sp.C;
      tn = sp.S1 + nc * sp.K;
    }
    const bool seg_ends = pos.key0 + 32 >= pos.len_k;
    const bool same_piece = in_range && !seg_ends;
    // The next step's loads are issued unconditionally (the final step of a
    // wave re-reads its own tiles, which hit in L2): a load inside a branch
    // makes the waitcnt pass assume it may be the newest and wait for the
    // prefetch before this step's MFMAs.
    DecodePos nxt = pos;
    if (more) {
      if (same_piece) {
        nxt.key0 += 32;
        nxt.seg_first = false;
      } else {
        nxt = locate(a, cu_q, cu_k, P, tn);
      }
    }
    load_step_k<T, D>(kn, a, table, nxt, col, g);
    const int32_t lo = pos.lo, len_k = pos.len_k, key0 = pos.key0;
    uint4 qf[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; ++c) qf[c] = qs[c * 64 + lane];
    const uint4 pf = attend_qk<T, D>(kc, qf, o, m_run, l_run, a.scale_log2, g, [&](int tt, int i) {
      const int32_t key = key0 + 16 * tt + 4 * (int32_t)g + i;
      return key >= lo && key < len_k;
    });
    load_step_v<T, D>(vn, a, table, nxt, col, g);
    attend_pv<T, D>(vc, pf, o);
#ifdef VK_DECODE_TRACE
    ++nsteps;
#endif
    if (!same_piece) {
      const uint32_t seg = pos.seq * a.kvh + pos.kh;
      flush_piece<T, D>(a, pos, piece_first && seg_ends, r + seg, o, m_run, l_run, col, g);
      if (!more) return false;
      m_run = kNegBig;
      l_run = 0.f;
#pragma unroll
      for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};
      load_q<T, D>(qs, a, nxt, lane, col, g);
      piece_first = nxt.seg_first;
    }
    if (!in_range) {
      r = sp.W + nc;
      t_end = min(tn + sp.K, sp.S);
      asked = false;
    }
    pos = nxt;
    t = tn;
    return true;
  };
  while (step(kA, vA, kB, vB) && step(kB, vB, kA, vA)) {
  }
#ifdef VK_DECODE_TRACE
  // Per wave: start/end (100 MHz ticks), steps done, last sequence.
  if (lane == 0) {
    uint64_t* tr = a.trace + 4ull * gw;
    tr[0] = tr0;
    tr[1] = __builtin_amdgcn_s_memrealtime();
    tr[2] = nsteps;
    tr[3] = pos.seq;
  }
#endif
}

// Combine the pieces of each split (sequence, kv head) segment; reset the
// chunk counter for the next launch.
template <typename T, int D>
__global__ __launch_bounds__(256) void paged_decode_merge(AttnArgs a) {
  const uint32_t seq = blockIdx.y, kh = blockIdx.x;
  const uint32_t* P = a.plan;
  if (seq == 0 && kh == 0 && threadIdx.x == 0) a.plan[a.batch + 1] = 0;
  const uint32_t p0 = P[seq], p1 = P[seq + 1];
  if (p0 == p1) return;  // not a decode row
  const Split sp(a, P[a.batch]);
  const uint32_t nst = (p1 - p0) / a.kvh;
  const uint32_t t0 = p0 + kh * nst, t1 = t0 + nst - 1;
  const uint32_t r0 = sp.range_of(t0), r1 = sp.range_of(t1);
  if (r0 == r1) return;  // one range held the whole segment and wrote the output
  const uint32_t G = a.group, seg = seq * a.kvh + kh;
  const uint32_t q0 = a.cu_q[seq];
  // One pass per output: an online merge of the pieces, four at a time so
  // their loads are in flight together.
  for (uint32_t idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const uint32_t hh = idx / D, d = idx % D;
    float M = kNegBig, L = 0.f, O = 0.f;
    for (uint32_t w = r0; w <= r1; w += 4) {
      float m[4], l[4], o[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t ww = min(w + u, r1);
        const uint64_t sl = (uint64_t)(ww + seg) * G + hh;
        const float2 x = *(const float2*)(a.ws_ml + sl * 2);
        m[u] = w + u <= r1 ? x.x : kNegBig;
        l[u] = x.y;
        o[u] = a.ws_o[sl * D + d];
      }
      const float Mn = fmaxf(fmaxf(M, fmaxf(m[0], m[1])), fmaxf(m[2], m[3]));
      const float f = fast_exp2(M - Mn);
      L *= f;
      O *= f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float e = fast_exp2(m[u] - Mn);
        L += l[u] * e;
        O += o[u] * e;
      }
      M = Mn;
    }
    T* orow = (T*)a.out + ((uint64_t)q0 * a.num_heads + kh * G + hh) * D;
    orow[d] = from_f32<T>(L > 0.f ? O / L : 0.f);
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

// Scheduling knobs: static fraction (percent) and chunk size (steps).
// VAPI_KV_DECODE_STATIC_PCT / VAPI_KV_DECODE_CHUNK override them, for tuning.
static uint32_t env_u32(const char* name, uint32_t def, uint32_t lo, uint32_t hi) {
  const char* e = getenv(name);
  if (!e) return def;
  const long v = atol(e);
  return (v < (long)lo || v > (long)hi) ? def : (uint32_t)v;
}
// Default: all static. Measured on config 2 (64 sequences, 2k median
// context), chunked tails cost more in piece switches and merge work than
// they recover in balance (150 us all-static vs 158-182 us at 70-30% static).
static uint32_t static_pct() {
  static const uint32_t v = env_u32("VAPI_KV_DECODE_STATIC_PCT", 100, 0, 100);
  return v;
}
static uint32_t chunk_steps() {
  static const uint32_t v = env_u32("VAPI_KV_DECODE_CHUNK", 8, 1, 1024);
  return v;
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// Slots: static ranges (W) + chunks (upper bound from max_seqlen_k) + one per
// segment.
static size_t decode_slots(uint32_t b, uint32_t kvh, uint32_t max_k, uint32_t num_waves) {
  const uint64_t s_max = (uint64_t)b * kvh * ((max_k + 31) / 32 + 1);
  const uint64_t chunks = (s_max * (100 - static_pct()) / 100 + chunk_steps()) / chunk_steps() + 1;
  return (size_t)num_waves + chunks + (size_t)b * kvh;
}

struct DecodeWs {
  size_t plan, ml, o, trace, total;
};
static DecodeWs decode_ws(uint32_t b, uint32_t kvh, uint32_t group, uint32_t head_dim,
                          uint32_t max_k, uint32_t num_waves) {
  const size_t slots = decode_slots(b, kvh, max_k, num_waves);
  DecodeWs w;
  w.plan = 0;
  w.ml = up256((b + 2) * sizeof(uint32_t));
  w.o = w.ml + up256(slots * group * 2 * sizeof(float));
  w.trace = w.o + up256(slots * group * head_dim * sizeof(float));
  w.total = w.trace;
#ifdef VK_DECODE_TRACE
  w.total += (size_t)num_waves * 4 * sizeof(uint64_t);
#endif
  return w;
}

size_t decode_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                              uint32_t max_k, uint32_t num_waves) {
  return decode_ws(std::min(batch, kMaxPlanSeqs), kvh, group, head_dim, max_k, num_waves).total;
}

void launch_decode(AttnArgs a, void* workspace, uint32_t head_dim, uint32_t max_k, bool bf16,
                   hipStream_t s) {
  const uint32_t W = a.num_waves;
  const uint32_t total = a.batch;
  a.static_num = static_pct();
  a.static_den = 100;
  a.chunk_steps = chunk_steps();
  for (uint32_t b0 = 0; b0 < total; b0 += kMaxPlanSeqs) {
    const uint32_t nb = std::min(kMaxPlanSeqs, total - b0);
    AttnArgs c = a;
    c.batch = nb;
    c.cu_q = a.cu_q + b0;
    c.cu_k = a.cu_k + b0;
    c.table = a.table + (uint64_t)b0 * a.max_blocks;
    const DecodeWs w = decode_ws(nb, a.kvh, a.group, head_dim, max_k, W);
    char* ws = (char*)workspace;
    c.plan = (uint32_t*)(ws + w.plan);
    c.ws_ml = (float*)(ws + w.ml);
    c.ws_o = (float*)(ws + w.o);
#ifdef VK_DECODE_TRACE
    c.trace = (uint64_t*)(ws + w.trace);
#endif
    const dim3 grid(W / kDecodeWavesPerWG), block(64 * kDecodeWavesPerWG);
    const dim3 mgrid(a.kvh, nb);
#define VK_DEC(T, DD)                                                                        \
  do {                                                                                       \
    hipLaunchKernelGGL((paged_decode_stream<T, DD>), grid, block, (nb + 1) * sizeof(uint32_t), \
                       s, c, c.cu_q, c.cu_k,                                                 \
                       c.table);                                                             \
    hipLaunchKernelGGL((paged_decode_merge<T, DD>), mgrid, dim3(256), 0, s, c);              \
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
