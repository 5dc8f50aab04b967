// Decode (len_q == 1) paged attention as one persistent stream, one launch.
//
// The work of a decode batch is the sequence of 32-key steps over every
// (sequence, kv head) segment: segment (s, h) has ceil((len_k - lo32)/32)
// steps, where lo32 is the window start rounded down to 32. The grid holds
// one workgroup of 4 waves per CU, one wave per SIMD: two waves sharing a
// SIMD do not share it fairly on gfx950 (the older one issues first and
// streams about 3x faster), so equal shares would not finish together. Each
// wave keeps a whole step (K and V, 16 KiB) in flight while it computes the
// current one, which keeps HBM saturated with 4 waves per CU.
//
// The XCDs differ in per-wave bandwidth (by up to ~15% on one box, and which
// XCD is slow differs between boxes), so the steps are split into 8 group
// ranges, one per XCD (workgroup b runs on XCD b % 8), in proportion to
// shares that each launch measures for the next: every wave records its
// steps and its entry and end times, and the merge kernel moves the shares
// halfway to the measured per-group rates, counted from the grid's first
// entry (the XCDs start the grid up to ~2.5 us apart). Within a group each wave takes an
// equal contiguous slice. Any shares give the same results up to the f32
// merge order; the shares only move where the pieces split.
//
// A wave's run of steps within one segment is a piece. A piece covering a
// whole segment writes the normalised output; the first and last piece of a
// slice may be partial and write (m, l, o) to slot range + segment (ranges
// and segments are both numbered in step order, so slots are unique; with a
// group split into n parts, range x n + virtual segment), and
// paged_decode_merge combines them: one wave per split segment, or, when a
// launch has at most 256 segments (each then split into many pieces), one
// workgroup per segment whose waves share its pieces. Each
// segment's first and last range are recorded by the waves holding its first
// and last step, and a wave whose slice is empty marks its slot empty, so
// the merge needs no step arithmetic. The merge
// kernel's extra workgroup turns the stream's per-wave timings into the
// next launch's shares. (Merging inside the stream, by the wave that
// completes a segment, needs write-through stores, L2-bypassing loads and
// counters across XCDs; measured, it costs more at the tail than the
// second launch.)
//
// All G query heads of a kv head ride one MFMA tile, so K/V bytes are read
// exactly once.
#pragma once
#include <cstdlib>
#include <type_traits>

#include "attn_common.hpp"


namespace vk {

constexpr int kDecodeWavesPerWG = 4;
constexpr int kDecodeWGsPerCU = 1;
constexpr uint32_t kGroups = 8;          // XCDs; workgroup b runs on XCD b % 8
constexpr uint32_t kMergeWaves = 4;  // merge: segments (waves) per workgroup
constexpr uint32_t kMaxPlanSeqs = 4096;  // sequences per launch (host chunks beyond)

// Balance block (u32 words, kept across launches at the start of the
// workspace): shares f32[8] at 0, per-wave (steps, entry tick, end tick, 0)
// from kBalStats.
constexpr uint32_t kBalStats = 64;
constexpr uint32_t kMinStepsPerWave = 8;  // launches that move the shares
constexpr uint32_t kStatWords = 4;

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

// Waves in group x and the number of waves in groups before it.
__device__ __forceinline__ uint32_t group_waves(uint32_t nwg, uint32_t x) {
  return nwg > x ? ((nwg - 1 - x) / kGroups + 1) * kDecodeWavesPerWG : 0u;
}
__device__ __forceinline__ uint32_t group_offset(uint32_t nwg, uint32_t x) {
  uint32_t off = 0;
  for (uint32_t y = 0; y < x; ++y) off += group_waves(nwg, y);
  return off;
}

// The shares of this launch: 8 positive f32, uniform when the workspace
// holds none yet (all zero) or anything unusable; 0 for groups without waves.
__device__ __forceinline__ void load_shares(const AttnArgs& a, uint32_t nwg, float (&w)[kGroups]) {
  bool ok = !a.deterministic;
#pragma unroll
  for (uint32_t x = 0; x < kGroups; ++x) {
    w[x] = __uint_as_float(a.bal[x]);
    ok = ok && w[x] > 0.f && w[x] < 1e6f;
  }
#pragma unroll
  for (uint32_t x = 0; x < kGroups; ++x) {
    if (!ok) w[x] = 1.f;
    if (!group_waves(nwg, x)) w[x] = 0.f;
  }
}

// Group x covers steps [F[x], F[x + 1]) of S.
__device__ __forceinline__ void group_bounds(const float (&w)[kGroups], uint32_t S,
                                             uint32_t (&F)[kGroups + 1]) {
  float tot = 0.f;
#pragma unroll
  for (uint32_t x = 0; x < kGroups; ++x) tot += w[x];
  float run = 0.f;
  F[0] = 0;
#pragma unroll
  for (uint32_t x = 1; x < kGroups; ++x) {
    run += w[x - 1];
    const uint32_t f = (uint32_t)fminf((float)S, floorf((float)S * (run / tot)));
    F[x] = max(F[x - 1], f);
  }
  F[kGroups] = S;
}

// Where global step t lives.
struct DecodePos {
  uint32_t seq, kh, q0;
  int32_t key0, len_k, lo;
  uint32_t seg_first;  // key0 is the segment's first step (a word, not a bool: no stack copy)
  uint32_t fuse;       // fused append: key len_k - 1 is read from the new rows
};

// kvh_plan: the kv heads the step order counts (a.kvh, or with a split
// group's parts side by side the pool heads: then the position is part
// `part` of pool head kp, virtual head kp * n + part).
__device__ __forceinline__ DecodePos locate(const AttnArgs& a, const uint32_t* __restrict__ cu_q,
                                            const uint32_t* __restrict__ cu_k, const uint32_t* P,
                                            const uint32_t* FZ, uint32_t t,
                                            uint32_t kvh_plan, uint32_t n, uint32_t part) {
  uint32_t lo_i = 0, hi_i = a.batch;  // P[lo_i] <= t < P[hi_i]
  while (hi_i - lo_i > 1) {
    const uint32_t mid = (lo_i + hi_i) >> 1;
    if (__builtin_amdgcn_readfirstlane(P[mid]) <= t) lo_i = mid;
    else hi_i = mid;
  }
  DecodePos p;
  p.seq = lo_i;
  const uint32_t p0 = __builtin_amdgcn_readfirstlane(P[lo_i]);
  const uint32_t nst = (__builtin_amdgcn_readfirstlane(P[lo_i + 1]) - p0) / kvh_plan;
  const uint32_t local = t - p0;
  const uint32_t kp = local / nst;
  p.kh = kp * n + part;
  const uint32_t ks = local - kp * nst;
  p.q0 = cu_q[p.seq];
  p.len_k = (int32_t)(cu_k[p.seq + 1] - cu_k[p.seq]);
  p.lo = a.wl >= 0 ? max(0, p.len_k - 1 - a.wl) : 0;
  p.key0 = (p.lo & ~31) + 32 * (int32_t)ks;
  p.seg_first = ks == 0;
  p.fuse = FZ ? FZ[lo_i] : 0u;
  return p;
}

// The first step of the segment after `cur` in step order: (seq, kh + 1),
// or kv head 0 of the next sequence that has decode steps. A wave's slice
// is contiguous, so the step after a segment's last is always this one,
// and a wave that moves on from a finished segment needs no search.
__device__ __forceinline__ DecodePos next_segment(const AttnArgs& a,
                                                  const uint32_t* __restrict__ cu_q,
                                                  const uint32_t* __restrict__ cu_k,
                                                  const uint32_t* P, const uint32_t* FZ,
                                                  const DecodePos& cur, uint32_t n) {
  // With n > 1 a wave walks one part of each pool head: kh steps by n.
  DecodePos p = cur;
  if (cur.kh + n < a.kvh) {
    p.kh = cur.kh + n;
  } else {
    uint32_t s = cur.seq + 1;
    while (s + 1 < a.batch && __builtin_amdgcn_readfirstlane(P[s + 1]) ==
                                  __builtin_amdgcn_readfirstlane(P[s]))
      ++s;  // sequences without decode steps
    p.seq = s;
    p.kh = cur.kh % n;
    p.q0 = cu_q[s];
    p.len_k = (int32_t)(cu_k[s + 1] - cu_k[s]);
    p.lo = a.wl >= 0 ? max(0, p.len_k - 1 - a.wl) : 0;
    p.fuse = FZ ? FZ[s] : 0u;
  }
  p.key0 = p.lo & ~31;
  p.seg_first = 1u;
  return p;
}

// The first query head of virtual kv head v, and how many it serves (the
// last part of a split group may serve fewer than a.group).
__device__ __forceinline__ uint32_t vhead_base(const AttnArgs& a, uint32_t v) {
  const uint32_t kp = a.kv_parts.div(v);
  return kp * a.g_real + (v - kp * a.kv_parts.d) * a.group;
}
__device__ __forceinline__ uint32_t vhead_count(const AttnArgs& a, uint32_t v) {
  const uint32_t part = v - a.kv_parts.div(v) * a.kv_parts.d;
  return min(a.group, a.g_real - part * a.group);
}

// kPad: the pool's head_dim a.hd is below D (its rows are a.hd apart);
// elements d >= a.hd are zeros.
template <typename T, int D, bool kPad = false>
__device__ __forceinline__ void load_q(uint4* qs, const AttnArgs& a, const DecodePos& p,
                                       uint32_t lane, uint32_t col, uint32_t g) {
  asm volatile("" : "+v"(lane), "+v"(col), "+v"(g));  // see flush_piece
  // MFMA columns past the group carry a copy of the group's first head: their
  // results are computed and never stored.
  const uint32_t h = col < vhead_count(a, p.kh) ? col : 0;
  const uint32_t hd = kPad ? a.hd : (uint32_t)D;
  const T* qrow =
      (const T*)a.q + ((uint64_t)p.q0 * a.num_heads + vhead_base(a, p.kh) + h) * hd;
  if constexpr (sizeof(T) == 4) {
    // f32: D / 16 float4 per lane, Q[h][16c + 4g .. +3] (the f32 MFMA's k
    // order); a negative scale flips the sign bit of every element.
    const uint32_t sg = a.q_sign ? 0x80000000u : 0u;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      uint4 x = !kPad || 16 * c + 4 * g < hd ? *(const uint4*)(qrow + 16 * c + 4 * g)
                                             : make_uint4(0u, 0u, 0u, 0u);
      x.x ^= sg, x.y ^= sg, x.z ^= sg, x.w ^= sg;
      qs[c * 64 + lane] = x;
    }
  } else {
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      uint4 x = !kPad || 32 * c + 8 * g < hd ? *(const uint4*)(qrow + 32 * c + 8 * g)
                                             : make_uint4(0u, 0u, 0u, 0u);
      x.x ^= a.q_sign, x.y ^= a.q_sign, x.z ^= a.q_sign, x.w ^= a.q_sign;
      qs[c * 64 + lane] = x;
    }
  }
}

template <typename T, int D, bool kPad = false, int KCL = D / 32, bool kNt = true>
__device__ __forceinline__ void load_step_k(KTile<D>& st, const AttnArgs& a,
                                            const uint32_t* __restrict__ table,
                                            const DecodePos& p, uint32_t col, uint32_t g) {
  const uint32_t* __restrict__ tab = table + (uint64_t)p.seq * a.max_blocks;
  const T* kb = (const T*)a.k + a.kv_parts.div(p.kh) * a.head_e;
  const char* knew =
      p.fuse ? a.k_new + ((uint64_t)p.q0 * a.kvh + p.kh) * D * sizeof(T) : nullptr;
  load_k<T, D, kPad, KCL, kNt>(st, tab, kb, a, p.key0, p.len_k - 1, col, g, knew);
}

template <typename T, int D, bool kPad = false, bool kNt = true>
__device__ __forceinline__ void load_step_v(VTile<D>& st, const AttnArgs& a,
                                            const uint32_t* __restrict__ table,
                                            const DecodePos& p, uint32_t col, uint32_t g) {
  const uint32_t* __restrict__ tab = table + (uint64_t)p.seq * a.max_blocks;
  const T* vb = (const T*)a.v + a.kv_parts.div(p.kh) * a.head_e;
  const char* vnew =
      p.fuse ? a.v_new + ((uint64_t)p.q0 * a.kvh + p.kh) * D * sizeof(T) : nullptr;
  load_v<T, D, kPad, kNt>(st, tab, vb, a, p.key0, p.len_k - 1, col, g, vnew);
}


// Write a finished piece of segment (p.seq, p.kh): the final output if the
// piece is the whole segment, else a partial in slot `slot`.
template <typename T, int D, bool kPad = false>
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
  if (col >= vhead_count(a, p.kh)) return;  // lanes of padding columns hold no head
  const uint32_t h0 = vhead_base(a, p.kh);
  if constexpr (sizeof(T) == 4) {
    if (whole) {
      const uint32_t hd = kPad ? a.hd : (uint32_t)D;
      float* orow = (float*)a.out + ((uint64_t)p.q0 * a.num_heads + h0 + col) * hd;
      store_row_f32<D, kPad>(orow, o, l_tot > 0.f ? 1.f / l_tot : 0.f, g, hd);
    } else {
      store_row_f32<D>(a.ws_o + ((uint64_t)slot * G + col) * D, o, 1.f, g);
      if (g == 0) *(float2*)(a.ws_ml + ((uint64_t)slot * G + col) * 2) = make_float2(m_run, l_tot);
    }
    return;
  }
  if (whole) {
    const uint32_t hd = kPad ? a.hd : (uint32_t)D;
    T* orow = (T*)a.out + ((uint64_t)p.q0 * a.num_heads + h0 + col) * hd;
    store_row<T, D, kPad>(orow, o, l_tot > 0.f ? 1.f / l_tot : 0.f, g, hd);
  } else {
    float* po = a.ws_o + ((uint64_t)slot * G + col) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < DPL; k += 4)
        *(float4*)(po + v_d<D>(4 * g + i, k)) =
            make_float4(o[k][i], o[k + 1][i], o[k + 2][i], o[k + 3][i]);
    if (g == 0) *(float2*)(a.ws_ml + ((uint64_t)slot * G + col) * 2) = make_float2(m_run, l_tot);
  }
}

// The persistent stream of workgroup `bid` of `nwg` (4 waves). P: the
// launch's dynamic LDS, step prefix sums (batch + 1), then with kFuse the
// per-sequence fused-append flags FZ (batch).
// DL: the 16-column d tiles that hold head_dim (kPad; D / 16 otherwise):
// K chunks past them are neither loaded nor multiplied (V and O keep D: a
// lane's V values spread over every d tile). kNt: K/V read with streaming
// loads; ordinary ones for a group split into virtual kv heads, whose
// parts read the same tiles at about the same time on one XCD (the plan
// puts a pool head's parts side by side), so all but the first hit in L2.
template <typename T, int D, bool kFuse, bool kPad = false, int DL = D / 16, bool kNt = true>
__device__ __forceinline__ void decode_stream_body(const AttnArgs& a,
                                                   const uint32_t* __restrict__ cu_q,
                                                   const uint32_t* __restrict__ cu_k,
                                                   const uint32_t* __restrict__ table,
                                                   uint32_t* P, uint32_t bid, uint32_t nwg) {
  constexpr int DPL = D / 16;
  uint32_t* const FZ = kFuse ? P + a.batch + 1 : nullptr;
  __shared__ uint32_t wave_tot[kDecodeWavesPerWG];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t B = a.batch;
  // A group split into n virtual kv heads: steps are counted per pool
  // head, each of n neighbouring waves walking one part (n = 1: the
  // virtual heads are the pool's).
  const uint32_t n_parts = a.kv_parts.d;
  const uint32_t kvh_plan = a.kvh / n_parts;
  // The shared 100 MHz clock at entry: XCDs start the grid up to ~2.5 us
  // apart, and the shares account for it.
  const uint32_t t_entry = (uint32_t)__builtin_amdgcn_s_memrealtime();

  // Step prefix sums over sequences (each sequence contributes kvh segments).
  {
    constexpr uint32_t NT = 64 * kDecodeWavesPerWG;
    const uint32_t per = (B + NT - 1) / NT;
    const uint32_t b0 = min(tid * per, B), b1 = min(b0 + per, B);
    uint32_t sum = 0;
    for (uint32_t s = b0; s < b1; ++s) sum += decode_steps(a, cu_q, cu_k, s) * kvh_plan;
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
      const uint32_t ns = decode_steps(a, cu_q, cu_k, s);
      run += ns * kvh_plan;
      if (kFuse) {
        // The row's new key (position len_k - 1) comes from token cu_q[s]
        // of the new rows if that token's slot is the one the block table
        // gives the position; otherwise the pool is read.
        uint32_t f = 0;
        if (ns) {
          const uint32_t q0 = cu_q[s], last = cu_k[s + 1] - cu_k[s] - 1;
          const uint32_t slot = q0 < a.n_new ? a.slots[q0] : 0xFFFFFFFFu;
          // Column clamped like every other table read: len_k past the row's
          // max_blocks * block_size reads the row's last entry.
          const uint32_t blk =
              table[(uint64_t)s * a.max_blocks + min(last >> a.bs_shift, a.max_blocks - 1)];
          f = slot < a.num_slots && slot == blk * a.block_size + (last & (a.block_size - 1));
        }
        FZ[s] = f;
      }
    }
    if (tid == NT - 1) P[B] = run;
    __syncthreads();
  }

  const uint32_t S = __builtin_amdgcn_readfirstlane(P[B]);
  float w[kGroups];
  load_shares(a, nwg, w);
  uint32_t F[kGroups + 1];
  group_bounds(w, S, F);
  const uint32_t x = bid % kGroups;
  const uint32_t j = (bid / kGroups) * kDecodeWavesPerWG + wave;
  const uint32_t len = F[x + 1] - F[x], nw = group_waves(nwg, x);
  // The group's waves form ranges of n consecutive waves, wave j taking
  // part j % n of range j / n (waves past the last whole range idle), so
  // the parts of a pool head's steps are read at once, by neighbouring
  // waves of one XCD. A piece's partial slot is r n + (virtual segment):
  // r + (pool segment) is distinct for every piece of one part, as in the
  // unsplit order, so the slots of all parts are too.
  const uint32_t nr = nw / n_parts;
  const uint32_t jr = j / n_parts;
  const uint32_t part = j - jr * n_parts;
  const uint32_t t_begin = jr < nr ? F[x] + (uint32_t)(((uint64_t)jr * len) / nr) : S;
  const uint32_t t_end = jr < nr ? F[x] + (uint32_t)(((uint64_t)(jr + 1) * len) / nr) : S;
  const uint32_t r = group_offset(nwg, x) / n_parts + jr;
  const uint32_t gw = bid * kDecodeWavesPerWG + wave;
  uint32_t* stat = a.bal + kBalStats + kStatWords * gw;
  if (t_begin >= t_end) {
    if (lane == 0) *(uint4*)stat = make_uint4(0u, t_entry, t_entry, 0u);
    // An empty slice between the first and last range of a segment: its
    // partial slot is marked empty (l = 0) for the merge.
    if (t_begin < S) {
      const DecodePos p = locate(a, cu_q, cu_k, P, FZ, t_begin, kvh_plan, n_parts, part);
      const uint64_t slot = (uint64_t)r * n_parts + p.seq * a.kvh + p.kh;
      if (lane < a.group) *(float2*)(a.ws_ml + (slot * a.group + lane) * 2) = make_float2(kNegBig, 0.f);
    }
    return;
  }

  uint32_t t = t_begin;
  const uint32_t col = lane & 15, g = lane >> 4;
  DecodePos pos = locate(a, cu_q, cu_k, P, FZ, t, kvh_plan, n_parts, part);
  // The Q^T operand of the current segment lives in LDS (read back every
  // step) to keep the K/V buffers in registers.
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int KCL = (DL + 1) / 2;  // live 32-column K chunks (16-bit)
  __shared__ uint4 q_lds[kDecodeWavesPerWG][D / 32 * 64 * sizeof(T) / 2];
  uint4* qs = q_lds[wave];
  load_q<T, D, kPad>(qs, a, pos, lane, col, g);
  bool piece_first = pos.seg_first;
  float m_run = kNegBig, l_run = 0.f;
  floatx4 o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};

  // 16-bit pools: two 32-key steps in registers (the next one loading while
  // the current one is computed). f32 pools: one 32-key step as two 16-key
  // halves, each reloaded with the next step's half once it is computed.
  using KBuf = std::conditional_t<kF32, KTileF32<D>, KTile<D>>;
  using VBuf = std::conditional_t<kF32, VTileF32<D>, VTile<D>>;
  KBuf kA, kB;
  VBuf vA, vB;
  const float* kbf = (const float*)a.k;
  const float* vbf = (const float*)a.v;
  auto load_halves = [&](KTileF32<D>& kt, VTileF32<D>& vt, const DecodePos& p, int tt)
      __attribute__((always_inline)) {
    load_half_f32<D, kNt, kPad, DL>(kt.h[tt], vt.h[tt], table + (uint64_t)p.seq * a.max_blocks,
                     kbf + a.kv_parts.div(p.kh) * a.head_e, vbf + a.kv_parts.div(p.kh) * a.head_e,
                     a, p.key0, tt, p.len_k - 1,
                     col, g);
  };
  if constexpr (kF32) {
    load_halves(kA, vA, pos, 0);
    load_halves(kA, vA, pos, 1);
  } else {
    load_step_k<T, D, kPad, KCL, kNt>(kA, a, table, pos, col, g);
    load_step_v<T, D, kPad, kNt>(vA, a, table, pos, col, g);
  }

  // One step: find the next step, issue its K and V, attend over the current
  // one, flush when the piece ends (segment or slice boundary). Returns
  // false when the slice is done.
  auto step = [&](KBuf& kc, VBuf& vc, KBuf& kn, VBuf& vn) -> bool {
    const bool more = t + 1 < t_end;
    const bool seg_ends = pos.key0 + 32 >= pos.len_k;
    const bool same_piece = more && !seg_ends;
    // The next step's loads are issued unconditionally: a load inside a
    // branch makes the waitcnt pass assume it may be the newest and wait for
    // the prefetch before this step's MFMAs. The final step of a wave points
    // them at key 0 of sequence 0 (one row of one tile per kv head, the same
    // for every wave, so they hit in L2): the K/V loads are streaming, and a
    // re-read of the wave's own tiles would go to HBM again (16 KiB per wave)
    // and hold the wave's end for a memory round trip.
    DecodePos nxt = pos;
    if (same_piece) {
      nxt.key0 += 32;
      nxt.seg_first = false;
    } else if (more) {
      nxt = next_segment(a, cu_q, cu_k, P, FZ, pos, n_parts);
    } else {
      nxt.seq = 0;
      nxt.key0 = 0;
      nxt.len_k = 1;
      nxt.fuse = 0;
    }
    const int32_t lo = pos.lo, len_k = pos.len_k, key0 = pos.key0;
    if constexpr (kF32) {
      // kn, vn are kc, vc: each half is refilled with the next step's once
      // it has been computed (16 KiB in flight per wave, as 16-bit steps).
      float4 qf[D / 16];
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const uint4 x = qs[c * 64 + lane];
        qf[c] = make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                            __uint_as_float(x.w));
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        attend_half_f32<D, DL>(kc.h[tt], vc.h[tt], qf, o, m_run, l_run, a.scale_log2, [&](int i) {
          const int32_t key = key0 + 16 * tt + 4 * (int32_t)g + i;
          return key >= lo && key < len_k;
        });
        load_halves(kn, vn, nxt, tt);
      }
    } else {
      load_step_k<T, D, kPad, KCL, kNt>(kn, a, table, nxt, col, g);
      load_step_v<T, D, kPad, kNt>(vn, a, table, nxt, col, g);
      uint4 qf[D / 32];
#pragma unroll
      for (int c = 0; c < D / 32; ++c) qf[c] = qs[c * 64 + lane];
      const uint4 pf = attend_qk<T, D, KCL>(kc, qf, o, m_run, l_run, a.scale_log2, g, [&](int tt, int i) {
        const int32_t key = key0 + 16 * tt + 4 * (int32_t)g + i;
        return key >= lo && key < len_k;
      });
      attend_pv<T, D>(vc, pf, o);
    }
    if (!same_piece) {
      const uint32_t seg = pos.seq * a.kvh + pos.kh;
      if (lane == 0) {
        if (piece_first) a.seg_ranges[2 * seg] = r;
        if (seg_ends) a.seg_ranges[2 * seg + 1] = r;
      }
      flush_piece<T, D, kPad>(a, pos, piece_first && seg_ends, r * n_parts + seg, o, m_run, l_run,
                              col, g);
      if (!more) return false;
      m_run = kNegBig;
      l_run = 0.f;
#pragma unroll
      for (int k = 0; k < DPL; ++k) o[k] = floatx4{0.f, 0.f, 0.f, 0.f};
      load_q<T, D, kPad>(qs, a, nxt, lane, col, g);
      piece_first = nxt.seg_first;
    }
    pos = nxt;
    ++t;
    return true;
  };
  if constexpr (kF32) {
    while (step(kA, vA, kA, vA)) {
    }
  } else {
    while (step(kA, vA, kB, vB) && step(kB, vB, kA, vA)) {
    }
  }
  const uint32_t t_done = (uint32_t)__builtin_amdgcn_s_memrealtime();
  if (lane == 0) {
    *(uint4*)stat = make_uint4(t_end - t_begin, t_entry, t_done, 0u);
  }
}

// The next launch's shares from this launch's per-wave timings: each group
// that ran keeps its total and moves halfway to its measured rate, steps
// per tick per wave counted from the grid's first entry (so a group whose
// XCD started late, or streamed slower, gets fewer steps and the groups end
// together); groups without steps keep their share. Ticks are the low 32
// bits of the shared 100 MHz clock, compared as differences.
__device__ __forceinline__ void update_shares(const AttnArgs& a, uint32_t nwg, uint32_t lane) {
  float steps[kGroups], ticks[kGroups];
  const uint32_t W = nwg * kDecodeWavesPerWG;
  // Wave gw belongs to group (gw / 4) % 8, so the waves lane l reads (l,
  // l + 64, ...) all belong to group (l / 4) % 8.
  // All of a lane's loads are issued before the first is used (one memory
  // round trip instead of W / 64 dependent ones).
  constexpr uint32_t kBatch = 16;
  const uint32_t* stats = a.bal + kBalStats;
  const uint32_t ref = __builtin_amdgcn_readfirstlane(stats[1]);  // wave 0's entry
  float st = 0.f, tk = 0.f, cnt = 0.f;
  int32_t first = 0;
  for (uint32_t base = 0; base < W; base += 64 * kBatch) {
    uint4 v[kBatch];
#pragma unroll
    for (uint32_t i = 0; i < kBatch; ++i) {
      const uint32_t gw = base + 64 * i + lane;
      v[i] = gw < W ? *(const uint4*)(stats + kStatWords * gw) : make_uint4(0u, ref, ref, 0u);
    }
#pragma unroll
    for (uint32_t i = 0; i < kBatch; ++i) {
      first = min(first, (int32_t)(v[i].y - ref));
      if (v[i].x) st += (float)v[i].x, tk += (float)(int32_t)(v[i].z - ref), cnt += 1.f;
    }
  }
  // tk holds end - ref summed over the lane's counted waves; the counts
  // turn it into end - (grid entry) below.
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) first = min(first, __shfl_xor(first, o));
  // Sum over the lanes of each group: lanes with equal (l / 4) % 8 are
  // l ^ 32 and l ^ 1, l ^ 2 (same l / 4).
  st += __shfl_xor(st, 1), tk += __shfl_xor(tk, 1), cnt += __shfl_xor(cnt, 1);
  st += __shfl_xor(st, 2), tk += __shfl_xor(tk, 2), cnt += __shfl_xor(cnt, 2);
  st += __shfl_xor(st, 32), tk += __shfl_xor(tk, 32), cnt += __shfl_xor(cnt, 32);
#pragma unroll
  for (uint32_t y = 0; y < kGroups; ++y) {
    steps[y] = __shfl(st, (int)(y * kDecodeWavesPerWG));
    ticks[y] = __shfl(tk, (int)(y * kDecodeWavesPerWG)) -
               __shfl(cnt, (int)(y * kDecodeWavesPerWG)) * (float)first;
  }
  if (lane != 0) return;
  // A launch of fewer than kMinStepsPerWave steps per wave is bound by its
  // fixed costs, and its timings say little about the XCDs' rates: the
  // shares stay as they are.
  float s_tot = 0.f;
  for (uint32_t y = 0; y < kGroups; ++y) s_tot += steps[y];
  if (s_tot < (float)(kMinStepsPerWave * W)) return;
  float w[kGroups], rate[kGroups], w_tot = 0.f, r_tot = 0.f;
  load_shares(a, nwg, w);
  for (uint32_t y = 0; y < kGroups; ++y) {
    rate[y] = steps[y] > 0.f && ticks[y] > 0.f ? steps[y] / ticks[y] : 0.f;
    if (rate[y] > 0.f) w_tot += w[y], r_tot += rate[y];
  }
  for (uint32_t y = 0; y < kGroups; ++y) {
    const float nw = rate[y] > 0.f ? 0.5f * w[y] + 0.5f * w_tot * rate[y] / r_tot : w[y];
    a.bal[y] = __float_as_uint(group_waves(nwg, y) ? fmaxf(nw, 1e-3f) : 0.f);
  }
}

// One wave per (sequence, kv head) segment combines the segment's partials
// if it was split; the extra last wave updates the shares. Lane l owns the
// E = G*D/64 contiguous outputs from l*E (at most two heads), merged 8 at a
// time over batches of 8 ranges. A partial with l = 0 is an empty slice's.
// Fused append: workgroups past the merge's write the new K/V rows to their
// slots (the stream read them from the new rows, so no read of this launch
// pair depends on these writes). Rows are D contiguous elements; 16-byte
// chunks, one per lane.
template <typename T, int D>
__device__ __forceinline__ void copy_new_rows(const AttnArgs& a, uint32_t wg, uint32_t n_wg) {
  static_assert(sizeof(T) == 2, "16-bit pools: 8 elements per 16-byte chunk");
  constexpr uint32_t kChunks = D / 8;  // per row
  constexpr uint32_t kThreads = 64 * kMergeWaves;
  const uint32_t rows = a.n_new * a.kvh;             // per tensor
  const uint64_t total = 2ull * rows * kChunks;
  if (threadIdx.x >= kThreads) return;  // workgroups of more waves (a wide merge's)
  for (uint64_t i = (uint64_t)wg * kThreads + threadIdx.x; i < total; i += (uint64_t)n_wg * kThreads) {
    const uint32_t c = (uint32_t)(i % kChunks);
    const uint64_t r2 = i / kChunks;
    const bool is_v = r2 >= rows;
    const uint32_t r = (uint32_t)(is_v ? r2 - rows : r2);
    const uint32_t t = r / a.kvh, h = r - t * a.kvh;
    const uint32_t slot = a.slots[t];
    const uint4 x = *(const uint4*)((const T*)(is_v ? a.v_new : a.k_new) + (uint64_t)r * D + 8 * c);
    if (slot < a.num_slots) {
      const uint32_t blk = slot >> a.bs_shift, off = slot & (a.block_size - 1);
      T* dst = (T*)(is_v ? a.v : a.k) + blk * a.blk_e + h * a.head_e + (uint64_t)off * a.tok_e;
      *(uint4*)(dst + 8 * c) = x;
    }
  }
}

// n <= 8 merged outputs O / L at dst: one 16-byte store when there are
// eight and dst is 16-byte aligned (output rows start 256-byte aligned),
// else one store per element.
template <typename T>
__device__ __forceinline__ void store_outputs(T* dst, uint32_t n, const float (&O)[8],
                                              const float (&L)[8]) {
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = L[j] > 0.f ? O[j] / L[j] : 0.f;
  if constexpr (sizeof(T) == 4) {
    if (n == 8 && ((uintptr_t)dst & 15) == 0) {
      ((float4*)dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
      ((float4*)dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
      return;
    }
  } else if (n == 8 && ((uintptr_t)dst & 15) == 0) {
    *(uint4*)dst = pack8<T>(v);
    return;
  }
  {
    for (uint32_t j = 0; j < n; ++j) dst[j] = from_f32<T>(v[j]);
  }
}

// WPS waves per segment: 1 (four segments per workgroup) when segments are
// many and each has a few pieces; 4 (one segment per workgroup) when they
// are few, so that each has many pieces: wave v then combines pieces r0 +
// v, r0 + v + 4, ..., 8 per round trip, and the four waves' results are
// combined through LDS.
// Workgroup `bid` of `nbid` (kMergeWaves waves); workgroups from merge_wgs
// on copy the fused append's new rows.
template <typename T, int D, bool kFuse, int WPS, bool kPad = false>
__device__ __forceinline__ void decode_merge_body(const AttnArgs& a, uint32_t nwg,
                                                  uint32_t merge_wgs, uint32_t bid,
                                                  uint32_t nbid, uint32_t ns = 1) {
  static_assert(WPS == 1 || WPS >= (int)kMergeWaves, "a wave or a workgroup per segment");
  if constexpr (kFuse) {
    if (bid >= merge_wgs) {
      copy_new_rows<T, D>(a, bid - merge_wgs, nbid - merge_wgs);
      return;
    }
  }
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t nseg = a.batch * a.kvh;
  constexpr uint32_t kSegsPerWG = WPS >= (int)kMergeWaves ? 1 : kMergeWaves / WPS;
  // Items are (segment, slice): ns slices of a segment's G x D outputs
  // (ns > 1 for wide groups, so that a lane combines at most 8 outputs in
  // one pass over the pieces).
  const uint32_t item = bid * kSegsPerWG + wave / WPS;
  const uint32_t v = wave % WPS;
  if (item == nseg * ns) {
    if (v == 0 && !a.deterministic) update_shares(a, nwg, lane);
    return;
  }
  if (item > nseg * ns) return;
  const uint32_t segi = item / ns, slice = item - segi * ns;
  const uint32_t seq = segi / a.kvh, kh = segi - seq * a.kvh;
  // One round trip: the row's extents and the segment's ranges (stale for
  // rows that are not decode rows, which return here; the same for all the
  // waves of a segment).
  const uint2 rr = *(const uint2*)(a.seg_ranges + 2 * segi);
  const uint32_t q0 = a.cu_q[seq], q1 = a.cu_q[seq + 1];
  const uint32_t k0 = a.cu_k[seq], k1 = a.cu_k[seq + 1];
  const uint32_t r0 = rr.x, r1 = rr.y;
  // One test of all six words (r0 == r1: one range held the whole segment
  // and wrote the output), so that the loads are issued together.
  const bool skip = (q1 - q0 != 1) | ((int32_t)(k1 - k0) <= 0) | (r0 >= r1) |
                    (r1 >= nwg * kDecodeWavesPerWG);
  if (skip) return;
  const uint32_t G = a.group, seg = segi;
  const uint32_t E = G * D / 64 / ns;
  const uint32_t e_lane = (slice * 64 + lane) * E;
  const uint32_t h0 = e_lane / D, h1 = (e_lane + E - 1) / D;
  // kPad: output rows are a.hd apart and elements d >= a.hd (padding) are
  // not stored; the n outputs from index e of the [G][D] partials are
  // stored one by one (they may span two heads).
  const uint32_t hd = kPad ? a.hd : (uint32_t)D;
  T* orow = (T*)a.out + ((uint64_t)q0 * a.num_heads + vhead_base(a, kh)) * hd;
  // The last part of a split group serves fewer heads: outputs past them
  // are not stored.
  const uint32_t e_end = vhead_count(a, kh) * D;
  auto store = [&](uint32_t e, uint32_t n_all, const float (&O)[8], const float (&L)[8]) {
    if (e >= e_end) return;
    const uint32_t n = min(n_all, e_end - e);
    if constexpr (kPad) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t ej = e + j, d = ej % D;
        if (j < (int)n && d < hd)
          orow[(ej / D) * hd + d] = from_f32<T>(L[j] > 0.f ? O[j] / L[j] : 0.f);
      }
    } else {
      store_outputs<T>(orow + e, n, O, L);
    }
  };
  // Up to R ranges per round trip; E is a multiple of 4 for G*D >= 256
  // (D is 64, 128 or 256), so outputs move as float4. (With a workgroup per
  // segment, 8 ranges per wave measured 0.6-2.4 us faster per call than 16
  // at B = 1-16, and 4 slower at B = 1.)
  constexpr int R = 8;
  __shared__ float cmb[WPS > 1 ? WPS : 1][3][WPS > 1 ? 64 * 8 : 1];
  for (uint32_t j0 = 0; j0 < E; j0 += 8) {
    const uint32_t n = min(8u, E - j0);
    // Running max and sum per head (a lane's eight outputs span at most two
    // heads, and all outputs of a head share them), output sums per element.
    float Mh[2] = {kNegBig, kNegBig}, Lh[2] = {0.f, 0.f}, O[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) O[j] = 0.f;
    for (uint32_t w = r0 + v; w <= r1; w += R * WPS) {
      float om[R][8], mm[R][2], ll[R][2];
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const uint32_t pc = w + u * WPS;
        const bool in = pc <= r1;
        const uint64_t sl = ((uint64_t)pc * a.kv_parts.d + seg) * G;
        const float* po = a.ws_o + sl * D + e_lane + j0;
        if (in && n == 8) {
          const float4 v0 = *(const float4*)po, v1 = *(const float4*)(po + 4);
          om[u][0] = v0.x, om[u][1] = v0.y, om[u][2] = v0.z, om[u][3] = v0.w;
          om[u][4] = v1.x, om[u][5] = v1.y, om[u][6] = v1.z, om[u][7] = v1.w;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) om[u][j] = in && j < (int)n ? po[j] : 0.f;
        }
        const float2 x0 = in ? *(const float2*)(a.ws_ml + (sl + h0) * 2) : make_float2(kNegBig, 0.f);
        const float2 x1 = in ? *(const float2*)(a.ws_ml + (sl + h1) * 2) : make_float2(kNegBig, 0.f);
        // Empty partials (l = 0) weigh nothing, whatever their m and o hold.
        mm[u][0] = x0.y > 0.f ? x0.x : kNegBig, ll[u][0] = x0.y;
        mm[u][1] = x1.y > 0.f ? x1.x : kNegBig, ll[u][1] = x1.y;
      }
      float f[2], e[R][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float Mn = Mh[h];
#pragma unroll
        for (int u = 0; u < R; ++u) Mn = fmaxf(Mn, mm[u][h]);
        f[h] = fast_exp2(Mh[h] - Mn);
        float Ln = Lh[h] * f[h];
#pragma unroll
        for (int u = 0; u < R; ++u) {
          e[u][h] = ll[u][h] > 0.f ? fast_exp2(mm[u][h] - Mn) : 0.f;
          Ln += ll[u][h] * e[u][h];
        }
        Mh[h] = Mn, Lh[h] = Ln;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int hw = e_lane + j0 + j >= (h0 + 1) * D;  // the lane's second head
        float Oj = O[j] * f[hw];
#pragma unroll
        for (int u = 0; u < R; ++u) {
          // A zero weight takes nothing from the piece's o (an empty slice's
          // slot holds whatever an earlier call left there).
          Oj += e[u][hw] != 0.f ? om[u][j] * e[u][hw] : 0.f;
        }
        O[j] = Oj;
      }
    }
    float M[8], L[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int hw = e_lane + j0 + j >= (h0 + 1) * D;
      M[j] = Mh[hw], L[j] = Lh[hw];
    }
    if constexpr (WPS > 1) {
      // The segment's waves hand their (M, L, O) to wave 0 through LDS, in
      // wave order, so the combination order is fixed.
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        cmb[v][0][lane * 8 + j] = M[j];
        cmb[v][1][lane * 8 + j] = L[j];
        cmb[v][2][lane * 8 + j] = O[j];
      }
      __syncthreads();
      if (v == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float Mn = M[j];
#pragma unroll
          for (int x = 1; x < WPS; ++x) Mn = fmaxf(Mn, cmb[x][0][lane * 8 + j]);
          float Lj = 0.f, Oj = 0.f;
#pragma unroll
          for (int x = 0; x < WPS; ++x) {
            const float f = fast_exp2(cmb[x][0][lane * 8 + j] - Mn);
            Lj += cmb[x][1][lane * 8 + j] * f;
            Oj += cmb[x][2][lane * 8 + j] * f;
          }
          L[j] = Lj, O[j] = Oj;
        }
        store(e_lane + j0, n, O, L);
      }
      __syncthreads();  // cmb is reused by the next eight outputs
    } else {
      store(e_lane + j0, n, O, L);
    }
  }
}

// Workgroups of a decode's merge launch for `batch` sequences (without a
// fused append's copy); *wide: one workgroup per segment (few segments).
inline uint32_t decode_merge_wgs(uint32_t batch, uint32_t kvh, bool* wide, uint32_t ns = 1) {
  *wide = batch * kvh <= 256;
  const uint32_t items = batch * kvh * ns;
  return *wide ? items + 1 : (items + kMergeWaves) / kMergeWaves;
}

// Slices per segment in the merge: the fewest that leave a lane at most 8
// of the segment's G x D outputs (G * D / 64 per lane unsliced), a divisor
// of G * D / 64. 1 for groups of up to 4 at head_dim 128.
inline uint32_t decode_merge_slices(uint32_t group, uint32_t head_dim) {
  const uint32_t e = group * head_dim / 64;
  for (uint32_t ns = 1; ns <= e; ++ns)
    if (e % ns == 0 && e / ns <= 8) return ns;
  return 1;
}

// Workspace layout of one decode launch: the balance block (shares and
// per-wave timings; the shares carry over between launches, so the block
// leads the workspace whatever the batch), the first and last range of
// every segment, and the partials: one slot per range plus one per segment.
struct DecodeWs {
  size_t bal, ranges, ml, o, total;
};
DecodeWs decode_ws(uint32_t b, uint32_t kvh, uint32_t group, uint32_t head_dim,
                   uint32_t num_waves);
// Points a's decode workspace fields into `workspace` (layout decode_ws).
void decode_bind(AttnArgs& c, void* workspace, uint32_t head_dim);
// The decode's merge launch alone (non-fused), after a stream of nwg
// workgroups that ran inside another launch.
void launch_decode_merge(const AttnArgs& c, uint32_t nwg, uint32_t head_dim, bool bf16,
                         hipStream_t s);

}  // namespace vk
