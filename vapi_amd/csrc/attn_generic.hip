// Generic VALU paged attention: any dtype (f32 included), any head_dim up
// to 256 and any GQA ratio, for the shapes the MFMA kernels do not take.
//
// One workgroup (4 waves) per 16 rows of one (sequence, kv head), a row
// being a (query token, query head of the kv head's group) pair, r = j*G +
// h. The rows share every K/V byte: 32-key tiles of K and V are staged in
// LDS as f32 by coalesced loads (consecutive threads walk a key row), then
//  * scores: thread (row, key) dots its row's Q (LDS broadcast) with the
//    key's row (LDS, rows padded by one word against bank conflicts);
//  * online softmax per row across the 32 lanes of its half-wave (shuffles),
//    in f32 with the row's running max, exactly as the CPU path orders it
//    up to summation order;
//  * PV: thread (row, d-slice) accumulates P (LDS broadcast) times V.
// Exact f32 arithmetic (no MFMA), which the f32 parity bar (max-abs 1e-5)
// needs.
//
// Long contexts are split: workgroup (sequence, kv head, row tile, chunk)
// takes keys [chunk * C, (chunk + 1) * C), C = 512 keys, or down to 64 when
// that leaves fewer than two workgroups per CU (a few short decode rows).
// When a row tile's visible keys span more than one chunk, each chunk writes
// (m, l, o) per row to the workspace and paged_attn_generic_merge combines
// them; a tile whose keys fit one chunk writes its output directly. Head
// dims 16, 32, 64, 80, 96, 128 and 256 are compiled as constants (unrolled
// dot products, 4-element staging loads, the next tile loaded while the
// current one is computed); others take the runtime-D kernel.
#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"

namespace vk {

constexpr uint32_t kGenRows = 16;   // rows per workgroup
constexpr uint32_t kGenKeys = 32;   // keys per LDS tile
constexpr uint32_t kGenThreads = 256;
constexpr uint32_t kGenChunk = 512;  // keys per workgroup, at most
constexpr uint32_t kGenMinChunk = 64;
// Dynamic LDS of the largest tile (head_dim 256: 84 KiB), past the 64 KiB
// a launch gets without asking.
constexpr size_t kGenMaxDynLds = 96 * 1024;
// The partials start past the words a decode keeps at the start of a
// workspace (its XCD shares), so one workspace serves both kinds of layer.
constexpr size_t kGenPartOffset = 256;

__host__ __device__ __forceinline__ uint32_t gen_k_stride(uint32_t d) {
  return (d & 3) ? d + 1 : d + 4;
}

// Chunks a tile with visible keys [klo, khi] spans: [c_first, c_last],
// within the launch's n_chunks. A len_k in device memory larger than the
// max_seqlen_k the launch was sized for would otherwise name chunks past
// the workspace; keys past the last launched chunk are treated as not
// visible (the attention is truncated there), and c_last < c_first when
// none of the tile's keys is covered.
__device__ __forceinline__ void tile_chunks(int32_t klo, int32_t khi, uint32_t chunk,
                                            uint32_t n_chunks, int32_t& c_first,
                                            int32_t& c_last) {
  c_first = klo / (int32_t)chunk;
  c_last = min(khi / (int32_t)chunk, (int32_t)n_chunks - 1);
}

// Four consecutive elements as f32 (16 bytes of f32, 8 of bf16 / f16).
template <typename T>
__device__ __forceinline__ float4 load4(const T* p);
template <>
__device__ __forceinline__ float4 load4<float>(const float* p) {
  return *(const float4*)p;
}
template <typename T>
__device__ __forceinline__ float4 load4(const T* p) {
  const uint2 x = *(const uint2*)p;
  const T* h = (const T*)&x;
  return make_float4(to_f32(h[0]), to_f32(h[1]), to_f32(h[2]), to_f32(h[3]));
}

// Partials of item i: (m, l) at part + i * kGenRows * (D + 2) + 2 r, then
// o at + 2 kGenRows + r * D.
template <typename T, int DT>
__global__ __launch_bounds__(kGenThreads) void paged_attn_generic(AttnArgs a, uint32_t head_dim,
                                                                  uint32_t row_tiles,
                                                                  uint32_t n_chunks,
                                                                  uint32_t chunk_keys,
                                                                  float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  // K rows padded against bank conflicts: by 4 words (keeping 16-byte
  // alignment) when head_dim is a multiple of 4, else by one.
  const uint32_t D = DT ? DT : head_dim, KS = gen_k_stride(D);
  float* ks = lds;                              // [32][KS]
  float* vs = ks + kGenKeys * KS;               // [32][D]
  float* qs = vs + kGenKeys * D;                // [16][D]
  float* ps = qs + kGenRows * D;                // [16][32]
  float* m_s = ps + kGenRows * kGenKeys;        // [16] running max
  float* l_s = m_s + kGenRows;                  // [16] running sum
  float* al_s = l_s + kGenRows;                 // [16] this tile's rescale

  const uint32_t tid = threadIdx.x;
  const uint32_t item = blockIdx.x;
  const uint32_t chunk = item % n_chunks;
  const uint32_t rt = (item / n_chunks) % row_tiles, rest = item / n_chunks / row_tiles;
  const uint32_t kh = rest % a.kvh, seq = rest / a.kvh;
  const uint32_t q0 = a.cu_q[seq], len_q = a.cu_q[seq + 1] - q0;
  const uint32_t G = a.group;
  const uint32_t nrows = len_q * G;
  const uint32_t row0 = rt * kGenRows;
  if (row0 >= nrows) return;
  const uint32_t rows = min(kGenRows, nrows - row0);
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const int32_t offset = len_k - (int32_t)len_q;

  // Keys any row of the tile can see, and this workgroup's chunk of them.
  int32_t klo, khi, unused;
  key_range(offset + (int32_t)(row0 / G), len_k, a.wl, a.wr, klo, unused);
  key_range(offset + (int32_t)((row0 + rows - 1) / G), len_k, a.wl, a.wr, unused, khi);
  int32_t c_first, c_last;
  tile_chunks(klo, khi, chunk_keys, n_chunks, c_first, c_last);
  if (khi < klo || (int32_t)chunk < c_first || (int32_t)chunk > c_last) return;
  const bool split = c_last > c_first;
  klo = max(klo, (int32_t)(chunk * chunk_keys));
  khi = min(khi, (int32_t)((chunk + 1) * chunk_keys) - 1);

  for (uint32_t i = tid; i < kGenRows * D; i += kGenThreads) {
    const uint32_t r = i / D, d = i - r * D;
    float x = 0.f;
    if (r < rows) {
      const uint32_t rr = row0 + r, j = rr / G, hl = rr - j * G;
      x = to_f32(((const T*)a.q)[((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D + d]);
    }
    qs[i] = x;
  }
  if (tid < kGenRows) m_s[tid] = kNegBig, l_s[tid] = 0.f;

  const uint32_t* table = a.table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;
  // Score phase: thread -> (row sr + 8 i, key sk), 8 rows per pass (one
  // pass when the tile has at most 8 rows). PV phase: the tile's rows
  // rounded up to R = 4, 8 or 16 share the threads, thread -> (row pr, d =
  // pd + S i) with S = 256 / R d-slices, so a decode tile (G rows) keeps
  // every thread on a real row.
  const uint32_t sk = tid & 31, sr = tid >> 5;
  const uint32_t pv_rows = rows <= 4 ? 4u : rows <= 8 ? 8u : 16u;
  const uint32_t S = kGenThreads / pv_rows;
  const uint32_t pr = tid / S, pd = tid % S;
  constexpr int kMaxDPer = DT ? (DT + 15) / 16 : 256 / 16;
  float acc[kMaxDPer];
#pragma unroll
  for (int i = 0; i < kMaxDPer; ++i) acc[i] = 0.f;

  // Staging map: thread tid moves elements i = tid + 256 u of the 32 x D
  // tile, key i / D and column i % D, stepped without divisions.
  const uint32_t k_step = kGenThreads / D, d_step = kGenThreads % D;
  const uint32_t k_first = tid / D, d_first = tid % D;
  const uint32_t n_el = (kGenKeys * D + kGenThreads - 1 - tid) / kGenThreads;  // this thread's
  // The chunk's block ids (one table read per block, not per key) and each
  // tile's per-key row offsets.
  __shared__ uint32_t blk_ids[kGenChunk];
  __shared__ uint64_t key_off[kGenKeys];
  const uint32_t col0 = (uint32_t)klo / a.block_size;
  const uint32_t n_cols = (uint32_t)khi / a.block_size - col0 + 1;
  for (uint32_t c = tid; c < n_cols; c += kGenThreads)
    blk_ids[c] = min(table[min(col0 + c, a.max_blocks - 1)], a.last_blk);
  // Constant head dims: each thread's 4-element chunks of the next tile are
  // loaded into registers while the current tile is computed (one HBM round
  // trip hidden per tile).
  constexpr bool kVec = DT > 0 && DT % 4 == 0;
  constexpr uint32_t kC4 = kVec ? kGenKeys * DT / 4 : 1;
  constexpr uint32_t kPer = (kC4 + kGenThreads - 1) / kGenThreads;
  float4 kx[kPer], vx[kPer];
  auto fetch = [&](int32_t cs) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
      const uint32_t c = tid + u * kGenThreads;
      kx[u] = vx[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      const int32_t key = cs + (int32_t)(c * 4 / D);
      if (c < kC4 && key <= khi) {
        const uint32_t d = c * 4 % D;
        const uint64_t off = (uint64_t)blk_ids[(uint32_t)key / a.block_size - col0] * a.blk_e +
                             (uint64_t)((uint32_t)key % a.block_size) * a.tok_e;
        kx[u] = load4<T>(kb + off + d);
        vx[u] = load4<T>(vb + off + d);
      }
    }
  };
  if constexpr (kVec) {
    __syncthreads();  // blk_ids
    fetch(klo);
  }
  for (int32_t c0 = klo; c0 <= khi; c0 += (int32_t)kGenKeys) {
    __syncthreads();  // the previous tile's K, V, P and key offsets are consumed
    // Stage keys c0 .. c0 + 31 (past khi: zeros, never visible).
    if constexpr (kVec) {
#pragma unroll
      for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t c = tid + u * kGenThreads;
        if (c < kC4) {
          const uint32_t key = c * 4 / DT, d = c * 4 % DT;
          *(float4*)(ks + key * KS + d) = kx[u];
          *(float4*)(vs + key * DT + d) = vx[u];
        }
      }
      __syncthreads();
      if (c0 + (int32_t)kGenKeys <= khi) fetch(c0 + (int32_t)kGenKeys);
    } else {
      if (tid < kGenKeys) {
        const int32_t key = c0 + (int32_t)tid;
        key_off[tid] = key <= khi ? (uint64_t)blk_ids[(uint32_t)key / a.block_size - col0] * a.blk_e +
                                        (uint64_t)((uint32_t)key % a.block_size) * a.tok_e
                                  : ~0ull;
      }
      __syncthreads();
      // Any head_dim: eight elements at a time, all eight loads issued
      // before their stores.
      {
        constexpr int kBatch = 8;
        uint32_t k = k_first, d = d_first;
        for (uint32_t u0 = 0; u0 < n_el; u0 += kBatch) {
          float kx1[kBatch], vx1[kBatch];
          uint32_t kk[kBatch], dd[kBatch];
#pragma unroll
          for (int u = 0; u < kBatch; ++u) {
            kk[u] = k, dd[u] = d;
            kx1[u] = 0.f, vx1[u] = 0.f;
            if (u0 + u < n_el) {
              const uint64_t off = key_off[k];
              if (off != ~0ull) {
                kx1[u] = to_f32(kb[off + d]);
                vx1[u] = to_f32(vb[off + d]);
              }
            }
            d += d_step, k += k_step;
            if (d >= D) d -= D, ++k;
          }
#pragma unroll
          for (int u = 0; u < kBatch; ++u) {
            if (u0 + u < n_el) {
              ks[kk[u] * KS + dd[u]] = kx1[u];
              vs[kk[u] * D + dd[u]] = vx1[u];
            }
          }
        }
      }
      __syncthreads();
    }
    // Scores and the online softmax, two passes of 8 rows.
#pragma unroll
    for (uint32_t pass = 0; pass < 2; ++pass) {
      if (pass == 1 && rows <= 8) break;
      const uint32_t r = sr + 8 * pass;
      const int32_t key = c0 + (int32_t)sk;
      float s = -INFINITY;
      if (r < rows) {
        int32_t lo, hi;
        key_range(offset + (int32_t)((row0 + r) / G), len_k, a.wl, a.wr, lo, hi);
        // Keys past this chunk (khi) are staged as zeros and belong to the
        // next chunk's workgroup, whatever the row's own range says.
        if (key >= lo && key <= min(hi, khi)) {
          const float* qr = qs + r * D;
          const float* kr = ks + sk * KS;
          float dot;
          if ((D & 3) == 0) {  // 16-byte LDS reads, four independent sums
            const float4* q4 = (const float4*)qr;
            const float4* k4 = (const float4*)kr;
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
            for (uint32_t d4 = 0; d4 < D / 4; ++d4) {
              const float4 qv = q4[d4], kv = k4[d4];
              s0 = __builtin_fmaf(qv.x, kv.x, s0);
              s1 = __builtin_fmaf(qv.y, kv.y, s1);
              s2 = __builtin_fmaf(qv.z, kv.z, s2);
              s3 = __builtin_fmaf(qv.w, kv.w, s3);
            }
            dot = (s0 + s1) + (s2 + s3);
          } else {
            dot = 0.f;
            for (uint32_t d = 0; d < D; ++d) dot = __builtin_fmaf(qr[d], kr[d], dot);
          }
          s = dot * a.scale;
        }
      }
      float cm = s;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o, 32));
      const float m_old = m_s[r];
      const float mn = fmaxf(m_old, cm);
      const float p = s == -INFINITY ? 0.f : __expf(s - mn);
      float cs = p;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) cs += __shfl_xor(cs, o, 32);
      ps[r * kGenKeys + sk] = p;
      if (sk == 0) {
        const float alpha = __expf(m_old - mn);
        al_s[r] = alpha;
        l_s[r] = l_s[r] * alpha + cs;
        m_s[r] = mn;
      }
    }
    __syncthreads();
    // O = O * alpha + P V.
    const float alpha = al_s[pr];
    const float* pp = ps + pr * kGenKeys;
#pragma unroll
    for (int i = 0; i < kMaxDPer; ++i) acc[i] *= alpha;
    // One copy of the loop per slice count, so that its d offsets and trip
    // count are constants.
    auto pv = [&](auto s_c) __attribute__((always_inline)) {
      constexpr uint32_t SC = decltype(s_c)::value;
      constexpr int kN = DT ? (int)((DT + SC - 1) / SC) : kMaxDPer;
      for (uint32_t k = 0; k < kGenKeys; ++k) {
        const float pk = pp[k];
        const float* vk = vs + k * D + pd;
#pragma unroll
        for (int i = 0; i < kN; ++i)
          if ((DT && DT % SC == 0) || pd + SC * i < D)
            acc[i] = __builtin_fmaf(pk, vk[SC * i], acc[i]);
      }
    };
    if (S == 64) pv(std::integral_constant<uint32_t, 64>{});
    else if (S == 32) pv(std::integral_constant<uint32_t, 32>{});
    else pv(std::integral_constant<uint32_t, 16>{});
  }
  __syncthreads();
  if (split) {
    float* pi = part + (uint64_t)item * kGenRows * (D + 2);
    if (tid < kGenRows) {
      pi[2 * tid] = m_s[tid];
      pi[2 * tid + 1] = l_s[tid];
    }
#pragma unroll
    for (int i = 0; i < kMaxDPer; ++i) {
      const uint32_t d = pd + S * i;
      if (d < D) pi[2 * kGenRows + pr * D + d] = acc[i];
    }
    return;
  }
  if (pr < rows) {
    const uint32_t rr = row0 + pr, j = rr / G, hl = rr - j * G;
    T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
    const float l = l_s[pr];
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int i = 0; i < kMaxDPer; ++i) {
      const uint32_t d = pd + S * i;
      if (d < D) orow[d] = from_f32<T>(acc[i] * inv);
    }
  }
}

// One workgroup per (sequence, kv head, row tile) whose keys were split:
// thread (row, d-slice) combines the chunks' partials.
template <typename T, int DT>
__global__ __launch_bounds__(kGenThreads) void paged_attn_generic_merge(
    AttnArgs a, uint32_t head_dim, uint32_t row_tiles, uint32_t n_chunks, uint32_t chunk_keys,
    const float* __restrict__ part) {
  const uint32_t D = DT ? DT : head_dim;
  const uint32_t tid = threadIdx.x;
  const uint32_t rt = blockIdx.x % row_tiles, rest = blockIdx.x / row_tiles;
  const uint32_t kh = rest % a.kvh, seq = rest / a.kvh;
  const uint32_t q0 = a.cu_q[seq], len_q = a.cu_q[seq + 1] - q0;
  const uint32_t G = a.group;
  const uint32_t nrows = len_q * G;
  const uint32_t row0 = rt * kGenRows;
  if (row0 >= nrows) return;
  const uint32_t rows = min(kGenRows, nrows - row0);
  const int32_t len_k = (int32_t)(a.cu_k[seq + 1] - a.cu_k[seq]);
  const int32_t offset = len_k - (int32_t)len_q;
  int32_t klo, khi, unused, c_first, c_last;
  key_range(offset + (int32_t)(row0 / G), len_k, a.wl, a.wr, klo, unused);
  key_range(offset + (int32_t)((row0 + rows - 1) / G), len_k, a.wl, a.wr, unused, khi);
  tile_chunks(klo, khi, chunk_keys, n_chunks, c_first, c_last);
  if (khi < klo || c_last <= c_first) return;
  const uint32_t pr = tid >> 4, pd = tid & 15;
  if (pr >= rows) return;
  const uint64_t base = (uint64_t)blockIdx.x * n_chunks;
  const uint64_t stride = (uint64_t)kGenRows * (D + 2);
  // Four chunks per memory round trip: every (m, l) and o load of a batch
  // is issued before any is used, then the batch joins the running (M, L,
  // o) (loading o only after testing l serialised two round trips per
  // chunk).
  constexpr int kMaxDPer = DT ? (DT + 15) / 16 : 256 / 16;
  constexpr int kB = 4;
  float M = kNegBig, L = 0.f;
  float o[kMaxDPer];
#pragma unroll
  for (int i = 0; i < kMaxDPer; ++i) o[i] = 0.f;
  for (int32_t c0 = c_first; c0 <= c_last; c0 += kB) {
    float m[kB], l[kB], x[kB][kMaxDPer];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const bool in = c0 + u <= c_last;
      const float* pc = part + (base + (in ? c0 + u : c0)) * stride;
      m[u] = pc[2 * pr];
      l[u] = in ? pc[2 * pr + 1] : 0.f;
#pragma unroll
      for (int i = 0; i < kMaxDPer; ++i) {
        const uint32_t d = pd + 16 * i;
        x[u][i] = d < D ? pc[2 * kGenRows + pr * D + d] : 0.f;
      }
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < kB; ++u)
      if (l[u] > 0.f) Mn = fmaxf(Mn, m[u]);
    const float f = __expf(M - Mn);
    L *= f;
#pragma unroll
    for (int i = 0; i < kMaxDPer; ++i) o[i] *= f;
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      if (!(l[u] > 0.f)) continue;  // a chunk no key of this row is visible in
      const float e = __expf(m[u] - Mn);
      L += l[u] * e;
#pragma unroll
      for (int i = 0; i < kMaxDPer; ++i) o[i] += x[u][i] * e;
    }
    M = Mn;
  }
  const uint32_t rr = row0 + pr, j = rr / G, hl = rr - j * G;
  T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * D;
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int i = 0; i < kMaxDPer; ++i) {
    const uint32_t d = pd + 16 * i;
    if (d < D) orow[d] = from_f32<T>(o[i] * inv);
  }
}

// Keys per workgroup: 512, halved down to 64 while that leaves fewer than
// two workgroups per CU of a 256-CU GPU (one rule for the launch and the
// workspace size).
static uint32_t gen_chunk_keys(uint64_t tiles, uint32_t max_k) {
  uint32_t c = kGenChunk;
  while (c > kGenMinChunk && tiles * (((uint64_t)max_k + c - 1) / c) < 512) c /= 2;
  return c;
}

uint64_t generic_grid(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t max_q,
                      uint32_t max_k) {
  const uint64_t row_tiles = ((uint64_t)max_q * group + kGenRows - 1) / kGenRows;
  const uint64_t tiles = row_tiles * kvh * batch;
  const uint32_t c = gen_chunk_keys(tiles, max_k);
  return tiles * std::max<uint64_t>(((uint64_t)max_k + c - 1) / c, 1);
}

size_t generic_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                               uint32_t max_q, uint32_t max_k) {
  const uint64_t row_tiles = ((uint64_t)max_q * group + kGenRows - 1) / kGenRows;
  const uint64_t tiles = row_tiles * kvh * batch;
  const uint32_t c = gen_chunk_keys(tiles, max_k);
  const uint64_t n_chunks = ((uint64_t)max_k + c - 1) / c;
  if (n_chunks <= 1) return 0;
  return kGenPartOffset + (size_t)(tiles * n_chunks * kGenRows * (head_dim + 2) * sizeof(float));
}

void launch_generic(const AttnArgs& a, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                    uint32_t dtype, void* workspace, hipStream_t s) {
  const uint32_t row_tiles = (uint32_t)(((uint64_t)max_q * a.group + kGenRows - 1) / kGenRows);
  const uint64_t tiles = (uint64_t)row_tiles * a.kvh * a.batch;
  const uint32_t chunk_keys = gen_chunk_keys(tiles, max_k);
  const uint32_t n_chunks = (uint32_t)(((uint64_t)max_k + chunk_keys - 1) / chunk_keys);
  const uint64_t n = tiles * std::max(n_chunks, 1u);
  float* part = (float*)((char*)workspace + kGenPartOffset);
  const size_t lds = ((size_t)kGenKeys * gen_k_stride(head_dim) + (size_t)kGenKeys * head_dim +
                      (size_t)kGenRows * head_dim + kGenRows * kGenKeys + 3 * kGenRows) *
                     sizeof(float);
#define VK_GEN(T, DT)                                                                        \
  do {                                                                                       \
    static bool lds_set = false;                                                             \
    if (lds > 64 * 1024 && !lds_set) {                                                       \
      if (hipFuncSetAttribute((const void*)paged_attn_generic<T, DT>,                        \
                              hipFuncAttributeMaxDynamicSharedMemorySize,                    \
                              (int)kGenMaxDynLds) == hipSuccess)                             \
        lds_set = true;                                                                      \
    }                                                                                        \
    hipLaunchKernelGGL((paged_attn_generic<T, DT>), dim3((uint32_t)n), dim3(kGenThreads), lds, \
                       s, a, head_dim, row_tiles, std::max(n_chunks, 1u), chunk_keys, part); \
    if (n_chunks > 1)                                                                        \
      hipLaunchKernelGGL((paged_attn_generic_merge<T, DT>), dim3((uint32_t)tiles),           \
                         dim3(kGenThreads), 0, s, a, head_dim, row_tiles, n_chunks,          \
                         chunk_keys, part);                                                  \
  } while (0)
#define VK_GEN_D(T)                                  \
  do {                                               \
    switch (head_dim) {                              \
      case 16: VK_GEN(T, 16); break;                 \
      case 32: VK_GEN(T, 32); break;                 \
      case 64: VK_GEN(T, 64); break;                 \
      case 80: VK_GEN(T, 80); break;                 \
      case 96: VK_GEN(T, 96); break;                 \
      case 128: VK_GEN(T, 128); break;               \
      case 256: VK_GEN(T, 256); break;               \
      default: VK_GEN(T, 0); break;                  \
    }                                                \
  } while (0)
  switch (dtype) {
    case VAPI_KV_F32: VK_GEN_D(float); break;
    case VAPI_KV_BF16: VK_GEN_D(bf16_t); break;
    default: VK_GEN_D(f16_t); break;
  }
#undef VK_GEN_D
#undef VK_GEN
}

}  // namespace vk
