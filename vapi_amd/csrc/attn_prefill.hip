// Chunked-prefill paged attention on MFMA (bf16/f16, head_dim 64, 128, 256).
//
// Rows are the (query token, head) pairs of one kv head, r = j*G + h_local,
// so the G query heads of a group share every K/V byte. A workgroup owns 256
// rows (8 waves x 2 tiles of 16; one workgroup per CU, two waves per SIMD;
// at head_dim 256, 128 rows of one tile per wave)
// and walks the keys they can see in 32-key steps. Each step's K and V rows
// are copied from HBM straight into LDS by direct loads (global_load_lds:
// no staging registers, no LDS store instructions) into a ring of three
// step buffers, issued two steps ahead, and every fragment read from LDS
// feeds both row tiles of a wave. The math per row tile is the decode's
// operand scheme (S^T = K Q^T, online softmax, O^T += V^T P^T) with the
// bottom-right causal mask and left window per row, applied only on steps
// that some row of the workgroup cannot fully see. Rows with len_q < 2 are
// left to the decode kernel, unless the call launches no decode kernel (the
// caller said the batch has no decode rows): then every row is done here.
#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"
#include "attn_decode.hpp"

namespace vk {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = 64 * kPfWaves;
// ---- K and V staged by direct global-to-LDS loads --------------------------
//
// Rows keep the pool's order (key rows of D elements); each row's 16-byte
// chunks are XOR-swizzled by a function of the row index (pf_swz) so that
// the fragment reads below spread over the LDS banks. V^T fragments for O^T = V^T P^T are read
// transposed from the V rows with ds_read_b64_tr_b16: for a 16-lane group,
// lane i receives element i % 4 of the 64-bit chunk addressed by lane
// 4 j + i / 4, for j = 0..3 (measured on gfx950), so lane 4 j + q pointing
// at key row k0 + j, columns 4 q .. 4 q + 3 hands lane i the column of d
// (i) over keys k0 .. k0 + 3. A d tile of 16 columns then lands in the
// MFMA's A rows in order (d = 16 t + m), and the output O^T holds row col
// at d = 16 t + 4 g + i.
using LdsVoid = __attribute__((address_space(3))) void;


// The XOR swizzle of key row r's 16-byte chunks. D = 128 (16 chunks, a row
// is 256 bytes: every row starts at bank 0): the row index rotated left by
// one bit, a bijection on 0..15, so the 16 rows a K fragment read touches
// use 16 distinct chunk positions for any chunk, and the 8 rows of one
// half-wave of a transposing V read (rows 0..7 or 8..15, chunks 2t, 2t + 1)
// use 8 distinct chunk pairs (XOR with r alone puts rows 2m and 2m + 1 on
// the same pair). Measured 0.5-1% faster than XOR with r; the bank-conflict
// counter reads the same either way (2 cycles per transposing read).
// D = 256 (32 chunks, 512-byte rows): the same rotation, XORed into the
// low four bits of the chunk index (chunks p and p ^ 16 share banks).
// D = 64: r mod 8.
template <int D>
__device__ __forceinline__ uint32_t pf_swz(uint32_t r) {
  if constexpr (D >= 128) {
    const uint32_t x = r & 15;
    return ((x << 1) | (x >> 3)) & 15;
  } else {
    return r & (D / 8 - 1);
  }
}

// Element offset of 16-byte chunk p of key row r (0..31) in a step buffer.
template <int D>
__device__ __forceinline__ uint32_t pf_chunk(uint32_t r, uint32_t p) {
  constexpr uint32_t CPR = D / 8;  // chunks per row
  return (r * CPR + (p ^ pf_swz<D>(r))) * 8;
}

// Issues the step at s0 into buffer b with W waves (8, or 4 in the mixed
// launch): each thread moves D / (16 W) 16-byte chunks of K and as many of
// V (D = 128, 256), or with 8 waves one of K or V (D = 64: waves 0-3 K,
// waves 4-7 V), with 4 waves one of each. LDS slot t of a tensor holds the chunk its swizzled
// position names; a wave's 64 slots are contiguous, as the load writes them.
// kPad (a head_dim a.hd below D, a multiple of 8): a chunk at or past a.hd
// lies outside the key's row, so its slot is filled from the row's chunk 0
// instead (the K fragment reads zero those chunks; the V columns past a.hd
// only reach output columns that are never stored).
template <typename T, int D, int W, bool kPad = false>
__device__ __forceinline__ void pf_dma(uint16_t* kdst, uint16_t* vdst, const uint32_t* __restrict__ tab,
                                       const T* kb, const T* vb, const AttnArgs& a, int32_t s0,
                                       int32_t last, uint32_t tid, uint32_t wave) {
  constexpr uint32_t CPR = D / 8;
  using ConstU32 = const __attribute__((address_space(4))) uint32_t;
  const int32_t ts0 = min(s0, last & ~15), ts1 = min(s0 + 16, last & ~15);
  const uint32_t c0 = min((uint32_t)ts0 >> a.bs_shift, a.max_blocks - 1);
  const uint32_t c1 = min((uint32_t)ts1 >> a.bs_shift, a.max_blocks - 1);
  const uint32_t blk0 = min(((ConstU32*)tab)[c0], a.last_blk);
  const uint32_t blk1 = min(((ConstU32*)tab)[c1], a.last_blk);
  const uint64_t off0 = (uint64_t)blk0 * a.blk_e + (uint64_t)((uint32_t)ts0 & (a.block_size - 1)) * a.tok_e;
  const uint64_t off1 = (uint64_t)blk1 * a.blk_e + (uint64_t)((uint32_t)ts1 & (a.block_size - 1)) * a.tok_e;
  auto one = [&](const T* base_t, uint16_t* buf, uint32_t slot, uint32_t wslot0)
                 __attribute__((always_inline)) {
    const uint32_t r = slot / CPR, pos = slot % CPR;
    uint32_t p = pos ^ pf_swz<D>(r);
    if (kPad && 8 * p >= a.hd) p = 0;
    // A wave's slots cover 64 / CPR whole rows of one 16-key tile.
    const bool second = __builtin_amdgcn_readfirstlane(r) >= 16;
    const T* base = base_t + (second ? off1 : off0);
    const int32_t lim = last - (second ? ts1 : ts0);
    const uint32_t kk = (uint32_t)min((int32_t)(r & 15), lim);
    __builtin_amdgcn_global_load_lds((const void*)(base + kk * a.tok_e + 8 * p),
                                     (LdsVoid*)(buf + wslot0 * 8), 16, 0, 0);
  };
  if constexpr (D >= 128) {
#pragma unroll
    for (int j = 0; j < D / (16 * W); ++j) {
      one(kb, kdst, tid + 64 * W * j, 64 * wave + 64 * W * j);
      one(vb, vdst, tid + 64 * W * j, 64 * wave + 64 * W * j);
    }
  } else if constexpr (W == 8) {
    if (wave < 4) one(kb, kdst, tid, 64 * wave);
    else one(vb, vdst, tid - 256, 64 * (wave - 4));
  } else {
    one(kb, kdst, tid, 64 * wave);
    one(vb, vdst, tid, 64 * wave);
  }
}

// Waits until at most n of this wave's vector memory loads are in flight
// (s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8). The
// ring's waits count only its own direct loads, which holds while the
// kernel uses no scratch (vapi_amd/build.py refuses a build where it does).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(n | (0x7 << 4) | (0xF << 8));
}

// The workgroup barrier of the ring: this wave's loads of the next step
// have landed (the caller's wait_vmcnt), then s_barrier alone. A
// __syncthreads() would add a release fence, which waits for every load
// in flight into LDS, including the step issued two ahead.
__device__ __forceinline__ void ring_barrier() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)p;
}

// Four ds_read_b64_tr_b16 issued without waiting (results valid only after
// a later lgkm wait that names the same registers).
__device__ __forceinline__ void ds_read_tr16_issue4(uint2 (&r)[4], const uint32_t (&addr)[4]) {
  __asm__ volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %5\n\t"
      "ds_read_b64_tr_b16 %2, %6\n\t"
      "ds_read_b64_tr_b16 %3, %7"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
      : "memory");
}
// Waits until at most N LDS/scalar-memory operations are in flight; the
// registers of the batch that completes are named so that no use of them
// moves above the wait.
template <int N>
__device__ __forceinline__ void lgkm_wait(uint2 (&r)[4]) {
  __asm__ volatile("s_waitcnt lgkmcnt(%4)"
                   : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3])
                   : "n"(N)
                   : "memory");
}


// With n_split > 1 the keys a workgroup would walk are cut into n_split
// contiguous runs of steps, one workgroup each (a batch too small to fill
// the GPU with query tiles alone); each writes its rows' (m, l, o) to
// `part` and paged_prefill_merge combines them.
// Workgroup `bid` of `n_items` (W waves) of a prefill launch.
// DL: the 16-column d tiles that hold head_dim (kPad; D / 16 otherwise):
// the score MFMAs, V^T reads, PV MFMAs and stores of the tiles past them
// are left out.
template <typename T, int D, int RT, int W, bool kSplit, bool kPad = false, int DL = D / 16>
__device__ __forceinline__ void prefill_body(
    const AttnArgs& a, const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ cu_k,
    const uint32_t* __restrict__ table, uint32_t qtiles, uint32_t n_split_arg,
    float* __restrict__ part, uint32_t bid, uint32_t n_items) {
  // The unsplit launch compiles without the split's arithmetic.
  const uint32_t n_split = kSplit ? n_split_arg : 1u;
  static_assert(W == 8 || W == 4, "a step's K and V are loaded by 8 or 4 waves");
  constexpr int KC = D / 32;
  constexpr int DT = D / 16;  // 16-column d tiles
  static_assert(DL >= 1 && DL <= DT && (kPad || DL == DT), "live d tiles");
  constexpr int KCL = (DL + 1) / 2;  // live 32-column chunks of d
  constexpr int kPfRT = RT;
  constexpr uint32_t kPfRows = 16 * RT * W;
  // Direct loads per thread per step (the ring's vmcnt waits count them).
  constexpr int kLoadsPerStep = D >= 128 ? 2 * D / (16 * W) : (W == 8 ? 1 : 2);
  // The ring's three buffers per tensor are separate LDS objects, each
  // named by a compile-time index where it is used: the compiler's wait
  // insertion then knows that a direct load into one buffer cannot alias
  // the reads of another, and does not wait for the loads in flight before
  // every LDS read.
  __shared__ __attribute__((aligned(16))) uint16_t k0[32 * D], k1[32 * D], k2[32 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v0[32 * D], v1[32 * D], v2[32 * D];
  const uint32_t item = xcd_remap(bid, n_items);
  // Item order: query tile fastest, then key split, kv head, sequence (the
  // q-tiles of one split read the same K/V and run on one XCD).
  const uint32_t qt = item % qtiles, rest_s = item / qtiles;
  const uint32_t split = rest_s % n_split, rest = rest_s / n_split;
  const uint32_t kh = rest % a.kvh;
  const uint32_t seq = a.pf_seqs ? a.pf_seqs[rest / a.kvh] : rest / a.kvh;
  if (seq >= a.batch) return;
  const uint32_t q0 = cu_q[seq];
  const uint32_t len_q = cu_q[seq + 1] - q0;
  if (len_q < a.pf_min_q || len_q == 0) return;
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

  const uint32_t wg_last = min(row_base + kPfRows, nrows) - 1;
  const int32_t wg_pmin = offset + (int32_t)(row_base / G);
  const int32_t wg_pmax = offset + (int32_t)(wg_last / G);
  const int32_t klo_wg = a.wl >= 0 ? max(0, wg_pmin - a.wl) : 0;
  const int32_t khi_wg = a.wr >= 0 ? min(last, wg_pmax + a.wr) : last;
  // This workgroup's run of 32-key steps: all of them, or split's share.
  int32_t klo = klo_wg, khi = khi_wg;
  if (kSplit) {
    const int32_t first = klo_wg & ~31;
    const uint32_t steps = khi_wg >= klo_wg ? (uint32_t)(((khi_wg & ~31) - first) / 32 + 1) : 0u;
    const uint32_t a0 = split * steps / n_split, a1 = (split + 1) * steps / n_split;
    klo = max(klo_wg, first + 32 * (int32_t)a0);
    khi = min(khi_wg, first + 32 * (int32_t)a1 - 1);  // < klo when the share is empty
  }

  const uint32_t row0 = row_base + wave * 16 * kPfRT;
  uint4 qf[kPfRT][KC];
  int32_t lo[kPfRT], cnt[kPfRT];
#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    const uint32_t r = row0 + 16 * t + col;
    const uint32_t rr = r < nrows ? r : 0;
    const uint32_t j = rr / G, hl = rr % G;
    int32_t hi;
    key_range(offset + (int32_t)j, len_k, a.wl, a.wr, lo[t], hi);
    cnt[t] = max(hi - lo[t] + 1, 0);
    const T* qrow =
        (const T*)a.q + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * (kPad ? a.hd : D);
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      uint4 x = make_uint4(0, 0, 0, 0);
      if (c < KCL && (!kPad || 32 * c + 8 * g < a.hd)) {
        x = *(const uint4*)(qrow + 32 * c + 8 * g);
        x.x ^= a.q_sign, x.y ^= a.q_sign, x.z ^= a.q_sign, x.w ^= a.q_sign;
      }
      qf[t][c] = x;
    }
  }

  const uint32_t* __restrict__ tab = table + (uint64_t)seq * a.max_blocks;
  const T* kb = (const T*)a.k + kh * a.head_e;
  const T* vb = (const T*)a.v + kh * a.head_e;

  float m_run[kPfRT], l_run[kPfRT];
  floatx4 o[kPfRT][DT];
#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    m_run[t] = kNegBig;
    l_run[t] = 0.f;
#pragma unroll
    for (int k = 0; k < DT; ++k) o[t][k] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  int32_t full_lo, full_hi, unused;
  key_range(wg_pmax, len_k, a.wl, a.wr, full_lo, unused);
  key_range(wg_pmin, len_k, a.wl, a.wr, unused, full_hi);

  // Per-lane fragment offsets (elements within a step buffer).
  uint32_t k_off[2][KC];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int c = 0; c < KC; ++c) k_off[tt][c] = pf_chunk<D>(16 * tt + col, 4 * c + g);
  const uint32_t vj = col >> 2, vq = col & 3;
  uint32_t v_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v_off[t][h] = pf_chunk<D>(16 * h + 4 * g + vj, 2 * t + (vq >> 1)) + 4 * (vq & 1);

  int32_t s0_ = klo & ~31;
  const int32_t s_last = khi & ~31;
  if (!kSplit || s0_ <= khi) {  // (uniform) an empty key split issues no loads
    pf_dma<T, D, W, kPad>(k0, v0, tab, kb, vb, a, s0_, last, tid, wave);
    pf_dma<T, D, W, kPad>(k1, v1, tab, kb, vb, a, min(s0_ + 32, s_last), last, tid, wave);
    wait_vmcnt<kLoadsPerStep>();
    ring_barrier();
  }
  // Step s reads buffer s % 3 and issues step s + 2 into (s + 2) % 3.
  auto step = [&](auto cur) __attribute__((always_inline)) {
    constexpr int B = decltype(cur)::value;
    uint16_t* const kbuf = B == 0 ? k0 : B == 1 ? k1 : k2;
    uint16_t* const vbuf = B == 0 ? v0 : B == 1 ? v1 : v2;
    uint16_t* const knext = B == 0 ? k2 : B == 1 ? k0 : k1;
    uint16_t* const vnext = B == 0 ? v2 : B == 1 ? v0 : v1;
    const int32_t s0 = __builtin_amdgcn_readfirstlane(s0_);
    pf_dma<T, D, W, kPad>(knext, vnext, tab, kb, vb, a, min(s0 + 64, s_last), last, tid, wave);
    // Steps inside [full_lo, full_hi] need no mask (a uniform branch).
    const bool masked = !(s0 >= full_lo && s0 + 31 <= full_hi);
    // V^T fragments in batches of two d tiles (four transposing reads): batch
    // b + 1 is issued before batch b's MFMAs, and batch 0 right after the
    // score MFMAs, so its reads land during the softmax.
    const uint32_t vbase = lds_addr(vbuf);
    constexpr int NB = (DL + 1) / 2;
    uint2 r[NB][4];
    auto issue = [&](int b) __attribute__((always_inline)) {
      uint32_t ad[4];
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int h = 0; h < 2; ++h) ad[2 * k + h] = vbase + 2 * v_off[2 * b + k][h];
      ds_read_tr16_issue4(r[b], ad);
    };
    float sc[kPfRT][8];
    {
      floatx4 acc[kPfRT][2];
      KTile<D> kt;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int c = 0; c < KCL; ++c) {
          kt.k[tt][c] = *(const uint4*)(kbuf + k_off[tt][c]);
          if (kPad && D < 256 && 32 * c + 8 * g >= a.hd) kt.k[tt][c] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) qk_scores<T, D, KCL>(kt, qf[t], acc[t]);
#pragma unroll
      for (int t = 0; t < kPfRT; ++t) {
        const uint32_t base = (uint32_t)(s0 + 4 * (int32_t)g - lo[t]), n = (uint32_t)cnt[t];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[t][4 * tt + i] = acc[t][tt][i];
        if (masked) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (!(base + 16 * tt + i < n)) sc[t][4 * tt + i] = -INFINITY;
        }
      }
    }
    issue(0);
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
      for (int t = 0; t < kPfRT; ++t) rescale_rows<D, DL>(mx[t], o[t], m_run[t], l_run[t]);
    }
    uint4 pf[kPfRT];
#pragma unroll
    for (int t = 0; t < kPfRT; ++t) pf[t] = exp_pack<T>(sc[t], m_run[t], l_run[t], a.scale_log2);
    // Measured on config 3 (runs alternated on one box): reads waited for
    // batch by batch 969-970 TFLOP/s, batch b + 1 issued before batch b's
    // MFMAs 996-999, and batch 0 issued before the softmax 1,017-1,018
    // against 1,012 (two batches before it: 964-968; the K fragments read
    // the same way, four and four: 941-943 against 981-984).
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + 1 < NB) {
        issue(b + 1);
        lgkm_wait<4>(r[b]);
      } else {
        lgkm_wait<0>(r[b]);
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint4 vf = make_uint4(r[b][2 * k].x, r[b][2 * k].y, r[b][2 * k + 1].x,
                                    r[b][2 * k + 1].y);
        if (2 * b + k < DL) {
#pragma unroll
          for (int t = 0; t < kPfRT; ++t)
            o[t][2 * b + k] = mfma16x16x32<T>(vf, pf[t], o[t][2 * b + k]);
        }
      }
    }
    // Step s + 1's chunks (issued a step ago) are in LDS once this wave's
    // loads older than step s + 2's have landed; the barrier makes that
    // hold for every wave.
    wait_vmcnt<kLoadsPerStep>();
    ring_barrier();
    s0_ += 32;
  };
  while (true) {
    if (s0_ > khi) break;
    step(std::integral_constant<int, 0>{});
    if (s0_ > khi) break;
    step(std::integral_constant<int, 1>{});
    if (s0_ > khi) break;
    step(std::integral_constant<int, 2>{});
  }
  wait_vmcnt<0>();  // no load may land in LDS after the workgroup ends

  if constexpr (kSplit) {
    // Partials of this split (pf_part_bytes per item and split): per row
    // (m in scaled log2 units, l) as f32, then per row o / l as f32 (the
    // merge weighs it by l). An empty share leaves l = 0 and its o
    // unwritten.
    char* pb = (char*)part + ((uint64_t)(rest * qtiles + qt) * n_split + split) *
                                 pf_part_bytes(kPfRows, D);
#pragma unroll
    for (int t = 0; t < kPfRT; ++t) {
      const float lt = wave_sum_g(l_run[t]);
      const uint32_t row = wave * 16 * kPfRT + 16 * t + col;
      if (g == 0) *(float2*)(pb + (uint64_t)row * 8) = make_float2(m_run[t], lt);
      float* po = (float*)(pb + (uint64_t)kPfRows * 8) + (uint64_t)row * D;
      const float sc = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
      for (int k = 0; k < DL; ++k)
        *(float4*)(po + 16 * k + 4 * g) = make_float4(o[t][k][0] * sc, o[t][k][1] * sc,
                                                      o[t][k][2] * sc, o[t][k][3] * sc);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < kPfRT; ++t) {
    const float lt = wave_sum_g(l_run[t]);
    const uint32_t r = row0 + 16 * t + col;
    if (r >= nrows) continue;
    const uint32_t j = r / G, hl = r % G;
    T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * (kPad ? a.hd : D);
    const float sc = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
    for (int k = 0; k < DL; ++k)
      if (!kPad || 16 * k + 4 * g < a.hd)
        *(uint2*)(orow + 16 * k + 4 * g) =
          make_uint2(pack2<T>(o[t][k][0] * sc, o[t][k][1] * sc),
                     pack2<T>(o[t][k][2] * sc, o[t][k][3] * sc));
  }
}

template <typename T, int D, int RT, int OCC, bool kSplit, bool kPad, int DL = D / 16>
__global__ __launch_bounds__(kPfThreads, OCC) void paged_prefill_tiled(
    AttnArgs a, const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ cu_k,
    const uint32_t* __restrict__ table, uint32_t qtiles, uint32_t n_split_arg,
    float* __restrict__ part) {
  prefill_body<T, D, RT, kPfWaves, kSplit, kPad, DL>(a, cu_q, cu_k, table, qtiles, n_split_arg, part,
                                           blockIdx.x, gridDim.x);
}

// Combines the key splits' partials of a prefill launch: thread (row, four
// consecutive d) over the splits, in split order. Output rows are a.hd
// elements apart; with a head_dim below D the columns past it are not
// stored.
template <typename T, int D>
__device__ __forceinline__ void prefill_merge_body(const AttnArgs& a, uint32_t qtiles,
                                                   uint32_t rows_per_item, uint32_t n_split,
                                                   const float* __restrict__ part,
                                                   uint32_t bid) {
  constexpr uint32_t kTpr = D / 4;           // threads per row
  constexpr uint32_t kRpw = 256 / kTpr;      // rows per workgroup
  const uint32_t blocks_per_item = rows_per_item / kRpw;
  const uint32_t base = bid / blocks_per_item;
  const uint32_t row_in = (bid % blocks_per_item) * kRpw + threadIdx.x / kTpr;
  const uint32_t dq = (threadIdx.x % kTpr) * 4;
  const uint32_t qt = base % qtiles, rest = base / qtiles;
  const uint32_t kh = rest % a.kvh;
  const uint32_t seq = a.pf_seqs ? a.pf_seqs[rest / a.kvh] : rest / a.kvh;
  if (seq >= a.batch) return;
  const uint32_t q0 = a.cu_q[seq], len_q = a.cu_q[seq + 1] - q0;
  if (len_q < a.pf_min_q || len_q == 0) return;
  const uint32_t G = a.group;
  const uint32_t row = qt * rows_per_item + row_in;
  if (row >= len_q * G || dq >= a.hd) return;
  const uint64_t stride = pf_part_bytes(rows_per_item, D);  // per split
  const char* p0 = (const char*)part + (uint64_t)base * n_split * stride;
  const uint64_t ml_off = (uint64_t)row_in * 8;
  const uint64_t o_off = (uint64_t)rows_per_item * 8 + ((uint64_t)row_in * D + dq) * sizeof(float);
  // Eight splits per memory round trip: every (m, l) and o load of a batch
  // is issued before any is used (loading o only after testing l serialised
  // two round trips per split), then the batch joins the running (M, L, o).
  constexpr uint32_t kB = 8;
  float M = kNegBig, L = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t s0 = 0; s0 < n_split; s0 += kB) {
    float2 ml[kB];
    float4 xb[kB];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) {
      const bool in = s0 + u < n_split;
      const char* pr = p0 + (uint64_t)(in ? s0 + u : s0) * stride;
      ml[u] = *(const float2*)(pr + ml_off);
      xb[u] = *(const float4*)(pr + o_off);
      if (!in) ml[u].y = 0.f;
    }
    float Mn = M;
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u)
      if (ml[u].y > 0.f) Mn = fmaxf(Mn, ml[u].x);
    const float f = fast_exp2(M - Mn);
    L *= f;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] *= f;
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) {
      if (!(ml[u].y > 0.f)) continue;  // a share with no visible key (its o is stale)
      const float e = fast_exp2(ml[u].x - Mn);
      const float w = ml[u].y * e;  // the partial's o is o / l
      L += w;
      o[0] += xb[u].x * w, o[1] += xb[u].y * w;
      o[2] += xb[u].z * w, o[3] += xb[u].w * w;
    }
    M = Mn;
  }
  const uint32_t j = row / G, hl = row % G;
  T* orow = (T*)a.out + ((uint64_t)(q0 + j) * a.num_heads + kh * G + hl) * a.hd + dq;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if constexpr (sizeof(T) == 4)
    *(float4*)orow = make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
  else
    *(uint2*)orow = make_uint2(pack2<T>(o[0] * inv, o[1] * inv), pack2<T>(o[2] * inv, o[3] * inv));
}

template <typename T, int D>
__global__ __launch_bounds__(256) void paged_prefill_merge(AttnArgs a, uint32_t qtiles,
                                                           uint32_t rows_per_item,
                                                           uint32_t n_split,
                                                           const float* __restrict__ part) {
  prefill_merge_body<T, D>(a, qtiles, rows_per_item, n_split, part, blockIdx.x);
}

// Row tiles (16 rows each) per wave, and workgroups per CU at head_dim 128.
// At head_dim 256 a wave holds one row tile (its O and Q^T fragments, 64 +
// 32 registers, beside a 64-register K tile: two tiles would not fit the
// 256 registers of a wave at two waves per SIMD), and the ring's six
// buffers take 96 KiB of LDS.
constexpr int kPfRowTiles = 2;
constexpr int kPfRowTiles256 = 1;
constexpr int kPfOcc = 1;
// head_dim 64 fits in 128 registers: two workgroups per CU (four waves per
// SIMD) measured 1% faster than one on a config-3-shaped batch (676-678
// against 669-673 TFLOP/s), and four row tiles per wave at one workgroup
// per CU no faster (817-819 against 823-824).
constexpr int kPfOcc64 = 2;

// Query rows of one prefill workgroup.
static uint32_t pf_rows(uint32_t head_dim) {
  return 16 * (head_dim == 256 ? kPfRowTiles256 : kPfRowTiles) * kPfWaves;
}

uint64_t prefill_grid(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t max_q,
                      uint32_t head_dim) {
  const uint64_t rows = pf_rows(head_dim);
  return ((uint64_t)max_q * group + rows - 1) / rows * kvh * batch;
}

// Key splits for a launch of `base` workgroups (query tiles x kv heads x
// sequences) over at most max_k keys: enough to give every CU of a 256-CU
// GPU a workgroup (one workgroup per CU is the kernel's occupancy at
// head_dim 128), each split keeping at least 8 steps of 32 keys, at most 64.
static uint32_t pf_splits(uint64_t base, uint32_t max_k) {
  constexpr uint64_t kTarget = 256;
  if (base == 0 || base >= kTarget) return 1;
  uint64_t n = (kTarget + base - 1) / base;
  n = std::min<uint64_t>(n, std::max<uint32_t>(1u, max_k / 256));
  return (uint32_t)std::min<uint64_t>(n, 64);
}

static uint64_t pf_split_bytes(uint64_t base, uint32_t n, uint32_t head_dim,
                               uint32_t rows = 16 * kPfRowTiles * kPfWaves) {
  return n > 1 ? base * n * pf_part_bytes(rows, head_dim) : 0;
}

// At most this much workspace for the partials (fewer splits beyond).
constexpr uint64_t kPfSplitMaxBytes = 256ull << 20;

static uint32_t pf_splits_within(uint64_t base, uint32_t max_k, uint32_t head_dim,
                                 uint64_t bytes, uint32_t rows = 16 * kPfRowTiles * kPfWaves) {
  uint32_t n = pf_splits(base, max_k);
  while (n > 1 && pf_split_bytes(base, n, head_dim, rows) > std::min(bytes, kPfSplitMaxBytes))
    --n;
  return n;
}

// ---- a mixed step in one launch ---------------------------------------------
//
// A step with decode rows and prefill chunks: workgroups 0 .. nwg - 1 are
// the decode's persistent stream (one per CU, workgroup b on XCD b % 8, as
// in paged_decode_stream), the rest run the prefill with 4 waves each (128
// rows). Each kind uses at most 256 registers per lane and 64 KiB of LDS,
// so a CU holds a decode workgroup and a prefill workgroup side by side:
// the HBM-bound decode wave and the MFMA-bound prefill wave of each SIMD
// overlap instead of running one launch after the other.
constexpr int kMixRowTiles = 2;
constexpr int kMixPfWaves = 4;
constexpr uint32_t kMixRows = 16 * kMixRowTiles * kMixPfWaves;

template <typename T, int D, bool kSplit, bool kPad>
__global__ __launch_bounds__(256, 2) void paged_mixed_stream(AttnArgs a, uint32_t nwg,
                                                             uint32_t qtiles, uint32_t n_split,
                                                             float* __restrict__ part) {
  static_assert(64 * kDecodeWavesPerWG == 256 && 64 * kMixPfWaves == 256, "256 threads");
  extern __shared__ uint32_t P[];
  if (blockIdx.x < nwg)
    decode_stream_body<T, D, false, kPad>(a, a.cu_q, a.cu_k, a.table, P, blockIdx.x, nwg);
  else {
    prefill_body<T, D, kMixRowTiles, kMixPfWaves, kSplit, kPad>(a, a.cu_q, a.cu_k, a.table, qtiles,
                                                          n_split, part, blockIdx.x - nwg,
                                                          gridDim.x - nwg);
  }
}

// The mixed step's merges in one launch: the decode's (workgroups 0 ..
// merge_wgs - 1) and the prefill key split's (the rest).
template <typename T, int D, int WPS, bool kPad>
__global__ __launch_bounds__(256) void paged_mixed_merge(AttnArgs a, uint32_t nwg,
                                                         uint32_t merge_wgs, uint32_t qtiles,
                                                         uint32_t n_split,
                                                         const float* __restrict__ part) {
  if (blockIdx.x < merge_wgs)
    decode_merge_body<T, D, false, WPS, kPad>(a, nwg, merge_wgs, blockIdx.x, merge_wgs);
  else
    prefill_merge_body<T, D>(a, qtiles, kMixRows, n_split, part, blockIdx.x - merge_wgs);
}

uint64_t mixed_prefill_items(uint32_t n_seqs, uint32_t kvh, uint32_t group, uint32_t max_q) {
  return ((uint64_t)max_q * group + kMixRows - 1) / kMixRows * kvh * n_seqs;
}

void launch_mixed(const AttnArgs& a_in, void* workspace, uint32_t max_q, uint32_t max_k,
                  uint32_t head_dim, bool bf16, void* split_ws, size_t split_ws_bytes,
                  hipStream_t s) {
  AttnArgs c = a_in;
  decode_bind(c, workspace, head_dim);
  const uint32_t nwg = c.num_waves / kDecodeWavesPerWG;
  const uint32_t qtiles = (uint32_t)(((uint64_t)max_q * c.group + kMixRows - 1) / kMixRows);
  const uint64_t base = (uint64_t)qtiles * c.kvh * c.pf_seqs_n;
  // The prefill workgroups run beside the decode's, one per CU: as many key
  // splits as keep them within one round of the GPU's CUs (a second round
  // starts late and ends late: config 2's pool with 63 decode rows and a
  // 512-token chunk, 128 items, took 145 us per step with 2 splits, 151
  // with 1, 167 with 3 or 4).
  uint32_t n_split = 1;
  if (split_ws && !c.deterministic && base > 0 && base < nwg) {
    n_split = std::min<uint32_t>((uint32_t)(nwg / base), std::max<uint32_t>(1u, max_k / 256));
    n_split = std::min<uint32_t>(n_split, 64);
    while (n_split > 1 && pf_split_bytes(base, n_split, head_dim, kMixRows) >
                              std::min<uint64_t>(split_ws_bytes, kPfSplitMaxBytes))
      --n_split;
  }
  float* part = n_split > 1 ? (float*)split_ws : nullptr;
  const dim3 grid((uint32_t)(nwg + base * n_split)), block(256);
  const size_t lds = (c.batch + 1) * sizeof(uint32_t);
  bool wide = false;
  const uint32_t merge_wgs = decode_merge_wgs(c.batch, c.kvh, &wide);
#define VK_MIX(T, DD, PAD)                                                                    \
  do {                                                                                        \
    if (n_split > 1)                                                                          \
      hipLaunchKernelGGL((paged_mixed_stream<T, DD, true, PAD>), grid, block, lds, s, c, nwg, \
                         qtiles, n_split, part);                                              \
    else                                                                                      \
      hipLaunchKernelGGL((paged_mixed_stream<T, DD, false, PAD>), grid, block, lds, s, c,     \
                         nwg, qtiles, 1u, nullptr);                                           \
    if (n_split == 1) {                                                                       \
      launch_decode_merge(c, nwg, DD, bf16, s);                                               \
    } else {                                                                                  \
      const uint32_t pf_wgs = (uint32_t)(base * (kMixRows / (256 / (DD / 4))));               \
      if (wide)                                                                               \
        hipLaunchKernelGGL((paged_mixed_merge<T, DD, kMergeWaves, PAD>),                      \
                           dim3(merge_wgs + pf_wgs), dim3(256), 0, s, c, nwg, merge_wgs,      \
                           qtiles, n_split, part);                                            \
      else                                                                                    \
        hipLaunchKernelGGL((paged_mixed_merge<T, DD, 1, PAD>), dim3(merge_wgs + pf_wgs),      \
                           dim3(256), 0, s, c, nwg, merge_wgs, qtiles, n_split, part);        \
    }                                                                                         \
  } while (0)
  // A head_dim below the kernel's D (a multiple of 8): the padded kernels.
#define VK_MIX_D(T, DD)                 \
  do {                                  \
    if (c.hd != DD) VK_MIX(T, DD, true); \
    else VK_MIX(T, DD, false);          \
  } while (0)
  if (bf16) {
    if (head_dim == 128) VK_MIX_D(bf16_t, 128);
    else VK_MIX_D(bf16_t, 64);
  } else {
    if (head_dim == 128) VK_MIX_D(f16_t, 128);
    else VK_MIX_D(f16_t, 64);
  }
#undef VK_MIX_D
#undef VK_MIX
}

// The merge of paged_prefill_f32's key split: `base` items of rows_per_item
// rows, n_split partials each.
void launch_prefill_merge_f32(const AttnArgs& a, uint32_t qtiles, uint32_t rows_per_item,
                              uint32_t n_split, const float* part, uint64_t base,
                              uint32_t head_dim, hipStream_t s) {
  if (head_dim == 128)
    hipLaunchKernelGGL((paged_prefill_merge<float, 128>),
                       dim3((uint32_t)(base * (rows_per_item / (256 / 32)))), dim3(256), 0, s, a,
                       qtiles, rows_per_item, n_split, part);
  else
    hipLaunchKernelGGL((paged_prefill_merge<float, 64>),
                       dim3((uint32_t)(base * (rows_per_item / (256 / 16)))), dim3(256), 0, s, a,
                       qtiles, rows_per_item, n_split, part);
}

size_t prefill_split_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                           uint32_t max_q, uint32_t max_k) {
  if (max_q <= 1) return 0;
  const uint32_t rows = pf_rows(head_dim);
  const uint64_t base = prefill_grid(batch, kvh, group, max_q, head_dim);
  return (size_t)pf_split_bytes(base, pf_splits_within(base, max_k, head_dim, ~0ull, rows),
                                head_dim, rows);
}

void launch_prefill(const AttnArgs& a_in, uint32_t max_q, uint32_t max_k, uint32_t head_dim,
                    bool bf16, void* split_ws, size_t split_ws_bytes, hipStream_t s) {
  AttnArgs a = a_in;
  const uint32_t rows = pf_rows(head_dim);
  const uint32_t qtiles = (uint32_t)(((uint64_t)max_q * a.group + rows - 1) / rows);
  const uint64_t base = (uint64_t)qtiles * a.kvh * a.pf_seqs_n;
  // As many splits as the workspace given holds (none without one); a
  // deterministic call does not split, so its output does not depend on
  // the workspace it is given.
  const uint32_t n_split = split_ws && !a.deterministic
                               ? pf_splits_within(base, max_k, head_dim, split_ws_bytes, rows)
                               : 1;
  float* part = n_split > 1 ? (float*)split_ws : nullptr;
  const dim3 grid((uint32_t)(base * n_split)), block(kPfThreads);
#define VK_PF(T, DD, PAD, DL)                                                                    \
  do {                                                                                           \
    constexpr int occ = DD == 64 ? kPfOcc64 : kPfOcc;                                            \
    constexpr int rt = DD == 256 ? kPfRowTiles256 : kPfRowTiles;                                 \
    if (n_split > 1) {                                                                           \
      hipLaunchKernelGGL((paged_prefill_tiled<T, DD, rt, occ, true, PAD, DL>), grid, block, 0,   \
                         s, a, a.cu_q, a.cu_k, a.table, qtiles, n_split, part);                  \
      hipLaunchKernelGGL((paged_prefill_merge<T, DD>),                                           \
                         dim3((uint32_t)(base * (rows / (256 / (DD / 4))))), dim3(256), 0, s, a, \
                         qtiles, rows, n_split, part);                                           \
    } else {                                                                                     \
      hipLaunchKernelGGL((paged_prefill_tiled<T, DD, rt, occ, false, PAD, DL>), grid, block, 0,  \
                         s, a, a.cu_q, a.cu_k, a.table, qtiles, 1u, nullptr);                    \
    }                                                                                            \
  } while (0)
  // A head_dim below the kernel's D (a multiple of 8) runs the padded
  // variant: Q and K chunks past it read as zeros, output columns past it
  // are not stored, and the d tiles wholly past it are skipped where the
  // launch has a variant that stops at fewer tiles (64: 32 columns; 128:
  // 80 or 96; 256: 160 or 192).
  const uint32_t live = (a.hd + 15) / 16;
#define VK_PF_D(T, DD)                                   \
  do {                                                   \
    if (a.hd == DD) VK_PF(T, DD, false, DD / 16);        \
    else if (DD == 64 && live <= 2) VK_PF(T, 64, true, 2); \
    else if (DD == 128 && live <= 5) VK_PF(T, 128, true, 5); \
    else if (DD == 128 && live <= 6) VK_PF(T, 128, true, 6); \
    else if (DD == 256 && live <= 10) VK_PF(T, 256, true, 10); \
    else if (DD == 256 && live <= 12) VK_PF(T, 256, true, 12); \
    else VK_PF(T, DD, true, DD / 16);                    \
  } while (0)
  if (bf16) {
    if (head_dim == 256) VK_PF_D(bf16_t, 256);
    else if (head_dim == 128) VK_PF_D(bf16_t, 128);
    else VK_PF_D(bf16_t, 64);
  } else {
    if (head_dim == 256) VK_PF_D(f16_t, 256);
    else if (head_dim == 128) VK_PF_D(f16_t, 128);
    else VK_PF_D(f16_t, 64);
  }
#undef VK_PF_D
#undef VK_PF
}

}  // namespace vk
