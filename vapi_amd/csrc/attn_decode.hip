// Decode kernels (the device code is in attn_decode.hpp) and their launch.
#include "attn_decode.hpp"

namespace vk {

template <typename T, int D, bool kFuse, bool kPad = false, int DL = D / 16, bool kNt = true>
__global__ __launch_bounds__(64 * kDecodeWavesPerWG, kDecodeWGsPerCU) void paged_decode_stream(
    AttnArgs a, const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ cu_k,
    const uint32_t* __restrict__ table) {
  extern __shared__ uint32_t P[];
  decode_stream_body<T, D, kFuse, kPad, DL, kNt>(a, cu_q, cu_k, table, P, blockIdx.x,
                                                 gridDim.x);
}

// The stream launch: a group split into virtual kv heads (no fused append,
// all d tiles live) reads K/V with ordinary loads, its parts (neighbouring
// waves on one range of steps) sharing the tiles through L2 (config 2's
// batch at G = 48: 67.5 us with streaming loads, 51.5 us so; G = 71: 102.2
// and 74.0 us); every other call with streaming loads.
template <typename T, int D, bool F, bool PAD, int DL>
static void launch_stream(const AttnArgs& c, uint32_t nwg, size_t lds, hipStream_t s) {
  if constexpr (!F && DL == D / 16) {
    if (c.kv_parts.d > 1) {
      hipLaunchKernelGGL((paged_decode_stream<T, D, F, PAD, DL, false>), dim3(nwg),
                         dim3(64 * kDecodeWavesPerWG), lds, s, c, c.cu_q, c.cu_k, c.table);
      return;
    }
  }
  hipLaunchKernelGGL((paged_decode_stream<T, D, F, PAD, DL, true>), dim3(nwg),
                     dim3(64 * kDecodeWavesPerWG), lds, s, c, c.cu_q, c.cu_k, c.table);
}

// Waves per segment of a merge with a workgroup per segment: 8 for at most
// kFewSegs segments (each then has many pieces), else 4. Per call, one box:
// B = 1 x 8,192 keys 22.2 against 24.8 us with 4 (x 32,768: 38.1 against
// 41.3); B = 4 x 4,096 (32 segments) 23.8 against 22.7; 16 waves slower
// everywhere (34.3 us at B = 1 x 8,192).
constexpr uint32_t kFewSegs = 16;
constexpr uint32_t merge_threads(int wps) { return 64u * (wps > (int)kMergeWaves ? wps : kMergeWaves); }

template <typename T, int D, bool kFuse, int WPS, bool kPad = false>
__global__ __launch_bounds__(merge_threads(WPS)) void paged_decode_merge(AttnArgs a, uint32_t nwg,
                                                                      uint32_t merge_wgs,
                                                                      uint32_t ns) {
  decode_merge_body<T, D, kFuse, WPS, kPad>(a, nwg, merge_wgs, blockIdx.x, gridDim.x, ns);
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
    cache[dev] = (uint32_t)cus * kDecodeWGsPerCU * kDecodeWavesPerWG;
  }
  return cache[dev];
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// The words before the per-wave timings: the shares (words 0..7) and
// reserved words. Only these carry over between launches.
const size_t kDecodeBalanceBytes = kBalStats * sizeof(uint32_t);

DecodeWs decode_ws(uint32_t b, uint32_t kvh, uint32_t group, uint32_t head_dim,
                   uint32_t num_waves) {
  const size_t slots = (size_t)num_waves + (size_t)b * kvh;
  DecodeWs w;
  w.bal = 0;
  w.ranges = up256((kBalStats + kStatWords * (size_t)num_waves) * sizeof(uint32_t));
  w.ml = w.ranges + up256((size_t)b * kvh * 2 * sizeof(uint32_t));
  w.o = w.ml + up256(slots * group * 2 * sizeof(float));
  w.total = w.o + up256(slots * group * head_dim * sizeof(float));
  return w;
}

size_t decode_workspace_bytes(uint32_t batch, uint32_t kvh, uint32_t group, uint32_t head_dim,
                              uint32_t num_waves) {
  return decode_ws(std::min(batch, kMaxPlanSeqs), kvh, group, head_dim, num_waves).total;
}

void decode_bind(AttnArgs& c, void* workspace, uint32_t head_dim) {
  const DecodeWs w = decode_ws(c.batch, c.kvh, c.group, head_dim, c.num_waves);
  char* ws = (char*)workspace;
  c.bal = (uint32_t*)(ws + w.bal);
  c.seg_ranges = (uint32_t*)(ws + w.ranges);
  c.ws_ml = (float*)(ws + w.ml);
  c.ws_o = (float*)(ws + w.o);
}

uint32_t decode_max_plan_seqs() { return kMaxPlanSeqs; }

// The merge launch of a (non-fused) decode whose stream ran in another
// launch (the mixed step's): c is bound to its workspace, nwg the stream's
// decode workgroups.
void launch_decode_merge(const AttnArgs& c, uint32_t nwg, uint32_t head_dim, bool bf16,
                         hipStream_t s) {
  bool wide = false;
  const uint32_t merge_wgs = decode_merge_wgs(c.batch, c.kvh, &wide);
#define VK_MRG(T, DD, PAD)                                                                   \
  do {                                                                                       \
    if (wide && c.batch * c.kvh <= kFewSegs)                                                 \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, false, 8, PAD>), dim3(merge_wgs),        \
                         dim3(merge_threads(8)), 0, s, c, nwg, merge_wgs, 1u);               \
    else if (wide)                                                                           \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, false, kMergeWaves, PAD>),               \
                         dim3(merge_wgs), dim3(merge_threads(kMergeWaves)), 0, s, c, nwg,    \
                         merge_wgs, 1u);                                                     \
    else                                                                                     \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, false, 1, PAD>), dim3(merge_wgs),        \
                         dim3(64 * kMergeWaves), 0, s, c, nwg, merge_wgs, 1u);               \
  } while (0)
  // A head_dim below the kernel's D: the padded merge.
  const bool pad = c.hd != head_dim;
  if (bf16) {
    if (head_dim == 128) {
      if (pad) VK_MRG(bf16_t, 128, true);
      else VK_MRG(bf16_t, 128, false);
    } else {
      if (pad) VK_MRG(bf16_t, 64, true);
      else VK_MRG(bf16_t, 64, false);
    }
  } else {
    if (head_dim == 128) {
      if (pad) VK_MRG(f16_t, 128, true);
      else VK_MRG(f16_t, 128, false);
    } else {
      if (pad) VK_MRG(f16_t, 64, true);
      else VK_MRG(f16_t, 64, false);
    }
  }
#undef VK_MRG
}

void launch_decode(AttnArgs a, void* workspace, uint32_t head_dim, uint32_t dtype,
                   hipStream_t s) {
  const bool bf16 = dtype == VAPI_KV_BF16;
  const uint32_t W = a.num_waves;
  const uint32_t nwg = W / kDecodeWavesPerWG;
  const uint32_t total = a.batch;
  for (uint32_t b0 = 0; b0 < total; b0 += kMaxPlanSeqs) {
    const uint32_t nb = std::min(kMaxPlanSeqs, total - b0);
    AttnArgs c = a;
    c.batch = nb;
    c.cu_q = a.cu_q + b0;
    c.cu_k = a.cu_k + b0;
    c.table = a.table + (uint64_t)b0 * a.max_blocks;
    decode_bind(c, workspace, head_dim);
    // Fused append: the first chunk's merge launch also writes the new rows
    // (every chunk's stream reads a row's new key from the new rows).
    const bool fuse = a.k_new != nullptr;
    // Few segments (each split over many waves): a workgroup per segment.
    bool wide = false;
    // Wide groups merge in slices of at most 8 outputs per lane: config 2's
    // batch at G = 32 (two parts of 16) 66.3 -> 58.5 us per call, G = 48
    // 51.5 -> 41.0, G = 71 74.0 -> 54.4; at head_dim 256 (G = 4, two slices)
    // 251.8 -> 248.6; config 2 itself (8 outputs per lane) unchanged.
    const uint32_t ns = decode_merge_slices(a.group, head_dim);
    const uint32_t merge_wgs = decode_merge_wgs(nb, a.kvh, &wide, ns);
    uint32_t copy_wgs = 0;
    if (fuse && b0 == 0) {
      const uint64_t chunks = 2ull * a.n_new * a.kvh * (head_dim / 8);
      copy_wgs = (uint32_t)std::min<uint64_t>((chunks + 64 * kMergeWaves - 1) / (64 * kMergeWaves), 1024);
    }
    const size_t lds = (nb + 1 + (fuse ? nb : 0)) * sizeof(uint32_t);
#define VK_DECL(T, DD, F, PAD, DL)                                                              \
  do {                                                                                          \
    launch_stream<T, DD, F, PAD, DL>(c, nwg, lds, s);                                           \
    if (wide && nb * c.kvh <= kFewSegs)                                                        \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, F, 8, PAD>), dim3(merge_wgs + copy_wgs),    \
                         dim3(merge_threads(8)), 0, s, c, nwg, merge_wgs, ns);                  \
    else if (wide)                                                                              \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, F, kMergeWaves, PAD>),                      \
                         dim3(merge_wgs + copy_wgs), dim3(merge_threads(kMergeWaves)), 0, s, c, \
                         nwg, merge_wgs, ns);                                                   \
    else                                                                                        \
      hipLaunchKernelGGL((paged_decode_merge<T, DD, F, 1, PAD>), dim3(merge_wgs + copy_wgs),    \
                         dim3(64 * kMergeWaves), 0, s, c, nwg, merge_wgs, ns);                  \
  } while (0)
#define VK_DECP(T, DD, F, PAD) VK_DECL(T, DD, F, PAD, DD / 16)
#define VK_DEC(T, DD, F) VK_DECP(T, DD, F, false)
    // A padded head_dim: the stream variant that loads and multiplies only
    // the K chunks holding it, where there is one (64: 32 columns; 128: 80
    // or 96; 256: 160 or 192).
    const uint32_t live = (a.hd + 15) / 16;
#define VK_DEC_PAD(T, DD)                                    \
  do {                                                       \
    if (DD == 64 && live <= 2) VK_DECL(T, 64, false, true, 2);      \
    else if (DD == 128 && live <= 5) VK_DECL(T, 128, false, true, 5); \
    else if (DD == 128 && live <= 6) VK_DECL(T, 128, false, true, 6); \
    else if (DD == 256 && live <= 10) VK_DECL(T, 256, false, true, 10); \
    else if (DD == 256 && live <= 12) VK_DECL(T, 256, false, true, 12); \
    else VK_DECP(T, DD, false, true);                        \
  } while (0)
#define VK_DEC2(T, DD) \
  do {                 \
    if (fuse)          \
      VK_DEC(T, DD, true); \
    else               \
      VK_DEC(T, DD, false); \
  } while (0)
    if (a.hd != head_dim && dtype == VAPI_KV_F32) {  // an f32 head dim run at the next D
      if (head_dim == 128) {
        if (live <= 5) VK_DECL(float, 128, false, true, 5);
        else if (live <= 6) VK_DECL(float, 128, false, true, 6);
        else VK_DECP(float, 128, false, true);
      } else {
        if (live <= 2) VK_DECL(float, 64, false, true, 2);
        else VK_DECP(float, 64, false, true);
      }
    } else if (a.hd != head_dim) {  // a 16-bit head dim run at the next D (no fused append)
      if (head_dim == 256) {
        if (bf16) VK_DEC_PAD(bf16_t, 256);
        else VK_DEC_PAD(f16_t, 256);
      } else if (head_dim == 128) {
        if (bf16) VK_DEC_PAD(bf16_t, 128);
        else VK_DEC_PAD(f16_t, 128);
      } else {
        if (bf16) VK_DEC_PAD(bf16_t, 64);
        else VK_DEC_PAD(f16_t, 64);
      }
    } else if (dtype == VAPI_KV_F32) {  // no fused append on f32 pools
      if (head_dim == 128) VK_DEC(float, 128, false);
      else VK_DEC(float, 64, false);
    } else if (bf16) {
      if (head_dim == 256) VK_DEC2(bf16_t, 256);
      else if (head_dim == 128) VK_DEC2(bf16_t, 128);
      else VK_DEC2(bf16_t, 64);
    } else {
      if (head_dim == 256) VK_DEC2(f16_t, 256);
      else if (head_dim == 128) VK_DEC2(f16_t, 128);
      else VK_DEC2(f16_t, 64);
    }
#undef VK_DEC2
#undef VK_DEC
#undef VK_DECP
#undef VK_DECL
#undef VK_DEC_PAD
  }
}

}  // namespace vk
