// HBM ceiling probes for the benchmark (libvapi_probe.so, not part of the
// product library): what this GPU's memory system delivers for the access
// patterns of the paged-KV kernels, measured in the same run as the kernels
// they bound.
//
//  * vapi_probe_read:       sequential read of a buffer (every byte once).
//  * vapi_probe_read_tiles: reads of `tile_bytes` runs at given tile indices
//                           (the decode's 4 KiB K or V tile of one (block,
//                           head), or an 8 KiB run).
//  * vapi_probe_copy:       sequential device-to-device copy, one 16-byte
//                           chunk per thread, 64 threads per workgroup.
//  * vapi_probe_copy_runs:  copies of `run_bytes` runs between given run
//                           indices (the block copy's 16 KiB (block, layer,
//                           K or V) run).
//
// Each probe comes in two forms: ordinary loads and stores, and streaming
// (non-temporal) ones, which the paged-KV kernels use for data they touch
// once. Each lane moves 16-byte chunks with all of its loads issued before any use;
// reads fold their data into one word per workgroup so they cannot be
// dropped. Grids are large (>> 256 workgroups) and one-shot.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // 16-byte loads in flight per lane

template <bool NT>
__device__ __forceinline__ uint4 ld(const uint4* p) {
  if constexpr (NT) return vk::load_stream(p);
  else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(uint4* p, uint4 v) {
  if constexpr (NT) vk::store_stream(p, v);
  else *p = v;
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void probe_read_kernel(const uint4* __restrict__ src,
                                                              uint64_t n16,
                                                              uint32_t* __restrict__ sink) {
  const uint64_t base = (uint64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x;
  uint4 v[kUnroll];
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) {
    const uint64_t j = base + (uint64_t)i * kThreads;
    v[i] = j < n16 ? ld<NT>(src + j) : make_uint4(0, 0, 0, 0);
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  // A data-dependent store no compiler can prove dead; almost never taken.
  if (x == 0x9E3779B9u) sink[blockIdx.x & 1023] = x;
}

// One wave per tile: tile_bytes / 1024 loads of 16 B per lane.
template <int LOADS, bool NT>
__global__ __launch_bounds__(kThreads) void probe_tiles_kernel(const char* __restrict__ base,
                                                               const uint32_t* __restrict__ ids,
                                                               uint32_t n_tiles,
                                                               uint32_t* __restrict__ sink) {
  const uint32_t wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  if (wave >= n_tiles) return;
  const uint4* t = (const uint4*)(base + (uint64_t)ids[wave] * (LOADS * 1024u));
  uint4 v[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) v[i] = ld<NT>(t + i * 64 + lane);
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (x == 0x9E3779B9u) sink[wave & 1023] = x;
}

// Sequential copy, one 16-byte chunk per thread in workgroups of 64: the
// fastest shape measured for a 2 GiB device copy (streaming loads and
// stores: 6.68 TB/s read + written, against 6.46 with 256 threads and 5.90
// with 256 threads of four chunks; 1,024 threads 6.20; hipMemcpyAsync 4.8).
constexpr int kCopyThreads = 64;
template <bool NT>
__global__ __launch_bounds__(kCopyThreads) void probe_copy_kernel(uint4* __restrict__ dst,
                                                                  const uint4* __restrict__ src,
                                                                  uint64_t n16) {
  const uint64_t j = (uint64_t)blockIdx.x * kCopyThreads + threadIdx.x;
  if (j < n16) st<NT>(dst + j, ld<NT>(src + j));
}

// One workgroup per 16 KiB piece of a run (runs of `pieces` pieces):
// 16 KiB / 4096 chunks of 16 B per thread.
template <int ITEMS, bool NT>
__global__ __launch_bounds__(kThreads) void probe_runs_kernel(char* __restrict__ base,
                                                              const uint32_t* __restrict__ pairs,
                                                              uint32_t n_runs, uint32_t pieces) {
  const uint32_t r = blockIdx.x / pieces, pc = blockIdx.x % pieces;
  if (r >= n_runs) return;
  constexpr uint64_t kPiece = ITEMS * kThreads * 16ull;
  const uint64_t run = kPiece * pieces;
  const uint4* s = (const uint4*)(base + (uint64_t)pairs[2 * r] * run + pc * kPiece);
  uint4* d = (uint4*)(base + (uint64_t)pairs[2 * r + 1] * run + pc * kPiece);
  uint4 v[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) v[i] = ld<NT>(s + i * kThreads + threadIdx.x);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) st<NT>(d + i * kThreads + threadIdx.x, v[i]);
}

}  // namespace

extern "C" {

// Every probe takes `streaming`: 0 for ordinary loads and stores, 1 for
// non-temporal ones.

// Sequential read of `bytes` (a multiple of 16) at src. sink: device
// u32[1024] (written only by a sentinel the data never hits).
int vapi_probe_read(const void* src, uint64_t bytes, void* sink, uint32_t streaming,
                    hipStream_t stream) {
  const uint64_t n16 = bytes / 16;
  const uint64_t grid = (n16 + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  if (streaming)
    hipLaunchKernelGGL(probe_read_kernel<true>, dim3((uint32_t)grid), dim3(kThreads), 0, stream,
                       (const uint4*)src, n16, (uint32_t*)sink);
  else
    hipLaunchKernelGGL(probe_read_kernel<false>, dim3((uint32_t)grid), dim3(kThreads), 0, stream,
                       (const uint4*)src, n16, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Reads of n_tiles runs of tile_bytes (4096 or 8192) at base + ids[i] *
// tile_bytes (ids: device u32[n_tiles]).
int vapi_probe_read_tiles(const void* base, const uint32_t* ids, uint32_t n_tiles,
                          uint32_t tile_bytes, void* sink, uint32_t streaming,
                          hipStream_t stream) {
  const uint32_t grid = (n_tiles + kThreads / 64 - 1) / (kThreads / 64);
#define VK_TILES(L, NT)                                                                   \
  hipLaunchKernelGGL((probe_tiles_kernel<L, NT>), dim3(grid), dim3(kThreads), 0, stream, \
                     (const char*)base, ids, n_tiles, (uint32_t*)sink)
  if (tile_bytes == 4096 && streaming)
    VK_TILES(4, true);
  else if (tile_bytes == 4096)
    VK_TILES(4, false);
  else if (tile_bytes == 8192 && streaming)
    VK_TILES(8, true);
  else if (tile_bytes == 8192)
    VK_TILES(8, false);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Sequential copy of `bytes` (a multiple of 16).
int vapi_probe_copy(void* dst, const void* src, uint64_t bytes, uint32_t streaming,
                    hipStream_t stream) {
  const uint64_t n16 = bytes / 16;
  const uint64_t grid = (n16 + kCopyThreads - 1) / kCopyThreads;
  if (grid > 0xFFFFFFFFull) return -1;
  if (streaming)
    hipLaunchKernelGGL(probe_copy_kernel<true>, dim3((uint32_t)grid), dim3(kCopyThreads), 0,
                       stream, (uint4*)dst, (const uint4*)src, n16);
  else
    hipLaunchKernelGGL(probe_copy_kernel<false>, dim3((uint32_t)grid), dim3(kCopyThreads), 0,
                       stream, (uint4*)dst, (const uint4*)src, n16);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Copies n_runs runs of run_bytes (a multiple of 16384) from base +
// pairs[2i] * run_bytes to base + pairs[2i + 1] * run_bytes (pairs: device
// u32[n_runs][2]), one workgroup per 16 KiB.
int vapi_probe_copy_runs(void* base, const uint32_t* pairs, uint32_t n_runs, uint32_t run_bytes,
                         uint32_t streaming, hipStream_t stream) {
  if (run_bytes == 0 || run_bytes % 16384) return -1;
  const uint32_t pieces = run_bytes / 16384;
  if ((uint64_t)n_runs * pieces >= (1ull << 31)) return -1;
  if (streaming)
    hipLaunchKernelGGL((probe_runs_kernel<4, true>), dim3(n_runs * pieces), dim3(kThreads), 0,
                       stream, (char*)base, pairs, n_runs, pieces);
  else
    hipLaunchKernelGGL((probe_runs_kernel<4, false>), dim3(n_runs * pieces), dim3(kThreads), 0,
                       stream, (char*)base, pairs, n_runs, pieces);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
