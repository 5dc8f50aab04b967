// Shared helpers for the gfx950 paged KV kernels: error reporting, pool
// geometry, element types and 16-byte vector access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/vapi_kv.h"

namespace vk {

// ---- error reporting ------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

#define VK_FAIL(code, ...)        \
  do {                            \
    ::vk::set_error(__VA_ARGS__); \
    return (code);                \
  } while (0)

#define VK_HIP(call)                                                      \
  do {                                                                    \
    hipError_t e_ = (call);                                               \
    if (e_ != hipSuccess)                                                 \
      VK_FAIL(VAPI_KV_EHIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

// Check the launch that was just enqueued.
#define VK_LAUNCHED(name)                                                   \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess)                                                   \
      VK_FAIL(VAPI_KV_EHIP, "launch of %s failed: %s", name,                \
              hipGetErrorString(e_));                                       \
  } while (0)

inline size_t dtype_size(uint32_t dt) {
  switch (dt) {
    case VAPI_KV_F32: return 4;
    case VAPI_KV_F16: return 2;
    case VAPI_KV_BF16: return 2;
    default: return 0;
  }
}

// Validates a pool descriptor; returns 0 or an error code with a message.
// Validates a pool and every pool chained to it through `next`.
int check_pool(const vapi_kv_pool* p, const char* who);
constexpr uint32_t kMaxPoolChain = 4096;  // chained pools beyond the first

// ---- geometry -------------------------------------------------------------

// Element strides of one layer buffer, for either layout.
struct Geom {
  uint32_t num_blocks, block_size, kvh, d;
  uint64_t blk;   // stride between blocks (elements)
  uint64_t blk_elems;  // elements of one block of one layer buffer
  uint64_t head;  // stride between kv heads
  uint64_t tok;   // stride between token offsets within a block
};

inline Geom make_geom(const vapi_kv_pool* p) {
  Geom g;
  g.num_blocks = p->num_blocks;
  g.block_size = p->block_size;
  g.kvh = p->num_kv_heads;
  g.d = p->head_dim;
  g.blk_elems = (uint64_t)p->block_size * p->num_kv_heads * p->head_dim;
  g.blk = p->block_stride_bytes ? p->block_stride_bytes / dtype_size(p->dtype) : g.blk_elems;
  if (p->layout == VAPI_KV_LAYOUT_HND) {
    g.head = (uint64_t)p->block_size * p->head_dim;
    g.tok = p->head_dim;
  } else {
    g.head = p->head_dim;
    g.tok = (uint64_t)p->num_kv_heads * p->head_dim;
  }
  return g;
}

// Largest power-of-two chunk (16, 8, 4, 2 or 1 bytes) dividing `bytes`.
inline int chunk_bytes_for(uint64_t bytes) {
  for (int c = 16; c > 1; c >>= 1)
    if (bytes % c == 0) return c;
  return 1;
}

// Unsigned division by a runtime constant via a precomputed multiplier
// (round-up method, exact for n < 2^31 and 1 <= d < 2^31).
struct FastDiv {
  uint32_t d, mul, shift;
  FastDiv() : d(1), mul(0), shift(0) {}
  explicit FastDiv(uint32_t div) : d(div) {
    shift = 0;
    while ((1u << shift) < div) ++shift;
    uint64_t m = ((1ull << 32) * ((1ull << shift) - div)) / div + 1;
    mul = (uint32_t)m;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint32_t t = __umulhi(n, mul);
    return (t + n) >> shift;
  }
};

// ---- element types ----------------------------------------------------------

template <int N>
struct Chunk;
template <> struct Chunk<16> { using T = uint4; };
template <> struct Chunk<8> { using T = uint2; };
template <> struct Chunk<4> { using T = uint32_t; };
template <> struct Chunk<2> { using T = uint16_t; };
template <> struct Chunk<1> { using T = uint8_t; };

// A streaming (non-temporal) store: the line goes to memory without staying
// dirty in L2. For a kernel whose writes are a few times the L2's size the
// write-back of dirty lines at kernel end is a large share of its time:
// measured, a config-1 append (16 MB written) 5.44 -> 4.41 us and an
// 8,192-key gather (67 MB) 22.4 -> 9.8 us; a 4-layer append (67 MB of
// scattered rows) 5.26 -> 5.40 us per layer and the 3.76 GB block copy
// 4.9 -> 4.6 TB/s, so those keep ordinary stores.
template <typename V>
__device__ __forceinline__ void store_stream(V* p, V v) {
  if constexpr (sizeof(V) == 16) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(__builtin_bit_cast(v4, v), (v4*)p);
  } else if constexpr (sizeof(V) == 8) {
    typedef uint32_t v2 __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(__builtin_bit_cast(v2, v), (v2*)p);
  } else {
    __builtin_nontemporal_store(v, p);
  }
}

// A streaming (non-temporal) load, for data a kernel reads exactly once.
// Measured on MI355X with a read probe over 758 MB: sequential 16-byte
// loads 6.18 -> 6.93 TB/s, random 4 KiB tiles 6.04 -> 6.80 TB/s.
template <typename V>
__device__ __forceinline__ V load_stream(const V* p) {
  // The loaded words are bit-cast, not converted, into V (uint4, float4 ...).
  if constexpr (sizeof(V) == 16) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const v4 r = __builtin_nontemporal_load((const v4*)p);
    return __builtin_bit_cast(V, r);
  } else if constexpr (sizeof(V) == 8) {
    typedef uint32_t v2 __attribute__((ext_vector_type(2)));
    const v2 r = __builtin_nontemporal_load((const v2*)p);
    return __builtin_bit_cast(V, r);
  } else {
    return __builtin_nontemporal_load(p);
  }
}

// load_stream when kNt, else an ordinary (cached) load: data that other
// waves on the same XCD read again at about the same time.
template <bool kNt, typename V>
__device__ __forceinline__ V load_kv(const V* p) {
  if constexpr (kNt) return load_stream(p);
  else return *p;
}

// 16-bit float storage types as raw bits.
struct bf16_t { uint16_t x; };
struct f16_t { uint16_t x; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v.x) << 16);
}
__device__ __forceinline__ float to_f32(f16_t v) {
  return (float)__builtin_bit_cast(_Float16, v.x);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // RNE
}

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <> __device__ __forceinline__ float from_f32<float>(float f) { return f; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float f) {
  return bf16_t{f32_to_bf16_bits(f)};
}
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float f) {
  return f16_t{__builtin_bit_cast(uint16_t, (_Float16)f)};
}

// Host-side unpack of the pool descriptor into a Geom plus layer base pointers.
struct LayerPtrs {
  char* k;
  char* v;
};
inline LayerPtrs layer_ptrs(const vapi_kv_pool* p, uint32_t layer) {
  LayerPtrs r;
  r.k = (char*)p->k + (uint64_t)layer * p->layer_stride_bytes;
  r.v = (char*)p->v + (uint64_t)layer * p->layer_stride_bytes;
  return r;
}

inline hipStream_t hs(vapi_stream_t s) { return (hipStream_t)s; }

}  // namespace vk
