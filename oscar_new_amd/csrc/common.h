// Shared device helpers for the gfx950 OSCAR INT2 KV-cache kernels.
//
// Conventions used by every kernel in this library:
//   * bf16 tensors are passed as uint16_t bit patterns;
//   * one wavefront = 64 lanes; workgroups are 256 threads (4 wavefronts);
//   * no kernel allocates, synchronizes the host or reads anything back to it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oscar_hip.h"

namespace oscar {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kHeadDim = 256;

// ---------------------------------------------------------------- number formats

__device__ __forceinline__ float bf16_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// float -> bf16 bits with the gfx950 hardware conversion (v_cvt_pk_bf16_f32): round to
// nearest even, NaN stays NaN -- the rounding of torch's .bfloat16().
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t float_to_bf16(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

// IEEE fp16 <-> fp32 (hardware conversion, round to nearest even, subnormals kept).
__device__ __forceinline__ float f16_bits_to_float(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint32_t float_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float half_lo_to_float(uint32_t packed) {
  return f16_bits_to_float(packed & 0xffffu);
}
__device__ __forceinline__ float half_hi_to_float(uint32_t packed) {
  return f16_bits_to_float(packed >> 16);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- integer helpers

// Exact unsigned division by a runtime constant (Granlund-Montgomery round-up method).
struct FastDiv {
  uint32_t divisor;
  uint32_t mul;
  uint32_t shift;  // ceil(log2(divisor)); 0 means divisor == 1
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0u, 0u};
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  f.shift = l;
  if (l) f.mul = static_cast<uint32_t>(((1ull << 32) * ((1ull << l) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fastdiv(uint32_t n, FastDiv f) {
  if (f.shift == 0) return n;
  uint32_t t = __umulhi(n, f.mul);
  return (t + ((n - t) >> 1)) >> (f.shift - 1);
}

__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------- wave reductions

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m, kWave));
  return v;
}
// Butterfly sum: every lane ends with the pairwise tree sum whose level k adds lane blocks
// (2j, 2j+1) of size 2^k, i.e. the canonical left-to-right pairwise order.
__device__ __forceinline__ float wave_tree_sum(float v) {
#pragma unroll
  for (int m = 1; m <= 32; m <<= 1) {
    float other = __shfl_xor(v, m, kWave);
    v = (threadIdx.x & m) ? other + v : v + other;
  }
  return v;
}

// DPP forms of the wavefront reductions: 16-lane rows reduce through data-parallel
// primitives (quad_perm xor 1, xor 2, row half-mirror, row mirror), then the four row results
// combine as uniform values. The sum keeps the pairwise tree of wave_tree_sum bit for bit:
// every level adds two equal-sized blocks, and a mirror partner holds the same block value as
// the xor partner once the blocks below are reduced.
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7 - i within 8 lanes
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15 - i within 16 lanes
constexpr int kDppRowRor8 = 0x128;        // lane i <- lane (i + 8) % 16 within 16 lanes

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
// Lane pairs (l, l ^ 16) and (l, l ^ 32) through v_permlane16_swap / v_permlane32_swap: both
// lanes of a pair receive the same combination (lower-numbered lane's value first).
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
               fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_min_dpp(float v) {
  v = fminf(v, dpp<kDppQuadXor1>(v));
  v = fminf(v, dpp<kDppQuadXor2>(v));
  v = fminf(v, dpp<kDppRowHalfMirror>(v));
  v = fminf(v, dpp<kDppRowMirror>(v));
  return fminf(fminf(lane_value(v, 0), lane_value(v, 16)),
               fminf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_tree_sum_dpp(float v) {
#pragma clang fp contract(off)
  v = v + dpp<kDppQuadXor1>(v);
  v = v + dpp<kDppQuadXor2>(v);
  v = v + dpp<kDppRowHalfMirror>(v);
  v = v + dpp<kDppRowMirror>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// ---------------------------------------------------------------- layout (device copy)

struct Layout {
  int64_t page_bytes;  // stripe_page_bytes
  int32_t head_dim, kv_heads, bp, bk, bk_shift, bpp;
  int32_t slot_bytes, vector_bytes, sink, recent, ring;
  FastDiv bpp_div;
  FastDiv ring_div;
  FastDiv bp_div;  // division by bp (slot -> page)
};

// Byte offset of slot `slot`, kv head `head` in the paged INT2 history: page slot / bp, token
// slot mod bp within it (layout.py:9-95 slot geometry). Slots below 2^32 take the
// multiply-shift division.
__device__ __forceinline__ int64_t slot_offset(const Layout& L, int64_t slot, int head) {
  const int64_t page = static_cast<uint64_t>(slot) < (1ull << 32)
                           ? static_cast<int64_t>(fastdiv(static_cast<uint32_t>(slot), L.bp_div))
                           : slot / L.bp;
  const int64_t within = slot - page * L.bp;
  return page * L.page_bytes + (within * L.kv_heads + head) * L.slot_bytes;
}

// Returns OSCAR_OK or an argument error code.
int make_layout(const oscar_layout* in, Layout* out);

hipStream_t as_stream(void* s);

// Device-coherent accesses for rows that one workgroup writes and another reads in the same
// launch: an agent-scope relaxed atomic store writes through to the device's point of
// coherence (the L2 of each XCD is not coherent with the others'), and the matching load reads
// from there. Pairing them with a wait for the stores and a counter atomic avoids whole-L2
// write-back / invalidate fences.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(float* p, float4 v) {
  store_coherent(p, v.x);
  store_coherent(p + 1, v.y);
  store_coherent(p + 2, v.z);
  store_coherent(p + 3, v.w);
}
// Loads of such rows through a raw buffer resource over a whole buffer (wave-uniform base,
// `bytes` < 2^32 long; reads past the end return zero; per-lane byte offsets) with the same
// device-coherent cache policy (sc1) as the stores above, 4 or 16 bytes at a time.
constexpr int32_t kBufferWord3 = 0x00020000;  // raw buffer, dword data (gfx9)
constexpr int kCoherentPolicy = 16;           // sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(bytes),
                                           kBufferWord3);
}
__device__ __forceinline__ float load_coherent(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __uint_as_float(
      __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(offset), 0, kCoherentPolicy));
}
__device__ __forceinline__ float4 load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  const u32x4 v =
      __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(offset), 0, kCoherentPolicy);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                     __uint_as_float(v[3]));
}

}  // namespace oscar
