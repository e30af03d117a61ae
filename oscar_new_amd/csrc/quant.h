// Clip + INT2 quantize + pack of one 256-element vector by one wavefront, shared by the
// store_int2 entry point and the fused pre-attention kernel.
//
// Reference: oscar_ascend/kernels.py:69-137 (`_clip_vec`, `_store_vec`). Numerics follow the
// reference test oracle (tests/oracle.py:6-21) bit for bit:
//   threshold  = torch.quantile(|x|, ratio): rank = f32(ratio)*255 (fp32),
//                a/b = ascending order statistics floor/ceil(rank), fma(w, b - a, a);
//   zero       = fp16(min x); scale = fp16(max((max - min) / 3, 2^-14));
//   code       = clamp(trunc((x - zero) / scale + 0.5), 0, 3)   (IEEE fp32, no contraction).
// Lane l owns elements 4l..4l+3, i.e. exactly packed byte l.
#pragma once

#include "common.h"

namespace oscar {

// Every function below evaluates its float arithmetic without contraction (each operation
// rounded on its own, as numpy and torch do on the CPU).

// BASELINE `search` clip factors: f32(0.6 + 0.4*i/7), evaluated in double then rounded.
__device__ __forceinline__ float search_factor(int i) {
  switch (i) {
    case 0: return static_cast<float>(0.6 + 0.4 * 0 / 7.0);
    case 1: return static_cast<float>(0.6 + 0.4 * 1 / 7.0);
    case 2: return static_cast<float>(0.6 + 0.4 * 2 / 7.0);
    case 3: return static_cast<float>(0.6 + 0.4 * 3 / 7.0);
    case 4: return static_cast<float>(0.6 + 0.4 * 4 / 7.0);
    case 5: return static_cast<float>(0.6 + 0.4 * 5 / 7.0);
    case 6: return static_cast<float>(0.6 + 0.4 * 6 / 7.0);
    default: return static_cast<float>(0.6 + 0.4 * 7 / 7.0);
  }
}

__device__ __forceinline__ int wave_count_ge(const uint32_t key[4], uint32_t t) {
  return __popcll(__ballot(key[0] >= t)) + __popcll(__ballot(key[1] >= t)) +
         __popcll(__ballot(key[2] >= t)) + __popcll(__ballot(key[3] >= t));
}
__device__ __forceinline__ int wave_count_gt(const uint32_t key[4], uint32_t t) {
  return __popcll(__ballot(key[0] > t)) + __popcll(__ballot(key[1] > t)) +
         __popcll(__ballot(key[2] > t)) + __popcll(__ballot(key[3] > t));
}

// torch.quantile(|x|, ratio) over the wavefront's 256 values. Keys are the bit patterns
// of |x| (monotone for non-negative floats); inputs come from bf16, so the low 16 bits of
// every key are zero and the order statistic is found by a 15-bit greedy search.
__device__ __forceinline__ float percentile_threshold(const float x[4], float ratio) {
#pragma clang fp contract(off)
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = __float_as_uint(x[i]) & 0x7fffffffu;
  const float rank = ratio * 255.0f;
  const int lo_idx = static_cast<int>(floorf(rank));
  const int hi_idx = static_cast<int>(ceilf(rank));
  const float weight = rank - static_cast<float>(lo_idx);
  // a = ascending order statistic lo_idx: the largest t with count(key >= t) >= 256 - lo_idx.
  const int need = kHeadDim - lo_idx;
  uint32_t t = 0;
  for (int bit = 30; bit >= 16; --bit) {
    const uint32_t cand = t | (1u << bit);
    if (wave_count_ge(key, cand) >= need) t = cand;
  }
  const float a = __uint_as_float(t);
  float b = a;
  if (hi_idx != lo_idx && wave_count_gt(key, t) >= kHeadDim - hi_idx) {
    float m = __uint_as_float(0x7f800000u);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (key[i] > t) m = fminf(m, __uint_as_float(key[i]));
    b = wave_min(m);
  }
  return __fmaf_rn(weight, b - a, a);
}

struct Quantized {
  uint32_t byte;   // this lane's packed byte
  uint32_t scale;  // fp16 bits
  uint32_t zero;   // fp16 bits
  float sf, zf;
  int code[4];
};

__device__ __forceinline__ Quantized quantize_clipped(const float xc[4]) {
#pragma clang fp contract(off)
  Quantized q;
  const float mn = wave_min(fminf(fminf(xc[0], xc[1]), fminf(xc[2], xc[3])));
  const float mx = wave_max(fmaxf(fmaxf(xc[0], xc[1]), fmaxf(xc[2], xc[3])));
  float spread = (mx - mn) / 3.0f;
  spread = spread < 6.103515625e-05f ? 6.103515625e-05f : spread;
  q.zero = float_to_f16_bits(mn);
  q.scale = float_to_f16_bits(spread);
  q.zf = f16_bits_to_float(q.zero);
  q.sf = f16_bits_to_float(q.scale);
  q.byte = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = (xc[i] - q.zf) / q.sf + 0.5f;
    int c = static_cast<int>(v);  // truncation toward zero, as torch .to(int32)
    c = c < 0 ? 0 : (c > 3 ? 3 : c);
    q.code[i] = c;
    q.byte |= static_cast<uint32_t>(c) << (2 * i);
  }
  return q;
}

__device__ __forceinline__ void clamp4(const float x[4], float thr, float out[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = fminf(fmaxf(x[i], -thr), thr);
}

// Quantize one vector and write codes + scale + zero (68 bytes) at `dst`.
__device__ __forceinline__ void quantize_store(const float x[4], int mode, float ratio, float factor,
                               uint8_t* dst) {
#pragma clang fp contract(off)
  float xc[4];
  const int lane = threadIdx.x & 63;
  if (mode == OSCAR_CLIP_FACTOR) {
    const float maxabs =
        wave_max(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
    clamp4(x, maxabs * factor, xc);
  } else if (mode == OSCAR_CLIP_SEARCH) {
    const float maxabs =
        wave_max(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
    float best_err = 0.f;
    int best = 0;
    for (int i = 0; i < 8; ++i) {
      float xi[4];
      clamp4(x, maxabs * search_factor(i), xi);
      const Quantized q = quantize_clipped(xi);
      float sq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dec = static_cast<float>(q.code[e]) * q.sf + q.zf;
        const float err = x[e] - dec;
        sq[e] = err * err;
      }
      const float err = wave_tree_sum((sq[0] + sq[1]) + (sq[2] + sq[3]));
      if (i == 0 || err < best_err) {
        best_err = err;
        best = i;
      }
    }
    clamp4(x, maxabs * search_factor(best), xc);
  } else if (ratio != 0.0f) {
    clamp4(x, percentile_threshold(x, ratio), xc);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) xc[i] = x[i];
  }
  const Quantized q = quantize_clipped(xc);
  // Gather the four bytes of packed dword (lane & 15) and store 16 dwords + scale/zero.
  const int src = (lane & 15) * 4;
  const uint32_t b0 = __shfl(q.byte, src, kWave), b1 = __shfl(q.byte, src + 1, kWave);
  const uint32_t b2 = __shfl(q.byte, src + 2, kWave), b3 = __shfl(q.byte, src + 3, kWave);
  if (lane < 16) {
    reinterpret_cast<uint32_t*>(dst)[lane] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
  } else if (lane == 16) {
    reinterpret_cast<uint32_t*>(dst)[16] = q.scale | (q.zero << 16);
  }
}

}  // namespace oscar
