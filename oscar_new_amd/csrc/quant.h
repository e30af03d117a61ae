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
    b = wave_min_dpp(m);
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

// Codes, scale and zero of clipped values whose minimum and maximum over the vector are mn and
// mx (tests/oracle.py:15-17): code = clamp(trunc(fl(fl(x - zero) / scale) + 0.5), 0, 3). The
// quotient is taken through the correctly rounded reciprocal of the (uniform) scale: within
// [0.5, 3.5] it differs from the correctly rounded quotient by less than 1.2e-6, so a value of
// y = q + 0.5 further than 2^-16 from 1, 2 and 3 truncates to the same code. If any lane has a
// value that close, the wavefront redoes its quotients with IEEE division.
__device__ __forceinline__ Quantized quantize_clipped(const float xc[4], float mn, float mx) {
#pragma clang fp contract(off)
  Quantized q;
  float spread = (mx - mn) / 3.0f;
  spread = spread < 6.103515625e-05f ? 6.103515625e-05f : spread;
  q.zero = float_to_f16_bits(mn);
  q.scale = float_to_f16_bits(spread);
  q.zf = f16_bits_to_float(q.zero);
  q.sf = f16_bits_to_float(q.scale);
  const float r = 1.0f / q.sf;
  float y[4];
  bool near = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = (xc[i] - q.zf) * r + 0.5f;
    near |= y[i] > 0.5f && y[i] < 3.5f && fabsf(y[i] - rintf(y[i])) < 1.52587890625e-05f;
  }
  if (__any(near)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = (xc[i] - q.zf) / q.sf + 0.5f;
  }
  q.byte = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int c = static_cast<int>(y[i]);  // truncation toward zero, as torch .to(int32)
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
__device__ __forceinline__ float clamp1(float x, float thr) { return fminf(fmaxf(x, -thr), thr); }

// Quantize one vector and write codes + scale + zero (68 bytes) at `dst`. Clipping is
// monotone, so the extremes of the clipped vector are the clipped extremes of the vector: one
// pair of wavefront reductions serves every candidate threshold.
__device__ __forceinline__ void quantize_store(const float x[4], int mode, float ratio, float factor,
                                               uint8_t* dst) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const float mn = wave_min_dpp(fminf(fminf(x[0], x[1]), fminf(x[2], x[3])));
  const float mx = wave_max_dpp(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
  const float maxabs = fmaxf(fabsf(mn), fabsf(mx));
  float thr = INFINITY;  // no clipping
  if (mode == OSCAR_CLIP_FACTOR) {
    thr = maxabs * factor;
  } else if (mode == OSCAR_CLIP_SEARCH) {
    // The uniform values of candidate i (threshold, fp16 zero and scale, 1 / scale: the
    // arithmetic of quantize_clipped) are computed once, by lane i, and read back per
    // candidate, instead of by every lane for every candidate.
    const int ci = lane & 7;
    float fc = search_factor(0);
#pragma unroll
    for (int i = 1; i < 8; ++i) fc = ci == i ? search_factor(i) : fc;
    const float tc = maxabs * fc;
    const float lo = clamp1(mn, tc), hi = clamp1(mx, tc);
    float spread = (hi - lo) / 3.0f;
    spread = spread < 6.103515625e-05f ? 6.103515625e-05f : spread;
    const float zc = f16_bits_to_float(float_to_f16_bits(lo));
    const float sc = f16_bits_to_float(float_to_f16_bits(spread));
    const float rc = 1.0f / sc;
    float best_err = 0.f;
    int best = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float t = lane_value(tc, i), zf = lane_value(zc, i), sf = lane_value(sc, i);
      const float r = lane_value(rc, i);
      float xi[4], y[4];
      // Clip (one median-of-three per element: the same value as the min/max pair for the
      // finite inputs here).
#pragma unroll
      for (int e = 0; e < 4; ++e) xi[e] = __builtin_amdgcn_fmed3f(x[e], -t, t);
      // As quantize_clipped, with the reciprocal product fused into its + 0.5 and a wider
      // test for the IEEE fallback (any y within 2^-16 of an integer): an estimate that far
      // from 1, 2 and 3 truncates to the code of the exact quotient, and codes can only be
      // redone exactly more often, never less.
      bool near = false;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y[e] = __builtin_fmaf(xi[e] - zf, r, 0.5f);
        near |= fabsf(y[e] - rintf(y[e])) < 1.52587890625e-05f;
      }
      if (__any(near)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (xi[e] - zf) / sf + 0.5f;
      }
      float sq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // The code as a float: truncation toward zero clamped to [0, 3], the value of the
        // integer code (a -0 here decodes to the same sum: -0 * sf + zf == 0 * sf + zf).
        const float c = __builtin_amdgcn_fmed3f(truncf(y[e]), 0.0f, 3.0f);
        const float dec = c * sf + zf;
        const float err = x[e] - dec;
        sq[e] = err * err;
      }
      const float err = wave_tree_sum_dpp((sq[0] + sq[1]) + (sq[2] + sq[3]));
      if (i == 0 || err < best_err) {
        best_err = err;
        best = i;
      }
    }
    thr = maxabs * search_factor(best);
  } else if (ratio != 0.0f) {
    thr = percentile_threshold(x, ratio);
  }
  float xc[4];
  if (thr == INFINITY) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xc[i] = x[i];
  } else {
    clamp4(x, thr, xc);
  }
  const Quantized q = thr == INFINITY ? quantize_clipped(xc, mn, mx)
                                      : quantize_clipped(xc, clamp1(mn, thr), clamp1(mx, thr));
  // Lane l owns packed byte l; lane 0 also writes scale | zero (bytes 64..67, 4-aligned).
  dst[lane] = static_cast<uint8_t>(q.byte);
  if (lane == 0) *reinterpret_cast<uint32_t*>(dst + 64) = q.scale | (q.zero << 16);
}

}  // namespace oscar
