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
// The same eight values as one FMA: fl(i * f32(0.4/7) + f32(0.6)) for i = 0..7.
constexpr float kSearchFactorStep = static_cast<float>(0.4 / 7.0);
constexpr float kSearchFactorBase = static_cast<float>(0.6);
__device__ __forceinline__ float search_factor(int i) {
  return __builtin_fmaf(static_cast<float>(i), kSearchFactorStep, kSearchFactorBase);
}

// Minimum and maximum of the wavefront's 256 finite values through order-preserving unsigned
// keys (a larger float has a larger key, -0 below +0): integer min / max need no NaN
// canonicalization, so the lane exchanges fold into them.
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t b = __float_as_uint(x);
  return b ^ (static_cast<uint32_t>(static_cast<int32_t>(b) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float(k ^ ((k >> 31) ? 0x80000000u : 0xffffffffu));
}
__device__ __forceinline__ void wave_min_max(const float x[4], float& mn, float& mx) {
  uint32_t k[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) k[i] = order_key(x[i]);
  uint32_t lo = min(min(k[0], k[1]), min(k[2], k[3]));
  uint32_t hi = max(max(k[0], k[1]), max(k[2], k[3]));
  auto lo_step = [&](auto ctrl) {
    lo = min(lo, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                     -1, static_cast<int>(lo), decltype(ctrl)::value, 0xF, 0xF, false)));
    hi = max(hi, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                     0, static_cast<int>(hi), decltype(ctrl)::value, 0xF, 0xF, false)));
  };
  lo_step(std::integral_constant<int, kDppQuadXor1>{});
  lo_step(std::integral_constant<int, kDppQuadXor2>{});
  lo_step(std::integral_constant<int, kDppRowHalfMirror>{});
  lo_step(std::integral_constant<int, kDppRowMirror>{});
  auto rl = [](uint32_t v, int l) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
  };
  lo = min(min(rl(lo, 0), rl(lo, 16)), min(rl(lo, 32), rl(lo, 48)));
  hi = max(max(rl(hi, 0), rl(hi, 16)), max(rl(hi, 32), rl(hi, 48)));
  mn = key_value(lo);
  mx = key_value(hi);
}

// Lane kLane's value in every lane through the LDS crossbar (ds_bpermute), for values that
// feed VALU operations anyway: three of them take one VALU move (the byte address) instead of
// three v_readlane. The address is materialized by asm so that the compiler does not turn a
// constant-index permute back into v_readlane.
template <int kLane>
__device__ __forceinline__ int bcast_addr() {
  int addr;
  asm("v_mov_b32 %0, %1" : "=v"(addr) : "n"(4 * kLane));
  return addr;
}
__device__ __forceinline__ float lane_bcast(float v, int addr) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(addr, __builtin_bit_cast(int, v)));
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

// x / 3 correctly rounded (fl(x / 3), as IEEE division gives it) for every finite x >= 0:
// q0 = fl(x * fl(1/3)), the residual x - 3 q0 exact in one FMA, one correction FMA. The
// identity was checked for all 2^31 non-negative finite floats on the CPU.
__device__ __forceinline__ float div3(float x) {
  constexpr float kThird = 1.0f / 3.0f;
  const float q0 = x * kThird;
  const float r = __builtin_fmaf(-q0, 3.0f, x);
  return __builtin_fmaf(r, kThird, q0);
}

// Reciprocal of a scale (an fp16 value, at least 2^-14) within one ulp (v_rcp_f32).
__device__ __forceinline__ float scale_rcp(float s) { return __builtin_amdgcn_rcpf(s); }

// Codes, scale and zero of clipped values whose minimum and maximum over the vector are mn and
// mx (tests/oracle.py:15-17): code = clamp(trunc(fl(fl(x - zero) / scale) + 0.5), 0, 3). The
// quotient is taken through a reciprocal r of the (uniform) scale within one ulp of 1 / scale:
// for y in [0.5, 3.5], fma(d, r, 0.5) differs from fl(fl(d / scale) + 0.5) by at most
// 3 (2^-23 + 2^-24) + 2^-22 < 1.2e-6, so a value of y = q + 0.5 further than 2^-16 from every
// integer truncates to the same code. If any lane has a value that close (a wider test than
// needed outside [0.5, 3.5], where the code is clamped anyway), the wavefront redoes its
// quotients with IEEE division.
// The codes of quantize_clipped for q.zf, q.sf and r = scale_rcp(q.sf).
__device__ __forceinline__ void quantize_codes(const float xc[4], float r, Quantized& q) {
#pragma clang fp contract(off)
  float y[4];
  bool near = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = __builtin_fmaf(xc[i] - q.zf, r, 0.5f);
    near |= fabsf(y[i] - rintf(y[i])) < 1.52587890625e-05f;
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
}

__device__ __forceinline__ Quantized quantize_clipped(const float xc[4], float mn, float mx) {
#pragma clang fp contract(off)
  Quantized q;
  float spread = div3(mx - mn);
  spread = spread < 6.103515625e-05f ? 6.103515625e-05f : spread;
  q.zero = float_to_f16_bits(mn);
  q.scale = float_to_f16_bits(spread);
  q.zf = f16_bits_to_float(q.zero);
  q.sf = f16_bits_to_float(q.scale);
  quantize_codes(xc, scale_rcp(q.sf), q);
  return q;
}

// Clip to [-thr, thr] (one median-of-three per value: the min/max pair's value for finite
// inputs; a zero's sign does not reach the codes, which use xc - zero).
__device__ __forceinline__ void clamp4(const float x[4], float thr, float out[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __builtin_amdgcn_fmed3f(x[i], -thr, thr);
}
__device__ __forceinline__ float clamp1(float x, float thr) { return fminf(fmaxf(x, -thr), thr); }

// Fast pass of candidate i over this lane's four values (search_best scales the sum by s^2 and
// bounds its distance to the exact MSE): u = x / s - z / s as one FMA (bz = -fl(z r), lane i's
// r and bz read through addr = bcast_addr<i>()), the code by rounding u to nearest (a tie gives
// the same |u - c| either way), clamped to [0, 3] (a clipped value's code is 0 or 3 either
// way), and the squares of u - c, the error in units of s, accumulated by FMA.
__device__ __forceinline__ float candidate_fast(const float x[4], float rc, float bzc, int addr) {
#pragma clang fp contract(off)
  const float r = lane_bcast(rc, addr), bz = lane_bcast(bzc, addr);
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float u = __builtin_fmaf(x[e], r, bz);
    const float d = u - __builtin_amdgcn_fmed3f(rintf(u), 0.0f, 3.0f);
    acc = __builtin_fmaf(d, d, acc);
  }
  return acc;
}

// Squared error of candidate i (lane i holds its threshold t, zero z, scale s and 1 / s) over
// this lane's four values, summed in pairs as the oracle's tree does: codes from the IEEE
// quotient wherever the reciprocal product lies within 2^-16 of a code boundary (the codes of
// quantize_clipped); otherwise from the reciprocal product alone.
template <bool kExact>
__device__ __forceinline__ float candidate_sq(const float x[4], float tc, float zc, float sc,
                                              float rc, int i) {
#pragma clang fp contract(off)
  static_assert(kExact, "the fast pass is candidate_fast");
  const float zf = lane_value(zc, i), sf = lane_value(sc, i), r = lane_value(rc, i);
  const float t = lane_value(tc, i);
  float xi[4], y[4];
  // Clip (one median-of-three per element: the same value as the min/max pair for the
  // finite inputs here).
#pragma unroll
  for (int e = 0; e < 4; ++e) xi[e] = __builtin_amdgcn_fmed3f(x[e], -t, t);
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf(xi[e] - zf, r, 0.5f);
  if constexpr (kExact) {
    // A wider test than quantize_clipped's (any y within 2^-16 of an integer): an estimate
    // that far from 1, 2 and 3 truncates to the code of the exact quotient, and codes can only
    // be redone exactly more often, never less.
    bool near = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) near |= fabsf(y[e] - rintf(y[e])) < 1.52587890625e-05f;
    if (__any(near)) {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = (xi[e] - zf) / sf + 0.5f;
    }
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
  return (sq[0] + sq[1]) + (sq[2] + sq[3]);
}

// The clip search's argmin (tests/oracle.py extension: the first of the 8 factors with the
// least float32 MSE, summed as a pairwise tree over the 256 values). Fast pass
// (candidate_fast): every candidate's MSE as s^2 sum (u - c)^2, the 8 sums reduced together
// (each tree level halves the candidates a lane keeps until lane l holds candidate
// (l&1)*4 + (l&2) + (l>>2&1)). Error bound (eps = 2^-24, m = max |x| >= |z|, r within one ulp
// of 1/s): u differs from q = (x - z)/s by at most 7.3 m eps / s; the exact code is that of
// fl(fl(x - z)/s) + 0.5, within (4 m / s + 4) eps of q + 0.5. Where the codes agree, s (u - c)
// and the oracle's x - fl(c s + z) differ by at most eps (10.3 m + 3 s + 2|D|), D = x - z - c s,
// |D| <= 2 m + 3 s, so the squares differ by at most eps (57.2 m^2 + 121.8 m s + 54 s^2);
// where they differ (q within (11.3 m / s + 4) eps of a code boundary) the two squares differ by
// at most eps (22.6 m s + 8 s^2). Per value at most 2^7 eps (m + s)^2, over 256 values
// 2^-9 (m + s)^2, and the two summations' rounding (at most 20 eps relative) 2^-19 MSE: each
// fast MSE lies within M = 2^-8 (m + s)^2 + 2^-18 MSE of the exact one (twice the bound;
// checked against the oracle on the CPU in tests/test_store_arith.py). If no other candidate's
// interval reaches the fast minimum's, that minimum is the exact one; otherwise the exact pass
// decides. Same result as the exact pass alone. The fast pass codes unclipped values, which
// is the clipped value's code (0 below the range, 3 above) only when the clipped range spans
// about three steps: `fast_ok` (lanes 0..7, candidate = lane) says the spread was not raised to
// 2^-14 and fp16 rounding moved the zero by at most s / 4 (then the top of the range sits at
// least 2.74 steps above the zero and the bottom at most 0.25); a candidate without it sends
// the vector to the exact pass.
__device__ __forceinline__ int search_best(const float x[4], float tc, float zc, float sc,
                                           float rc, float maxabs, bool fast_ok, int lane) {
#pragma clang fp contract(off)
  const int addr[8] = {bcast_addr<0>(), bcast_addr<1>(), bcast_addr<2>(), bcast_addr<3>(),
                       bcast_addr<4>(), bcast_addr<5>(), bcast_addr<6>(), bcast_addr<7>()};
  const float bzc = -(zc * rc);
  float part[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) part[i] = candidate_fast(x, rc, bzc, addr[i]);
  // Levels 3-5 of the tree (lane pairs 1, 2 and 4 apart), keeping half the candidates each.
  const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4;
  float q4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float keep = b0 ? part[k + 4] : part[k], give = b0 ? part[k] : part[k + 4];
    q4[k] = keep + dpp<kDppQuadXor1>(give);
  }
  float q2[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b1 ? q4[k + 2] : q4[k], give = b1 ? q4[k] : q4[k + 2];
    q2[k] = keep + dpp<kDppQuadXor2>(give);
  }
  const float keep = b2 ? q2[1] : q2[0], give = b2 ? q2[0] : q2[1];
  float v = keep + __shfl_xor(give, 4, kWave);
  // Levels 6-8: lanes 8, 16 and 32 apart.
  v = v + dpp<kDppRowRor8>(v);
  v = sum_xor16(v);
  v = sum_xor32(v);
  // Lane c (< 8) takes candidate c's sum, its margin and the decision.
  const int c = lane & 7;
  const float fv = __shfl(v, ((c >> 2) & 1) | (c & 2) | ((c & 1) << 2), kWave) * (sc * sc);
  const float ms = maxabs + sc;
  const float margin = 0.00390625f * ms * ms + 3.814697265625e-06f * fv;
  // Lanes 0..7 hold the non-negative sums: their bit patterns order like the values.
  uint32_t m8 = __float_as_uint(fv);
  m8 = min(m8, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(-1, static_cast<int>(m8),
                                                                 kDppQuadXor1, 0xF, 0xF, false)));
  m8 = min(m8, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(-1, static_cast<int>(m8),
                                                                 kDppQuadXor2, 0xF, 0xF, false)));
  m8 = min(m8, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                   -1, static_cast<int>(m8), kDppRowHalfMirror, 0xF, 0xF, false)));
  const float fmin = __uint_as_float(static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(m8), 0)));
  const uint64_t at_min = __ballot(lane < 8 && fv == fmin);
  const int best = __ffsll(static_cast<long long>(at_min)) - 1;
  if (best >= 0 && !__any(lane < 8 && !fast_ok)) {
    const float reach = lane_value(fv + margin, best);
    if (!__any(lane < 8 && lane != best && fv - margin <= reach)) return best;
  }
  // A near tie: the exact pass over the 8 candidates, in order.
  float best_err = 0.f;
  int exact = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float err = wave_tree_sum_dpp(candidate_sq<true>(x, tc, zc, sc, rc, i));
    if (i == 0 || err < best_err) {
      best_err = err;
      exact = i;
    }
  }
  return exact;
}

// Quantize one vector and write codes + scale + zero (68 bytes) at `dst` (nothing is written
// when dst is null: the caller's row is skipped, the arithmetic still runs). Clipping is
// monotone, so the extremes of the clipped vector are the clipped extremes of the vector: one
// pair of wavefront reductions serves every candidate threshold.
__device__ __forceinline__ void quantize_store(const float x[4], int mode, float ratio, float factor,
                                               uint8_t* dst) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float mn, mx;
  wave_min_max(x, mn, mx);
  const float maxabs = fmaxf(fabsf(mn), fabsf(mx));
  float thr = INFINITY;  // no clipping
  if (mode == OSCAR_CLIP_FACTOR) {
    thr = maxabs * factor;
  } else if (mode == OSCAR_CLIP_SEARCH) {
    // The uniform values of candidate i (threshold, fp16 zero and scale, 1 / scale: the
    // arithmetic of quantize_clipped) are computed once, by lane i, and read back per
    // candidate, instead of by every lane for every candidate.
    const float tc = maxabs * search_factor(lane & 7);
    const float lo = clamp1(mn, tc), hi = clamp1(mx, tc);
    const float spread_raw = div3(hi - lo);
    const float spread = spread_raw < 6.103515625e-05f ? 6.103515625e-05f : spread_raw;
    const float zc = f16_bits_to_float(float_to_f16_bits(lo));
    const float sc = f16_bits_to_float(float_to_f16_bits(spread));
    const float rc = scale_rcp(sc);
    const bool fast_ok = spread_raw >= 6.103515625e-05f && fabsf(lo - zc) <= 0.25f * sc;
    const int best = search_best(x, tc, zc, sc, rc, maxabs, fast_ok, lane);
    // The winner's threshold, zero and scale are the values its lane computed above (those of
    // quantize_clipped on the clipped extremes), so only its codes are left to compute.
    const float t = lane_value(tc, best), zf = lane_value(zc, best), sf = lane_value(sc, best);
    Quantized q;
    q.zero = float_to_f16_bits(zf);
    q.scale = float_to_f16_bits(sf);
    q.zf = zf;
    q.sf = sf;
    float xc[4];
    clamp4(x, t, xc);
    quantize_codes(xc, lane_value(rc, best), q);
    if (dst) {
      dst[lane] = static_cast<uint8_t>(q.byte);
      if (lane == 0) *reinterpret_cast<uint32_t*>(dst + 64) = q.scale | (q.zero << 16);
    }
    return;
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
  if (dst) {
    dst[lane] = static_cast<uint8_t>(q.byte);
    if (lane == 0) *reinterpret_cast<uint32_t*>(dst + 64) = q.scale | (q.zero << 16);
  }
}

}  // namespace oscar
