// Row arithmetic of the two LSE merges, shared by the merge_splits / merge_paths entry points
// and the fused post-attention kernel so that both paths produce the same bits.
//
// Reference: oscar_ascend/kernels.py:485-527 (`_merge_splits_kernel`, `_merge_paths_kernel`).
// One wavefront per (token, query head) row; lane l owns dims 4l..4l+3.
#pragma once

#include "common.h"

namespace oscar {

constexpr float kDenFloor = 1.0e-30f;

struct SplitMerge {
  float acc[4];  // sum_s w_s P_s for this lane's dims
  float den;     // sum_s w_s
  float mx;      // max_s lse_s (-inf: no live split)
};

// kernels.py:489-503: w_s = e^{lse_s - M}, splits with lse -inf contribute nothing. `part`
// is the row's [splits][256] partials (this lane's dims), `ls` its [splits] LSEs. Padded rows
// (valid false, uniform over the wavefront) merge to nothing; their loads are issued anyway,
// since they stay inside the row's buffers, so that no load waits for the token count.
// The partials are accumulated in split order.
__device__ __forceinline__ void merge_group(SplitMerge& r, const float (&l)[16],
                                            const float4 (&v)[16], float safe) {
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if (l[k] == -INFINITY) continue;  // zero weight: that split's row is never used
    const float w = expf(l[k] - safe);
    r.den += w;
    r.acc[0] = fmaf(w, v[k].x, r.acc[0]);
    r.acc[1] = fmaf(w, v[k].y, r.acc[1]);
    r.acc[2] = fmaf(w, v[k].z, r.acc[2]);
    r.acc[3] = fmaf(w, v[k].w, r.acc[3]);
  }
}

// Splits [s0, min(s0 + 16, end)) of a row: LSEs and this lane's partial values (-inf / zero
// past `end`, or for every split of a padded row).
__device__ __forceinline__ void load_group(const float* p, const float* ls, int s0, int end,
                                           bool valid, float (&l)[16], float4 (&v)[16]) {
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const bool in = s0 + k < end;
    l[k] = in ? ls[s0 + k] : -INFINITY;
    v[k] = in ? *reinterpret_cast<const float4*>(p + static_cast<int64_t>(s0 + k) * kHeadDim)
              : make_float4(0.f, 0.f, 0.f, 0.f);
    l[k] = valid ? l[k] : -INFINITY;
  }
}

__device__ __forceinline__ SplitMerge empty_merge() {
  SplitMerge r;
  r.mx = -INFINITY;
  r.den = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.acc[i] = 0.f;
  return r;
}

// Up to 16 splits: one wavefront, one round of loads.
__device__ __forceinline__ SplitMerge merge_splits_row(const float* part, const float* ls,
                                                       int splits, bool valid, int lane) {
  SplitMerge r = empty_merge();
  float l[16];
  float4 v[16];
  load_group(part + lane * 4, ls, 0, splits, valid, l, v);
#pragma unroll
  for (int k = 0; k < 16; ++k) r.mx = fmaxf(r.mx, l[k]);
  merge_group(r, l, v, r.mx == -INFINITY ? 0.f : r.mx);
  return r;
}

// Above 16 splits a row's split slots may be partly unwritten (token-bounded splits give a
// request fewer splits than the launch; kernels write LSE -inf and no partial row there).
// A first pass over the row's LSEs (one per lane, 64 at a time) gives the row max and `end`,
// one past the last finite LSE: every slot below `end` holds a partial row, so the second
// round reads only those.
constexpr int kWaveMergeSplits = 16;

struct LseScan {
  float mx;
  int end;
};
__device__ __forceinline__ LseScan scan_lse(const float* ls, int splits, bool valid) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY, last = -1.f;
  for (int s = lane; s < splits; s += kWave) {
    const float l = ls[s];
    mx = fmaxf(mx, l);
    last = l != -INFINITY ? static_cast<float>(s) : last;  // exact below 2^24
  }
  LseScan r;
  r.mx = valid ? wave_max_dpp(mx) : -INFINITY;
  r.end = valid ? static_cast<int>(wave_max_dpp(last)) + 1 : 0;
  return r;
}

// Splits [s_begin, s_end) of a row by one wavefront into r (r.mx set), 16 per round with
// the next round's loads in flight, in split order.
__device__ __forceinline__ void merge_range(SplitMerge& r, const float* p, const float* ls,
                                            int s_begin, int s_end) {
  const float safe = r.mx == -INFINITY ? 0.f : r.mx;
  float l[16];
  float4 v[16];
  load_group(p, ls, s_begin, s_end, true, l, v);
  for (int s0 = s_begin; s0 < s_end; s0 += 16) {
    float ln[16];
    float4 vn[16];
    load_group(p, ls, s0 + 16, s_end, true, ln, vn);  // empty past the range
    merge_group(r, l, v, safe);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      l[k] = ln[k];
      v[k] = vn[k];
    }
  }
}

// merge_range with its first round (splits [s_begin, s_begin + 16)) already loaded for every
// slot below `splits`, before the LSE scan that sets s_end was complete: slots at or past
// s_end are dropped here, and the rest is merge_range's arithmetic in the same order.
__device__ __forceinline__ void merge_range_pre(SplitMerge& r, const float* p, const float* ls,
                                                int s_begin, int s_end, float (&l)[16],
                                                float4 (&v)[16]) {
  const float safe = r.mx == -INFINITY ? 0.f : r.mx;
#pragma unroll
  for (int k = 0; k < 16; ++k) l[k] = s_begin + k < s_end ? l[k] : -INFINITY;
  for (int s0 = s_begin; s0 < s_end; s0 += 16) {
    float ln[16];
    float4 vn[16];
    load_group(p, ls, s0 + 16, s_end, true, ln, vn);  // empty past the range
    merge_group(r, l, v, safe);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      l[k] = ln[k];
      v[k] = vn[k];
    }
  }
}

// More than 16 splits, one wavefront per row (batches with many rows). The first round's
// loads are requested with the LSE scan's (every slot is inside the row's buffers), so the
// row takes one round of latency less.
__device__ __forceinline__ SplitMerge merge_splits_row_scan(const float* part, const float* ls,
                                                            int splits, bool valid, int lane) {
  SplitMerge r = empty_merge();
  float l[16];
  float4 v[16];
  load_group(part + lane * 4, ls, 0, splits, true, l, v);
  const LseScan sc = scan_lse(ls, splits, valid);
  r.mx = sc.mx;
  merge_range_pre(r, part + lane * 4, ls, 0, sc.end, l, v);
  return r;
}

struct GroupMergeLds {
  float acc[4][kHeadDim];
  float den[4];
};

// More than 16 splits, one workgroup per row (batches with few rows): wavefront w merges
// splits [w q, (w + 1) q) below `end`, q = ceil(splits / 4), and the four partial sums are
// added in wavefront order through LDS. Every wavefront of the workgroup calls this for the
// same row and receives the same result.
__device__ __forceinline__ SplitMerge merge_splits_row_group(const float* part, const float* ls,
                                                             int splits, bool valid,
                                                             GroupMergeLds* lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  SplitMerge r = empty_merge();
  const int q = (splits + 3) >> 2;
  float l[16];
  float4 v[16];
  load_group(part + lane * 4, ls, min(wave * q, splits), splits, true, l, v);
  const LseScan sc = scan_lse(ls, splits, valid);
  r.mx = sc.mx;
  const int s_begin = min(wave * q, sc.end), s_end = min(s_begin + q, sc.end);
  merge_range_pre(r, part + lane * 4, ls, s_begin, s_end, l, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) lds->acc[wave][lane * 4 + i] = r.acc[i];
  if (lane == 0) lds->den[wave] = r.den;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r.acc[i] = ((lds->acc[0][lane * 4 + i] + lds->acc[1][lane * 4 + i]) +
                lds->acc[2][lane * 4 + i]) + lds->acc[3][lane * 4 + i];
  r.den = ((lds->den[0] + lds->den[1]) + lds->den[2]) + lds->den[3];
  __syncthreads();  // the area may be reused by the caller
  return r;
}

// How a launch merges its rows: one round per wavefront-row (<= 16 splits), a scanned
// wavefront-row (more splits, at least 256 rows: four rows share a workgroup), or a
// scanned workgroup-row (more splits, fewer rows). The split merge entry point and the
// post-attention launch use the same rule, so both produce the same bits.
enum MergeMode { kMergeOneRound = 0, kMergeScanWave = 1, kMergeScanGroup = 2 };
__host__ __device__ inline int merge_mode(int64_t rows, int splits) {
  if (splits <= kWaveMergeSplits) return kMergeOneRound;
  return rows >= 256 ? kMergeScanWave : kMergeScanGroup;
}

// The merged row as bf16 (two packed words) and its natural-log LSE.
__device__ __forceinline__ uint2 merge_splits_out(const SplitMerge& r) {
  const float dn = fmaxf(r.den, kDenFloor);
  return make_uint2(pack_bf16x2(r.acc[0] / dn, r.acc[1] / dn),
                    pack_bf16x2(r.acc[2] / dn, r.acc[3] / dn));
}
__device__ __forceinline__ float merge_splits_lse(const SplitMerge& r) {
  return r.den > 0.f ? r.mx + logf(fmaxf(r.den, kDenFloor)) : -INFINITY;
}

// kernels.py:514-527: (e^{la-M} a + e^{lb-M} b) / (e^{la-M} + e^{lb-M}), M = max(la, lb)
// (0 when both are -inf). Padded rows pass la = lb = -inf and zero a, b.
struct PathWeights {
  float wa, wb, den, mx;
};
__device__ __forceinline__ PathWeights path_weights(float la, float lb) {
  PathWeights w;
  w.mx = fmaxf(la, lb);
  w.mx = w.mx == -INFINITY ? 0.f : w.mx;
  w.wa = expf(la - w.mx);
  w.wb = expf(lb - w.mx);
  w.den = fmaxf(w.wa + w.wb, kDenFloor);
  return w;
}
__device__ __forceinline__ float path_merge(const PathWeights& w, float a, float b) {
  return fmaf(w.wa, a, w.wb * b) / w.den;
}
__device__ __forceinline__ float path_lse(const PathWeights& w) {
  return (w.wa + w.wb) > 0.f ? w.mx + logf(w.wa + w.wb) : -INFINITY;
}

}  // namespace oscar
