// Post-attention of the layer step: split merge, inverse V rotation and path merge of a group
// of (token, query head) rows, for the post-attention launch. It runs the row arithmetic of
// the merge_splits / rotate / merge_paths entry points, so both paths produce the same bits.
//
// Reference: oscar_ascend/backend.py:209-210, 223 (`merge_splits`, `rotate(hrot, Rv.T)`,
// `merge_paths`; kernels.py:485-541).
#pragma once

#include "merge.h"
#include "rotate.h"
#include "window.h"

namespace oscar {

struct PostArgs {
  const float* hp;  // history partials [rows][splits][256]
  const float* hl;  // history LSE [rows][splits]
  int32_t splits;
  const float* rp;  // BF16-branch partials [rows][256]
  const float* rl;  // BF16-branch LSE [rows]
  const int32_t* counts;
  const uint16_t* rv;  // R_v, row-major: column c of R_v^T is row c of R_v
  int64_t rows;        // n * hq
  int32_t hq;
  uint16_t* out;       // [rows][256]
  float* merged_lse;   // [rows] or null
  WindowArgs win;
  int64_t win_requests;  // min(n, max_reqs)
  int32_t merge_wgs;     // workgroups of the merge role; the rest store windows
};

// Rows [row0, min(row0 + R, row_end, p.rows)) by the four wavefronts of a workgroup:
// wavefront w merges rows w, w + 4, ... into LDS (s_h: R x 256 bf16, s_l: R floats), or, with
// R = 1 (kMergeScanGroup), all four merge the one row together; then every wavefront rotates
// the R rows back for 64 output columns and merges them with the BF16 branch. Every read
// that does not depend on the merge (R_v, the BF16-branch values and LSEs) is requested
// before it, and none waits for the token count.
template <int R, int kMode>
__device__ __forceinline__ void post_rows(const PostArgs& p, int64_t row0, int64_t row_end,
                                          uint16_t (*s_h)[kHeadDim], float* s_l,
                                          GroupMergeLds* group_lds) {
  static_assert(R == 1 || R == 4 || R == 16, "row groups of 1, 4 or 16");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int active = p.counts[1];
  row_end = min(row_end, p.rows);
  // R_v operands of this wavefront's four column tiles, requested first.
  RotateOperands op;
  u32x4 rb[4][8];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    rotate_load_b<true>(op, p.rv + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[ct][m] = op.b[m];
  }
  // BF16-branch values merged by this lane: tile rows 4g + v (rows below R).
  float bv[4][4], lb[4];
  bool valid[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * g + v;
    const int64_t row = row0 + r;
    const bool in = r < R && row < row_end;
    const int64_t lrow = in ? row : 0;
    valid[v] = in && row / p.hq < active;
    const float l = p.rl[lrow];
    lb[v] = valid[v] ? l : -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const float x = p.rp[lrow * kHeadDim + 64 * wave + 16 * ct + n];
      bv[v][ct] = valid[v] ? x : 0.f;
    }
  }
  if (R == 1) {
    const bool in = row0 < row_end;
    const int64_t lrow = in ? row0 : 0;
    const SplitMerge m = merge_splits_row_group(p.hp + lrow * p.splits * kHeadDim,
                                                p.hl + lrow * p.splits, p.splits,
                                                in && row0 / p.hq < active, group_lds);
    if (wave == 0) {
      *reinterpret_cast<uint2*>(&s_h[0][lane * 4]) = merge_splits_out(m);
      if (lane == 0) s_l[0] = merge_splits_lse(m);
    }
  } else {
    for (int r = wave; r < R; r += kThreads / kWave) {
      const int64_t row = row0 + r;
      const bool in = row < row_end;
      const float* part = p.hp + (in ? row : 0) * p.splits * kHeadDim;
      const float* ls = p.hl + (in ? row : 0) * p.splits;
      const bool live = in && row / p.hq < active;
      const SplitMerge m = kMode == kMergeOneRound
                               ? merge_splits_row(part, ls, p.splits, live, lane)
                               : merge_splits_row_scan(part, ls, p.splits, live, lane);
      *reinterpret_cast<uint2*>(&s_h[r][lane * 4]) = merge_splits_out(m);
      if (lane == 0) s_l[r] = merge_splits_lse(m);
    }
  }
  __syncthreads();
  // Inverse rotation of the R merged rows (rows R..15 of the MFMA tile are zero), then the
  // path merge of each element with the BF16 branch.
  rotate_load_a<true>(op, n < R ? &s_h[n][0] : nullptr, 1, g);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * wave + 16 * ct + n;
    const f32x4 acc = rotate_mfma(op.a, rb[ct]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      const int64_t row = row0 + r;
      if (r >= R || row >= row_end) continue;
      const PathWeights w = path_weights(valid[v] ? s_l[r] : -INFINITY, lb[v]);
      const float av = valid[v] ? bf16_to_float(float_to_bf16(acc[v])) : 0.f;
      p.out[row * kHeadDim + col] =
          static_cast<uint16_t>(float_to_bf16(path_merge(w, av, bv[v][ct])));
      if (p.merged_lse && wave == 0 && ct == 0 && n == 0) p.merged_lse[row] = path_lse(w);
    }
  }
}

}  // namespace oscar
