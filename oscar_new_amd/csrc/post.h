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

// BF16-branch operands of this lane's tile rows 4g + v (rows below R) for the path merge.
struct PathRows {
  int64_t row[4];  // row index, or -1
  bool valid[4];   // a row below the token count
  float bv[4][4];  // BF16-branch values of columns 64 wave + 16 ct + n
  float lb[4];     // BF16-branch LSEs
};

template <int R, class RowOf>
__device__ __forceinline__ void load_path_rows(const PostArgs& p, RowOf row_of, int active,
                                               PathRows& pr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * g + v;
    pr.row[v] = r < R ? row_of(r) : -1;
    const bool in = pr.row[v] >= 0;
    const int64_t lrow = in ? pr.row[v] : 0;
    pr.valid[v] = in && pr.row[v] / p.hq < active;
    const float l = p.rl[lrow];
    pr.lb[v] = pr.valid[v] ? l : -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const float x = p.rp[lrow * kHeadDim + 64 * wave + 16 * ct + n];
      pr.bv[v][ct] = pr.valid[v] ? x : 0.f;
    }
  }
}

// Inverse rotation of the R merged rows in s_h (rows R..15 of the MFMA tile are zero) by this
// wavefront's four R_v column tiles (get_b(ct, b) supplies tile ct's B operand), then the path
// merge of each element with the BF16 branch; put(r, row, col, bits) stores output element
// (tile row r, row index `row`, column col), and the merged LSE is stored here.
template <int R, class GetB, class Put>
__device__ __forceinline__ void rotate_merge(const PostArgs& p, const PathRows& pr, GetB get_b,
                                             uint16_t (*s_h)[kHeadDim], const float* s_l,
                                             Put put) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  RotateOperands op;
  rotate_load_a<true>(op, n < R ? &s_h[n][0] : nullptr, 1, g);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * wave + 16 * ct + n;
    u32x4 b[8];
    get_b(ct, b);
    const f32x4 acc = rotate_mfma(op.a, b);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      const int64_t row = pr.row[v];
      if (r >= R || row < 0) continue;
      const PathWeights w = path_weights(pr.valid[v] ? s_l[r] : -INFINITY, pr.lb[v]);
      const float av = pr.valid[v] ? bf16_to_float(float_to_bf16(acc[v])) : 0.f;
      put(r, row, col, static_cast<uint16_t>(float_to_bf16(path_merge(w, av, pr.bv[v][ct]))));
      if (p.merged_lse && wave == 0 && ct == 0 && n == 0) p.merged_lse[row] = path_lse(w);
    }
  }
}

// Rows row_of(0 .. R-1) (a row index in [0, p.rows), or -1 for none) by the four wavefronts
// of a workgroup: wavefront w merges rows w, w + 4, ... into LDS (s_h: R x 256 bf16, s_l: R
// floats), or, with R = 1 (kMergeScanGroup), all four merge the one row together; then every
// wavefront rotates the R rows back for 64 output columns and merges them with the BF16
// branch. Splits at or past `live_splits` are not read (the row stride stays p.splits).
// The reads that do not depend on the merge (the BF16-branch values and LSEs, and the R_v
// operands of the first kEarly column tiles) are requested before it, the other R_v tiles
// after it (fewer registers live across the merge); none waits for the token count.
// kTiles 2 (R = 16): rows row_of(0 .. 31), the two groups of 16 one after the other, R_v's
// operands read once for both.
template <int R, int kMode, int kEarly = 4, int kTiles = 1, class RowOf>
__device__ __forceinline__ void post_rows_map(const PostArgs& p, RowOf row_of, int live_splits,
                                              uint16_t (*s_h)[kHeadDim], float* s_l,
                                              GroupMergeLds* group_lds) {
  static_assert(R == 1 || R == 4 || R == 8 || R == 16, "row groups of 1, 4, 8 or 16");
  static_assert(kEarly >= 0 && kEarly <= 4, "four column tiles per wavefront");
  static_assert(kTiles == 1 || (kTiles == 2 && R == 16), "two tiles of 16 rows");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int active = p.counts[1];
  RotateOperands op;
  u32x4 rb[4][8];
  auto load_rv = [&](int ct) {
    rotate_load_b<true>(op, p.rv + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[ct][m] = op.b[m];
  };
#pragma unroll
  for (int ct = 0; ct < kEarly; ++ct) load_rv(ct);
  // kTiles 2: rows row_of(0 .. 2R-1) as two groups of R, one after the other, with R_v's
  // operands read once (the group barrier ends the first group's reads of s_h and s_l).
  for (int t = 0; t < kTiles; ++t) {
    if (t > 0) __syncthreads();
    auto rof = [&](int r) -> int64_t { return row_of(R * t + r); };
    PathRows pr;
    load_path_rows<R>(p, rof, active, pr);
    if (R == 1) {
      const int64_t row0 = rof(0);
      const bool in = row0 >= 0;
      const int64_t lrow = in ? row0 : 0;
      const SplitMerge m = merge_splits_row_group(p.hp + lrow * p.splits * kHeadDim,
                                                  p.hl + lrow * p.splits, live_splits,
                                                  in && row0 / p.hq < active, group_lds);
      if (wave == 0) {
        *reinterpret_cast<uint2*>(&s_h[0][lane * 4]) = merge_splits_out(m);
        if (lane == 0) s_l[0] = merge_splits_lse(m);
      }
    } else if (kMode == kMergeOneRound && R > 4 && live_splits == 1) {
      // One split (long chunks): every row's partial and LSE requested before any is merged
      // (one round of latency instead of one per row), then merge_splits_row's arithmetic.
      constexpr int kPer = R / (kThreads / kWave);
      float l0[kPer];
      float4 v0[kPer];
      bool live[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int64_t row = rof(wave + (kThreads / kWave) * i);
        const bool in = row >= 0;
        live[i] = in && row / p.hq < active;
        l0[i] = p.hl[(in ? row : 0) * p.splits];
        v0[i] = *reinterpret_cast<const float4*>(p.hp + (in ? row : 0) * p.splits * kHeadDim +
                                                 lane * 4);
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int r = wave + (kThreads / kWave) * i;
        float l[16];
        float4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          l[k] = k == 0 && live[i] ? l0[i] : -INFINITY;
          v[k] = k == 0 ? v0[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        SplitMerge m = empty_merge();
#pragma unroll
        for (int k = 0; k < 16; ++k) m.mx = fmaxf(m.mx, l[k]);
        merge_group(m, l, v, m.mx == -INFINITY ? 0.f : m.mx);
        *reinterpret_cast<uint2*>(&s_h[r][lane * 4]) = merge_splits_out(m);
        if (lane == 0) s_l[r] = merge_splits_lse(m);
      }
    } else {
      for (int r = wave; r < R; r += kThreads / kWave) {
        const int64_t row = rof(r);
        const bool in = row >= 0;
        const float* part = p.hp + (in ? row : 0) * p.splits * kHeadDim;
        const float* ls = p.hl + (in ? row : 0) * p.splits;
        const bool live = in && row / p.hq < active;
        const SplitMerge m = kMode == kMergeOneRound
                                 ? merge_splits_row(part, ls, live_splits, live, lane)
                                 : merge_splits_row_scan(part, ls, live_splits, live, lane);
        *reinterpret_cast<uint2*>(&s_h[r][lane * 4]) = merge_splits_out(m);
        if (lane == 0) s_l[r] = merge_splits_lse(m);
      }
    }
    if (t == 0) {
#pragma unroll
      for (int ct = kEarly; ct < 4; ++ct) load_rv(ct);
    }
    __syncthreads();
    rotate_merge<R>(
        p, pr,
        [&](int ct, u32x4(&b)[8]) {
#pragma unroll
          for (int m = 0; m < 8; ++m) b[m] = rb[ct][m];
        },
        s_h, s_l,
        [&](int, int64_t row, int col, uint16_t bits) { p.out[row * kHeadDim + col] = bits; });
  }
}

// Rows [row0, min(row0 + R, p.rows)) (R <= 4, one per wavefront) for kQuarters quarters of
// 64 output columns starting at `quarter`: wavefront w merges row w into LDS, then, per
// quarter, rotates the merged rows back for column tile w of the quarter (16 columns) and
// merges them with the BF16 branch. kQuarters 1 (few rows): the four quarter workgroups of a
// row group each merge the same rows (the same bits) and read a quarter of R_v, so that no
// workgroup streams all of R_v (a latency-bound workgroup's reads are limited by its own
// outstanding requests). kQuarters 4 (many rows): one workgroup per row group merges once and
// walks the four quarters, the next quarter's R_v columns and BF16 values requested before
// the current quarter is computed. Each output element takes the arithmetic of rotate_merge
// (same operands, same MFMA k order, same path merge).
// kMode: the split merge of the launch (merge_mode): one round or a scan per wavefront-row,
// or (R = 1) the four wavefronts merging the row together, as the other post paths do.
template <int R, int kMode, int kQuarters = 1>
__device__ __forceinline__ void post_rows_quarter(const PostArgs& p, int64_t row0, int quarter,
                                                  uint16_t (*s_h)[kHeadDim], float* s_l,
                                                  GroupMergeLds* group_lds) {
  static_assert(R >= 1 && R <= 4, "one merged row per wavefront");
  static_assert(kMode != kMergeScanGroup || R == 1, "a workgroup-row merge serves one row");
  static_assert(kQuarters == 1 || kQuarters == 4, "one quarter or all four");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t end = min(row0 + R, p.rows);
  const int active = p.counts[1];
  int64_t row[4];
  bool valid[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * g + v;
    row[v] = r < R && row0 + r < end ? row0 + r : -1;
    valid[v] = row[v] >= 0 && row[v] / p.hq < active;
  }
  // R_v columns and BF16-branch values and LSEs of this lane's rows 4g + v at column `col`.
  auto load_quarter = [&](int q, u32x4 (&rb)[8], float (&bv)[4], float (&lb)[4]) {
    const int col = 64 * q + 16 * wave + n;
    RotateOperands op;
    rotate_load_b<true>(op, p.rv + static_cast<int64_t>(col) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[m] = op.b[m];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t lrow = row[v] >= 0 ? row[v] : 0;
      const float l = p.rl[lrow];
      const float x = p.rp[lrow * kHeadDim + col];
      lb[v] = valid[v] ? l : -INFINITY;
      bv[v] = valid[v] ? x : 0.f;
    }
  };
  u32x4 rb[8];
  float bv[4], lb[4];
  load_quarter(quarter, rb, bv, lb);
  if constexpr (kMode == kMergeScanGroup) {
    const bool in = row0 < end;
    const SplitMerge m = merge_splits_row_group(p.hp + (in ? row0 : 0) * p.splits * kHeadDim,
                                                p.hl + (in ? row0 : 0) * p.splits, p.splits,
                                                in && row0 / p.hq < active, group_lds);
    if (wave == 0) {
      *reinterpret_cast<uint2*>(&s_h[0][lane * 4]) = merge_splits_out(m);
      if (lane == 0) s_l[0] = merge_splits_lse(m);
    }
  } else if (wave < R) {
    const int64_t r = row0 + wave;
    const bool in = r < end;
    const float* part = p.hp + (in ? r : 0) * p.splits * kHeadDim;
    const float* ls = p.hl + (in ? r : 0) * p.splits;
    const bool live = in && r / p.hq < active;
    const SplitMerge m = kMode == kMergeOneRound
                             ? merge_splits_row(part, ls, p.splits, live, lane)
                             : merge_splits_row_scan(part, ls, p.splits, live, lane);
    *reinterpret_cast<uint2*>(&s_h[wave][lane * 4]) = merge_splits_out(m);
    if (lane == 0) s_l[wave] = merge_splits_lse(m);
  }
  __syncthreads();
  RotateOperands op;
  rotate_load_a<true>(op, n < R ? &s_h[n][0] : nullptr, 1, g);
#pragma unroll 1
  for (int qq = 0; qq < kQuarters; ++qq) {
    const int q = quarter + qq;
    const int col = 64 * q + 16 * wave + n;
    u32x4 rb_next[8];
    float bv_next[4], lb_next[4];
    if (kQuarters > 1 && qq + 1 < kQuarters) load_quarter(q + 1, rb_next, bv_next, lb_next);
    const f32x4 acc = rotate_mfma(op.a, rb);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      if (r >= R || row[v] < 0) continue;
      const PathWeights w = path_weights(valid[v] ? s_l[r] : -INFINITY, lb[v]);
      const float av = valid[v] ? bf16_to_float(float_to_bf16(acc[v])) : 0.f;
      p.out[row[v] * kHeadDim + col] =
          static_cast<uint16_t>(float_to_bf16(path_merge(w, av, bv[v])));
      if (p.merged_lse && q == 0 && wave == 0 && n == 0) p.merged_lse[row[v]] = path_lse(w);
    }
    if (kQuarters > 1 && qq + 1 < kQuarters) {
#pragma unroll
      for (int m = 0; m < 8; ++m) rb[m] = rb_next[m];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        bv[v] = bv_next[v];
        lb[v] = lb_next[v];
      }
    }
  }
}

}  // namespace oscar
