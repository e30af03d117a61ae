// One-launch layer step: the pieces the history launch takes over from the pre- and
// post-attention launches (their work is latency, which hides under the INT2 stream).
//
// Reference: oscar_ascend/backend.py:171-226, the layer step (rotate K, V, q; store_int2;
// attention_partials history and BF16 branches; merge_splits; rotate(hrot, Rv.T);
// merge_paths; store_windows), kernels.py:51-620.
//
// In a history workgroup (task, kv head, split s) of the layer-step launch:
//   * prologue, while the first INT2 chunks are in flight:
//       - the task's query rows are rotated by R_k in the workgroup (rows 0..7 of a 16-row
//         bf16 MFMA tile, the bits of the rotate entry point), and so are the current key
//         rows of the task (tile rows 8..11) in the workgroup that stores them; a second
//         pass by R_v rotates the current value rows (tile rows 12..15) where they are
//         stored;
//       - the key rows are clipped, INT2-quantized and packed into their slots by split
//         4 % nsplit, the value rows by split 5 % nsplit (the bytes of store_int2);
//       - the BF16 branch is shared by the first min(4, nsplit) splits: raw split r takes the
//         32-token blocks r, r + 4, ... of the task's sink/recent/current tokens, on one
//         wavefront, and writes a normalized partial row and LSE per query row;
//   * epilogue: the workgroup that completes the task (finish.h protocol) merges the history
//     splits and the BF16 splits, rotates the history rows back, merges the two branches,
//     writes the output rows and merged LSE, and stores the task's windows (every split of
//     the task, and so every read of its window, is done by then).
// Coverage: query rows per task <= 8, splits <= 16, one task per request (max_query_len <=
// query_tile); other steps use the three-launch form.
#pragma once

#include "finish.h"
#include "quant.h"
#include "raw.h"
#include "rotate.h"

namespace oscar {

constexpr int kRawSplits = 4;  // BF16-branch partials per task row
constexpr int kStageRowBytes = 512;

struct LayerArgs {
  const uint16_t* rk_t;  // R_k^T, contiguous [256][256] (rk_t[c][k] = R_k[k][c])
  const uint16_t* rv_t;  // R_v^T, contiguous
  uint8_t* history;      // K stripe, written by the INT2 store of the step's tokens
  const int64_t* slots;
  int32_t mode;
  float k_ratio, v_ratio, k_factor, v_factor;
  float* raw_part;       // [rows][kRawSplits][256], device-coherent
  float* raw_lse;        // [rows][kRawSplits]
};

// Byte offset of element `col` of row `row` in a 16-row staging tile whose 512-byte rows keep
// their 16-byte pieces at position piece ^ (row & 31) (the query staging swizzle).
__device__ __forceinline__ int stage_offset(int row, int col) {
  return row * kStageRowBytes + 16 * ((col >> 3) ^ (row & 31)) + 2 * (col & 7);
}

// B operands of this wavefront's four column tiles of R (given as R^T rows), as the rotate
// entry point loads them: lane (n, g) k-step m holds R[32 m + 8 g .. + 7][64 w + 16 ct + n].
__device__ __forceinline__ void load_rt_tiles(const uint16_t* rt, u32x4 (&rb)[4][8]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  RotateOperands op;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    rotate_load_b<true>(op, rt + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[ct][m] = op.b[m];
  }
}

// A operand of the staging tile (row n of lane (n, g), k-step m: elements 32 m + 8 g .. + 7).
__device__ __forceinline__ void load_stage_a(const uint8_t* stage, u32x4 (&a)[8]) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int m = 0; m < 8; ++m)
    a[m] = *reinterpret_cast<const u32x4*>(stage + n * kStageRowBytes +
                                           16 * ((4 * m + g) ^ (n & 31)));
}

// Rows [row_lo, row_hi) of tile @ R into `out` (same swizzle) as bf16: the bits of
// rotate_rows16 (same operands, same k order, one rounding).
__device__ __forceinline__ void rotate_stage(const u32x4 (&a)[8], const u32x4 (&rb)[4][8],
                                             uint8_t* out, int row_lo, int row_hi) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * wave + 16 * ct + n;
    const f32x4 acc = rotate_mfma(a, rb[ct]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      if (r >= row_lo && r < row_hi)
        *reinterpret_cast<uint16_t*>(out + stage_offset(r, col)) =
            static_cast<uint16_t>(float_to_bf16(acc[v]));
    }
  }
}

// This lane's four elements (4 l .. 4 l + 3) of staging row `row`, as floats.
__device__ __forceinline__ void stage_row_floats(const uint8_t* stage, int row, float (&x)[4]) {
  const int lane = threadIdx.x & 63;
  const uint2 w = *reinterpret_cast<const uint2*>(stage + row * kStageRowBytes +
                                                  16 * ((lane >> 1) ^ (row & 31)) + 8 * (lane & 1));
  x[0] = bf16_to_float(w.x & 0xffffu);
  x[1] = bf16_to_float(w.x >> 16);
  x[2] = bf16_to_float(w.y & 0xffffu);
  x[3] = bf16_to_float(w.y >> 16);
}

// store_int2 of one rotated row (kernels.py:104-202 semantics, the pre-attention store):
// token `token`, kv head `head`, K (is_v false) or V bytes of its slot.
__device__ __forceinline__ void store_int2_row(const AttnArgs& a, const LayerArgs& l,
                                               int64_t token, int head, bool is_v,
                                               const float (&x)[4]) {
  if (token < 0 || token >= a.counts[1]) return;
  const int64_t slot = l.slots[token];
  if (slot < 0) return;
  const int64_t base = slot_offset(a.L, slot, head);
  if (base + 2 * a.L.vector_bytes > a.history_bytes) return;
  quantize_store(x, l.mode, is_v ? l.v_ratio : l.k_ratio, is_v ? l.v_factor : l.k_factor,
                 l.history + base + (is_v ? a.L.vector_bytes : 0));
}

// The BF16 branch share of raw split `rs` (< nraw) on the calling wavefront: 32-token blocks
// rs, rs + nraw, ... of the task's raw tokens (sink, recent ring, causal current), query rows
// 0..15 of the task (rows past the task's are masked), the unrotated query `qb` (k-step m of
// lane (n, g): dims 64 g + 8 m .. + 7 of row n). Writes the normalized partial rows and LSEs
// of raw split rs with device-coherent stores (finish.h protocol).
__device__ __forceinline__ void raw_share(const AttnArgs& a, const LayerArgs& l, const Task& t,
                                          const RawTask& r, int head, int rs, int nraw,
                                          const u32x4 (&qb)[8]) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int total = r.high + t.qlen;
  const RowInfo me = row_info(a, t, head, n);
  State<1> st;
  state_init(st);
  for (int t0 = kBlock * rs; t0 < total; t0 += kBlock * nraw) {
    // K rows of the two 16-token score tiles first; the V rows are requested once the score
    // MFMAs have taken the K operands (one fewer operand set in registers: the wavefront runs
    // beside the history stream's registers).
    const uint16_t* kp[2];
    int kpos;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) kp[tt] = raw_token(a, t, r, head, t0 + 16 * tt + n, total, 0, kpos);
    f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    {
      u32x4 kd[2][8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int m = 0; m < 8; ++m)
          kd[tt][m] = kp[tt] ? *reinterpret_cast<const u32x4*>(kp[tt] + 64 * g + 8 * m)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) sc[tt] = mfma16x16x32(kd[tt][m], qb[m], sc[tt]);
    }
    const uint16_t* vp[8];
    int pos[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vp[e] = raw_token(a, t, r, head, t0 + tau(g, e), total, 1, pos[e]);
    u32x4 vd[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      vd[e][0] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n) : u32x4{0u, 0u, 0u, 0u};
      vd[e][1] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n + 8)
                       : u32x4{0u, 0u, 0u, 0u};
    }
    float s2[1][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool ok = vp[e] != nullptr && pos[e] <= t.prefix + me.qi;
      s2[0][e] = ok ? sc[e >> 2][e & 3] * a.scale_log2 : -INFINITY;
    }
    update_max<1, 16>(st, s2, g);
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = s2[0][e] == -INFINITY ? 0.f : exp2f(s2[0][e] - st.m[0]);
      st.psum[0] += p[e];
    }
    u32x4 ap;
#pragma unroll
    for (int f = 0; f < 4; ++f) ap[f] = pack_bf16x2(p[2 * f], p[2 * f + 1]);
#pragma unroll
    for (int tile = 0; tile < 16; ++tile) {
      const uint32_t sel = (tile & 1) ? 0x07060302u : 0x05040100u;
      u32x4 bv;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        bv[f] = __builtin_amdgcn_perm(vd[2 * f + 1][tile >> 3][(tile & 7) >> 1],
                                      vd[2 * f][tile >> 3][(tile & 7) >> 1], sel);
      st.o[0][tile] = mfma16x16x32(ap, bv, st.o[0][tile]);
    }
  }
  // Row totals: lane (n, g) holds row n's max and its share of the row's sum.
  float psum = st.psum[0];
  psum += __shfl_xor(psum, 16, kWave);
  psum += __shfl_xor(psum, 32, kWave);
  // Accumulator element v of lane (n, g) is row 4 g + v, dims 16 n + tile.
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = 4 * g + v;
    const float mx = __shfl(st.m[0], row, kWave);
    const float den = __shfl(psum, row, kWave);
    const RowInfo ri = row_info(a, t, head, row);
    if (!ri.valid) continue;
    const int64_t slot = (ri.token * a.hq + ri.qhead) * kRawSplits + rs;
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    float* dst = l.raw_part + slot * kHeadDim + 16 * n;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      store_coherent(dst + 4 * c, make_float4(st.o[0][4 * c][v] * inv, st.o[0][4 * c + 1][v] * inv,
                                              st.o[0][4 * c + 2][v] * inv,
                                              st.o[0][4 * c + 3][v] * inv));
    if (n == 0)
      store_coherent(l.raw_lse + slot, den > 0.f ? (mx + log2f(den)) * kLn2 : -INFINITY);
  }
}

// Finisher of the layer step (the workgroup that completes the task): finish_task8's
// one-round history merge, plus the merge of the task's `nraw` BF16 partials (fp32, in split
// order, the merge_splits weights) in the same round; then the inverse V rotation, the path
// merge, the output rows and merged LSEs. LDS: `ring` (the history ring: R_v tiles 2, 3 of
// every wavefront, then the 8 x 256 fp32 BF16-branch rows, aliased by the output rows) and
// `fin` (the merged history rows and both branches' LSEs).
constexpr int kLayerRingBytes = kFinishRvBytes + 8 * kHeadDim * 4;
constexpr int kLayerFinBytes = kFinishRowBytes + 2 * 8 * 4;

__device__ __forceinline__ void finish_layer8(const FinishArgs& f, const LayerArgs& l,
                                              const AttnArgs& a, const Task& t, int head,
                                              int nsplit, int nraw, uint8_t* lds, uint8_t* fin) {
  const PostArgs& p = f.p;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int task_rows = a.qt * a.g;
  auto row_of = [&](int r) -> int64_t {
    if (r >= task_rows) return -1;
    const RowInfo ri = row_info(a, t, head, r);
    return ri.valid ? ri.token * a.hq + ri.qhead : -1;
  };
  auto* s_h = reinterpret_cast<uint16_t(*)[kHeadDim]>(fin);
  float* s_l = reinterpret_cast<float*>(fin + kFinishRowBytes);  // history LSEs
  float* s_lb = s_l + 8;                                          // BF16-branch LSEs
  float* s_b = reinterpret_cast<float*>(lds + kFinishRvBytes);
  auto* s_out = reinterpret_cast<uint16_t(*)[kHeadDim]>(s_b);
  const uint32_t rv_lds = lds_addr(lds) + wave * 2 * 8 * 64 * 16;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int m = 0; m < 8; ++m)
      dma_dwordx4(p.rv + static_cast<int64_t>(64 * wave + 16 * (c + 2) + n) * kHeadDim + 32 * m +
                      8 * g,
                  rv_lds + (c * 8 + m) * 64 * 16);
  u32x4 rb[2][8];
  {
    RotateOperands op;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      rotate_load_b<true>(op, p.rv + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1,
                          g);
#pragma unroll
      for (int k = 0; k < 8; ++k) rb[ct][k] = op.b[k];
    }
  }
  const int r = lane >> 3, d0 = 64 * wave + 8 * (lane & 7);
  const int64_t row = row_of(r);
  const bool live = row >= 0;
  const int end = live ? min(nsplit, 16) : 0;
  const int rend = live ? nraw : 0;
  const auto part = coherent_rsrc(p.hp, static_cast<uint32_t>(p.rows * p.splits * kHeadDim * 4));
  const auto lses = coherent_rsrc(p.hl, static_cast<uint32_t>(p.rows * p.splits * 4));
  const auto rpart = coherent_rsrc(l.raw_part,
                                   static_cast<uint32_t>(p.rows * kRawSplits * kHeadDim * 4));
  const auto rlses = coherent_rsrc(l.raw_lse, static_cast<uint32_t>(p.rows * kRawSplits * 4));
  const uint32_t slot0 = static_cast<uint32_t>((live ? row : 0) * p.splits);
  const uint32_t rslot0 = static_cast<uint32_t>((live ? row : 0) * kRawSplits);
  const float lse_lo = load_coherent(lses, (slot0 + (lane & 7)) * 4);
  const float lse_hi = load_coherent(lses, (slot0 + 8 + (lane & 7)) * 4);
  const float rlse = load_coherent(rlses, (rslot0 + (lane & 3)) * 4);
  float4 v[16][2], w[kRawSplits][2];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t at = ((slot0 + k) * kHeadDim + d0) * 4;
    v[k][0] = load_coherent4(part, at);
    v[k][1] = load_coherent4(part, at + 16);
  }
#pragma unroll
  for (int k = 0; k < kRawSplits; ++k) {
    const uint32_t at = ((rslot0 + k) * kHeadDim + d0) * 4;
    w[k][0] = load_coherent4(rpart, at);
    w[k][1] = load_coherent4(rpart, at + 16);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the merges start
  const int group = lane & ~7;
  auto lse_of = [&](int k) {
    const float x = __shfl(k < 8 ? lse_lo : lse_hi, group + (k & 7), kWave);
    return k < end ? x : -INFINITY;
  };
  // History splits: merge_splits arithmetic, bf16 rows for the inverse rotation.
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) mx = fmaxf(mx, lse_of(k));
  float safe = mx == -INFINITY ? 0.f : mx;
  float den = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float lk = lse_of(k);
    if (lk == -INFINITY) continue;
    const float wk = expf(lk - safe);
    den += wk;
    const float x[8] = {v[k][0].x, v[k][0].y, v[k][0].z, v[k][0].w,
                        v[k][1].x, v[k][1].y, v[k][1].z, v[k][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(wk, x[i], acc[i]);
  }
  SplitMerge m0, m1;
  m0.den = m1.den = den;
  m0.mx = m1.mx = mx;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m0.acc[i] = acc[i];
    m1.acc[i] = acc[4 + i];
  }
  *reinterpret_cast<uint2*>(&s_h[r][d0]) = merge_splits_out(m0);
  *reinterpret_cast<uint2*>(&s_h[r][d0 + 4]) = merge_splits_out(m1);
  if (wave == 0 && (lane & 7) == 0) s_l[r] = merge_splits_lse(m0);
  // BF16 splits: the same weights, kept in fp32 (the BF16 branch's rows enter the path merge
  // as fp32, kernels.py:514-527).
  auto rlse_of = [&](int k) {
    const float x = __shfl(rlse, group + (k & 3), kWave);
    return k < rend ? x : -INFINITY;
  };
  float rmx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kRawSplits; ++k) rmx = fmaxf(rmx, rlse_of(k));
  safe = rmx == -INFINITY ? 0.f : rmx;
  float rden = 0.f, racc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < kRawSplits; ++k) {
    const float lk = rlse_of(k);
    if (lk == -INFINITY) continue;
    const float wk = expf(lk - safe);
    rden += wk;
    const float x[8] = {w[k][0].x, w[k][0].y, w[k][0].z, w[k][0].w,
                        w[k][1].x, w[k][1].y, w[k][1].z, w[k][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) racc[i] = fmaf(wk, x[i], racc[i]);
  }
  {
    const float dn = fmaxf(rden, kDenFloor);
    float* dst = s_b + r * kHeadDim + d0;
    *reinterpret_cast<float4*>(dst) =
        make_float4(racc[0] / dn, racc[1] / dn, racc[2] / dn, racc[3] / dn);
    *reinterpret_cast<float4*>(dst + 4) =
        make_float4(racc[4] / dn, racc[5] / dn, racc[6] / dn, racc[7] / dn);
    if (wave == 0 && (lane & 7) == 0)
      s_lb[r] = rden > 0.f ? rmx + logf(fmaxf(rden, kDenFloor)) : -INFINITY;
  }
  OSCAR_WAIT_VM(0);  // the R_v DMA of this wavefront
  __syncthreads();
  // BF16-branch operands of the path merge (rows 4 g + v, columns 64 w + 16 ct + n).
  PathRows pr;
#pragma unroll
  for (int vv = 0; vv < 4; ++vv) {
    const int rr = 4 * g + vv;
    pr.row[vv] = rr < 8 ? row_of(rr) : -1;
    pr.valid[vv] = pr.row[vv] >= 0;
    pr.lb[vv] = pr.valid[vv] ? s_lb[rr < 8 ? rr : 0] : -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      pr.bv[vv][ct] = pr.valid[vv] ? s_b[(rr < 8 ? rr : 0) * kHeadDim + 64 * wave + 16 * ct + n]
                                   : 0.f;
  }
  __syncthreads();  // s_b is read; the output rows overwrite it
  const uint8_t* rv_tiles = lds + wave * 2 * 8 * 64 * 16;
  rotate_merge<8>(
      p, pr,
      [&](int ct, u32x4(&b)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          b[k] = ct < 2 ? rb[ct][k]
                        : *reinterpret_cast<const u32x4*>(rv_tiles + ((ct - 2) * 8 + k) * 64 * 16 +
                                                          lane * 16);
      },
      s_h, s_l, [&](int tr, int64_t, int col, uint16_t bits) { s_out[tr][col] = bits; });
  __syncthreads();
  {
    const int orow = threadIdx.x >> 5, c0 = 8 * (threadIdx.x & 31);
    const int64_t out_row = row_of(orow);
    if (out_row >= 0)
      *reinterpret_cast<uint4*>(p.out + out_row * kHeadDim + c0) =
          *reinterpret_cast<const uint4*>(&s_out[orow][c0]);
  }
}

// Output rows of tokens at or past the token count (graph padding): zero, LSE -inf, the
// path merge of two empty branches. Split 0 of task x clears tokens x, x + programs, ...
__device__ __forceinline__ void clear_padded_rows(const FinishArgs& f, int x) {
  const int active = f.p.counts[1];
  const int64_t tokens = f.p.rows / f.p.hq;
  for (int64_t tok = x; tok < tokens; tok += f.programs) {
    if (tok < active) continue;
    uint16_t* out = f.p.out + tok * f.p.hq * kHeadDim;
    for (int e = threadIdx.x; e < f.p.hq * kHeadDim; e += kThreads) out[e] = 0;
    if (f.p.merged_lse && threadIdx.x < f.p.hq) f.p.merged_lse[tok * f.p.hq + threadIdx.x] = -INFINITY;
  }
}

hipError_t launch_layer_step(const AttnArgs& a, const FinishArgs& f, const LayerArgs& l,
                             hipStream_t stream);

}  // namespace oscar
