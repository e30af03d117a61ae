// The BF16 branch of the split-KV attention (sink, recent ring and current tokens), shared by
// the attention_partials entry point, the fused pre-attention launch, the history launch's
// pre-attention roles and (row for row) the initial-prefill kernel.
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel` with IS_RAW true: raw
// positions = sink + recent window + causal current tokens, kernels.py:421-470).
//
// Row arithmetic (what every path reproduces bit for bit): each query row streams the split's
// 32-token blocks in order through one online softmax on bf16 MFMA (v_mfma_f32_16x16x32_bf16):
// scores S^T = K Q^T (16-token tiles, k in eight 32-dim steps), a lazy running max (a row moves
// its max only when a block's row maximum passes it by 2^8), p = 2^(s - m) packed to bf16, and
// P*V accumulated in fp32; the row sum is reduced across its four lane groups at the end.
// Scores come out transposed, so the MFMA output layout (lane holds 4 consecutive tokens of
// one query row) is the A-operand layout of the P*V MFMA with no shuffle in between. A row's
// bits depend only on its own query, the keys and values, not on which rows share its tile,
// its wavefront or its workgroup.
//
// Decode workgroup: 4 wavefronts over the same rows and blocks, wavefront w accumulating the
// 64 output dims 16 n + 4 w + {0..3} (n = lane & 15) of every row; each computes the scores
// itself (the same bits in every wavefront), so no merge of wavefront states is needed.
#pragma once

#include "attention.h"
#include "dma.h"

namespace oscar {

constexpr float kRescale = 8.0f;  // lazy-max slack, log2 units
constexpr int kBlock = 32;        // tokens per block

// Per-lane token of element e of the PV k-group g: 4 consecutive tokens of each 16-token
// QK tile, matching the transposed-score output layout.
__device__ __forceinline__ int tau(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

// 2^x by the hardware instruction (v_exp_f32; results below 2^-126 flush to zero): the p and
// rescale factors of the BF16 branch, whose bf16 P operand cannot hold smaller values anyway.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- softmax state

// kTiles P*V accumulator tiles per row tile: tile j of lane (n, g) holds rows 4 g + v, one
// output dim each (the caller's dim map; 16 tiles: dims 16 n + j).
template <int RT, int kTiles = 16>
struct State {
  float m[RT];          // running max (log2 units) of query row n + 16 rt
  float psum[RT];       // sum p over this lane's tokens
  f32x4 o[RT][kTiles];  // P*V accumulators
};

template <int RT, int kTiles>
__device__ __forceinline__ void state_init(State<RT, kTiles>& st) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st.m[rt] = -INFINITY;
    st.psum[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) st.o[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// Lazy running max, per row. Each lane first checks its own 8 scores of the block against
// m + 2^8 (block_need, no cross-lane traffic); only if some lane of the wavefront sees a larger
// score are the block's row maxima reduced across the 4 lane groups (block_rescale), and then
// exactly the rows whose block maximum passes m + 2^8 move m to it and rescale their sum and
// accumulators (the other rows multiply by exactly 1). Between updates p <= 2^8.
template <int RT>
__device__ __forceinline__ void block_scores(const f32x4 (&sc)[RT][2], const bool (&ok)[RT][8],
                                             float scale_log2, float (&s2)[RT][8]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int e = 0; e < 8; ++e) s2[rt][e] = ok[rt][e] ? sc[rt][e >> 2][e & 3] * scale_log2 : -INFINITY;
}

// Scores of a block every row sees in full (no mask).
template <int RT>
__device__ __forceinline__ void block_scores_full(const f32x4 (&sc)[RT][2], float scale_log2,
                                                  float (&s2)[RT][8]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int e = 0; e < 8; ++e) s2[rt][e] = sc[rt][e >> 2][e & 3] * scale_log2;
}

template <int RT, int kTiles>
__device__ __forceinline__ bool block_need(const State<RT, kTiles>& st, const float (&s2)[RT][8],
                                           float (&lm)[RT]) {
  bool need = false;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float v = s2[rt][0];
#pragma unroll
    for (int e = 1; e < 8; ++e) v = fmaxf(v, s2[rt][e]);
    lm[rt] = v;
    need |= v > st.m[rt] + kRescale;
  }
  return need;
}

template <int RT, int kTiles>
__device__ __forceinline__ void block_rescale(State<RT, kTiles>& st, const float (&lm)[RT], int g) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float v = lm[rt];
    v = fmaxf(v, __shfl_xor(v, 16, kWave));
    v = fmaxf(v, __shfl_xor(v, 32, kWave));
    const float mo = st.m[rt];
    const float mn = v > mo + kRescale ? v : mo;
    const float alpha = mn == mo ? 1.0f : (mn == -INFINITY ? 1.0f : exp2_hw(mo - mn));
    st.m[rt] = mn;
    st.psum[rt] *= alpha;
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const float av = __shfl(alpha, 4 * g + v4, kWave);
#pragma unroll
      for (int t = 0; t < kTiles; ++t) st.o[rt][t][v4] *= av;
    }
  }
}

template <int RT, int kTiles>
__device__ __forceinline__ void update_max(State<RT, kTiles>& st, const float (&s2)[RT][8], int g) {
  float lm[RT];
  if (__any(block_need(st, s2, lm))) block_rescale(st, lm, g);
}

// p = 2^(s - m), the lane's sum and the bf16 P operand (lane (n, g): row n, tokens tau(g, e)).
template <int RT, int kTiles>
__device__ __forceinline__ void block_p(State<RT, kTiles>& st, const float (&s2)[RT][8],
                                        u32x4 (&ap)[RT]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = s2[rt][e] == -INFINITY ? 0.f : exp2_hw(s2[rt][e] - st.m[rt]);
      st.psum[rt] += p[e];
    }
#pragma unroll
    for (int f = 0; f < 4; ++f) ap[rt][f] = pack_bf16x2(p[2 * f], p[2 * f + 1]);
  }
}

// The block's scores of row tile rt to log2 units with the causal / range mask, then the
// lazy max, p, the lane's sum and the bf16 P operand.
template <int RT, int kTiles>
__device__ __forceinline__ void block_softmax(State<RT, kTiles>& st, const f32x4 (&sc)[RT][2],
                                              const bool (&ok)[RT][8], float scale_log2, int g,
                                              u32x4 (&ap)[RT]) {
  float s2[RT][8];
  block_scores(sc, ok, scale_log2, s2);
  update_max(st, s2, g);
  block_p(st, s2, ap);
}

// B operand of P*V for output dim 16 n + j: the bf16 values of dim j of this lane's eight
// tokens, as token pairs (vd2[e]: dims 2 d, 2 d + 1 of the lane's dword d = j / 2 of token e).
__device__ __forceinline__ u32x4 pv_operand(const uint32_t (&vd2)[8], int j) {
  const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
  u32x4 bv;
#pragma unroll
  for (int f = 0; f < 4; ++f) bv[f] = __builtin_amdgcn_perm(vd2[2 * f + 1], vd2[2 * f], sel);
  return bv;
}

// The row's normalizer and natural-log LSE from the lane's sum (all 4 lane groups of row n
// hold the full sum after the reduction) and max.
__device__ __forceinline__ float row_sum(float psum) {
  psum += __shfl_xor(psum, 16, kWave);
  psum += __shfl_xor(psum, 32, kWave);
  return psum;
}
__device__ __forceinline__ float row_lse(float mx, float den) {
  return den > 0.f ? (mx + log2f(den)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------- raw (BF16) branch

struct RawTask {
  int high;     // sink_len + prefix - recent_begin: first current-token index
  int64_t win;  // element offset of (window index 0, K, this head), or -1
};

// Position and bf16 row pointer (K if kv == 0, else V) of raw index ns; nullptr if masked.
__device__ __forceinline__ const uint16_t* raw_token(const AttnArgs& a, const Task& t,
                                                     const RawTask& r, int head, int ns, int end,
                                                     int kv, int& pos) {
  pos = 0x7fffffff;
  if (ns < 0 || ns >= end) return nullptr;
  if (ns < t.sink_len)
    pos = ns;
  else if (ns < r.high)
    pos = t.recent_begin + ns - t.sink_len;
  else
    pos = t.prefix + ns - r.high;
  if (pos >= t.prefix) {
    const int64_t ci = static_cast<int64_t>(t.qstart) + pos - t.prefix;
    if (ci < 0 || ci >= a.n) return nullptr;
    return kv ? a.value + ci * a.vs0 + head * a.vs1 : a.key + ci * a.ks0 + head * a.ks1;
  }
  if (r.win < 0 || pos < 0) return nullptr;
  const uint32_t lap = fastdiv(static_cast<uint32_t>(pos), a.L.ring_div);
  const int wi = pos < a.L.sink ? pos : a.L.sink + pos - static_cast<int>(lap) * a.L.ring;
  const int64_t off = r.win + (static_cast<int64_t>(wi) * 2 + kv) * a.L.kv_heads * kHeadDim;
  if (off + kHeadDim > a.window_elems) return nullptr;
  return a.window + off;
}

// raw_token for K and V at once: the position of raw index ns, or INT_MAX if the index holds
// no token (no V row; raw_token's nullptr), and both row pointers (nullptr where raw_token
// gives nullptr).
__device__ __forceinline__ int raw_row(const AttnArgs& a, const Task& t, const RawTask& r,
                                       int head, int ns, int end, const uint16_t*& kp,
                                       const uint16_t*& vp) {
  kp = vp = nullptr;
  if (ns < 0 || ns >= end) return 0x7fffffff;
  int pos;
  if (ns < t.sink_len)
    pos = ns;
  else if (ns < r.high)
    pos = t.recent_begin + ns - t.sink_len;
  else
    pos = t.prefix + ns - r.high;
  if (pos >= t.prefix) {
    const int64_t ci = static_cast<int64_t>(t.qstart) + pos - t.prefix;
    if (ci < 0 || ci >= a.n) return 0x7fffffff;
    kp = a.key + ci * a.ks0 + head * a.ks1;
    vp = a.value + ci * a.vs0 + head * a.vs1;
    return pos;
  }
  if (r.win < 0 || pos < 0) return 0x7fffffff;
  const uint32_t lap = fastdiv(static_cast<uint32_t>(pos), a.L.ring_div);
  const int wi = pos < a.L.sink ? pos : a.L.sink + pos - static_cast<int>(lap) * a.L.ring;
  const int64_t off = r.win + static_cast<int64_t>(wi) * 2 * a.L.kv_heads * kHeadDim;
  const int64_t voff = off + static_cast<int64_t>(a.L.kv_heads) * kHeadDim;
  if (off + kHeadDim <= a.window_elems) kp = a.window + off;
  if (voff + kHeadDim > a.window_elems) return 0x7fffffff;
  vp = a.window + voff;
  return pos;
}

__device__ __forceinline__ const uint16_t* shfl_ptr(const uint16_t* p, int src) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __shfl(static_cast<uint32_t>(v), src, kWave);
  const uint32_t hi = __shfl(static_cast<uint32_t>(v >> 32), src, kWave);
  return reinterpret_cast<const uint16_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// K rows of the block's two 16-token score tiles (A operands: lane (n, g), k-step m holds dims
// 64 g + 8 m .. + 7 of token 16 tt + n).
__device__ __forceinline__ void raw_load_k(const AttnArgs& a, const Task& t, const RawTask& r,
                                           int head, int t0, int end, int g, int n,
                                           u32x4 (&kd)[2][8]) {
  const uint16_t* kp[2];
  int kpos;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) kp[tt] = raw_token(a, t, r, head, t0 + 16 * tt + n, end, 0, kpos);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int m = 0; m < 8; ++m)
      kd[tt][m] = kp[tt] ? *reinterpret_cast<const u32x4*>(kp[tt] + 64 * g + 8 * m)
                         : u32x4{0u, 0u, 0u, 0u};
}

// V dims 16 n + 4 w .. + 3 of this lane's eight tokens (two dwords each), with the positions
// that mask them.
__device__ __forceinline__ void raw_load_v(const AttnArgs& a, const Task& t, const RawTask& r,
                                           int head, int t0, int end, int g, int n, int w,
                                           uint2 (&vq)[8], int (&pos)[8], bool (&live)[8]) {
  const uint16_t* vp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    vp[e] = raw_token(a, t, r, head, t0 + tau(g, e), end, 1, pos[e]);
    live[e] = vp[e] != nullptr;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    vq[e] = vp[e] ? *reinterpret_cast<const uint2*>(vp[e] + 16 * n + 4 * w) : make_uint2(0u, 0u);
}

struct RawBlock {
  u32x4 kd[2][8];
  uint2 vq[8];
  int pos[8];
  bool live[8];
};

// Task, query rows and block range of one BF16-branch workgroup (task, kv head, split).
template <int RT>
struct RawSetup {
  Task t;
  RawTask r;
  int begin, end;
  u32x4 qb[RT][8];  // unrotated query as B operand of S^T = K Q^T: k-step m, d = 64 g + 8 m ..
  int qi_row[RT];
  int row0 = 0;  // the task's first row of this workgroup's row tiles
};

// The unrotated query rows of the workgroup's row tiles (lane (n, g): row n + 16 rt, dims
// 64 g .. 64 g + 63), zeros for rows that are not live.
template <int RT>
__device__ __forceinline__ void raw_load_query(const AttnArgs& a, int head, int n, int g,
                                               RawSetup<RT>& s) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const RowInfo ri = row_info(a, s.t, head, s.row0 + n + 16 * rt);
    s.qi_row[rt] = ri.qi;
#pragma unroll
    for (int m = 0; m < 8; ++m) s.qb[rt][m] = u32x4{0u, 0u, 0u, 0u};
    if (ri.valid) {
      const uint16_t* qp = a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 64 * g;
#pragma unroll
      for (int m = 0; m < 8; ++m) s.qb[rt][m] = *reinterpret_cast<const u32x4*>(qp + 8 * m);
    }
  }
}

// kQuery false: the query rows are left to the caller (raw_load_query).
template <int RT, bool kQuery = true>
__device__ __forceinline__ bool raw_setup(const AttnArgs& a, int task, int head, int split,
                                          int n, int g, RawSetup<RT>& s) {
  if (!read_task(a, s.t, task)) return false;
  const Task& t = s.t;
  // The owner page (block-table column 0) is requested together with the request's
  // metadata rows: both depend only on the task row.
  const int first = a.table_columns > 0 ? a.table[static_cast<int64_t>(t.req) * a.table_stride]
                                        : -1;
  s.r.high = t.sink_len + t.prefix - t.recent_begin;
  s.r.win = -1;
  if (first >= 0) {
    const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
    s.r.win = owner * (a.L.page_bytes / 2) + static_cast<int64_t>(head) * kHeadDim;
  }
  split_range(s.r.high + t.qlen, a.block_n, a.splits, split, s.begin, s.end);
  if constexpr (kQuery) raw_load_query(a, head, n, g, s);
  return true;
}

// Everything of a block after its scores: causal / range mask, online softmax, P*V into the
// wavefront's 4 output tiles (dims 16 n + 4 w + jj).
template <int RT>
__device__ __forceinline__ void raw_block_tail(State<RT, 4>& st, const f32x4 (&sc)[RT][2],
                                               const RawSetup<RT>& s, const uint2 (&vq)[8],
                                               const int (&pos)[8], const bool (&live)[8],
                                               float scale_log2, int g) {
  bool ok[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int e = 0; e < 8; ++e) ok[rt][e] = live[e] && pos[e] <= s.t.prefix + s.qi_row[rt];
  u32x4 ap[RT];
  block_softmax(st, sc, ok, scale_log2, g, ap);
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    uint32_t vd2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vd2[e] = (jj >> 1) ? vq[e].y : vq[e].x;
    const u32x4 bv = pv_operand(vd2, jj);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) st.o[rt][jj] = mfma16x16x32(ap[rt], bv, st.o[rt][jj]);
  }
}

// Normalized rows and LSEs of the workgroup: lane (n, g) of wavefront w holds rows 4 g + v,
// dims 16 n + 4 w + jj.
template <int RT, bool kDirect>
__device__ __forceinline__ void raw_finish(const AttnArgs& a, const RawSetup<RT>& s, int head,
                                           int split, const State<RT, 4>& st, int n, int g,
                                           int wave) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float den_n = row_sum(st.psum[rt]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = s.row0 + 16 * rt + 4 * g + v;
      const float den = fmaxf(__shfl(den_n, 4 * g + v, kWave), 1.0e-30f);
      const RowInfo ri = row_info(a, s.t, head, row);
      if (!ri.valid) continue;
      const int d = 16 * n + 4 * wave;
      const float o0 = st.o[rt][0][v] / den, o1 = st.o[rt][1][v] / den;
      const float o2 = st.o[rt][2][v] / den, o3 = st.o[rt][3][v] / den;
      if constexpr (kDirect) {
        const int64_t out_row = ri.token * a.hq + ri.qhead;
        *reinterpret_cast<uint2*>(a.direct_out + out_row * kHeadDim + d) =
            make_uint2(pack_bf16x2(o0, o1), pack_bf16x2(o2, o3));
      } else {
        const int64_t orow = (ri.token * a.hq + ri.qhead) * a.splits + split;
        *reinterpret_cast<float4*>(a.partials + orow * kHeadDim + d) = make_float4(o0, o1, o2, o3);
      }
    }
    // LSE of row n (wavefront 0, lane group 0).
    if (wave == 0 && g == 0) {
      const RowInfo ri = row_info(a, s.t, head, s.row0 + n + 16 * rt);
      const float lse = row_lse(st.m[rt], den_n);
      if constexpr (kDirect) {
        if (ri.valid && a.direct_lse) a.direct_lse[ri.token * a.hq + ri.qhead] = lse;
      } else {
        if (ri.valid) a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] = lse;
      }
    }
  }
}

// One workgroup of the BF16 branch: (task, kv head, split). Wavefront w writes output dims
// 16 n + 4 w .. + 3 of every row. kDirect: the normalized rows go to a.direct_out as bf16 (and
// the LSE to a.direct_lse): the bits merge_paths gives a row whose history branch is empty.
// kLean: the block's K rows are loaded and scored before its V rows, with no prefetch (fewer
// registers); same bits.
template <int RT, bool kDirect = false, bool kLean = false>
__device__ __forceinline__ void raw_block(const AttnArgs& a, int task, int head, int split) {
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  RawSetup<RT> s;
  if (!raw_setup(a, task, head, split, n, g, s)) return;
  const Task& t = s.t;
  const RawTask& r = s.r;
  const int end = s.end;
  State<RT, 4> st;
  state_init(st);

  // The K/V rows of the next block are requested before the current block is computed
  // (kLean: none; two row tiles: none, for registers).
  constexpr bool kPrefetch = RT == 1 && !kLean;
  RawBlock cur, nxt;
  int t0 = s.begin;
  if (kPrefetch && t0 < end) {
    raw_load_k(a, t, r, head, t0, end, g, n, cur.kd);
    raw_load_v(a, t, r, head, t0, end, g, n, wave, cur.vq, cur.pos, cur.live);
  }
  for (; t0 < end; t0 += kBlock) {
    const bool more = kPrefetch && t0 + kBlock < end;
    if (more) {
      raw_load_k(a, t, r, head, t0 + kBlock, end, g, n, nxt.kd);
      raw_load_v(a, t, r, head, t0 + kBlock, end, g, n, wave, nxt.vq, nxt.pos, nxt.live);
    }
    if (!kPrefetch) raw_load_k(a, t, r, head, t0, end, g, n, cur.kd);
    if (!kPrefetch && !kLean) raw_load_v(a, t, r, head, t0, end, g, n, wave, cur.vq, cur.pos, cur.live);
    f32x4 sc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          sc[rt][tt] = mfma16x16x32(cur.kd[tt][m], s.qb[rt][m], sc[rt][tt]);
    if (kLean) raw_load_v(a, t, r, head, t0, end, g, n, wave, cur.vq, cur.pos, cur.live);
    raw_block_tail(st, sc, s, cur.vq, cur.pos, cur.live, a.scale_log2, g);
    if (more) cur = nxt;
  }
  raw_finish<RT, kDirect>(a, s, head, split, st, n, g, wave);
}

// LDS ring of the staged BF16 branch: a slot holds one 32-token block, K rows then V rows
// (16 KiB each). K row i (token t0 + i) at 512 i with its 16-byte piece p at slot p ^ (i & 7),
// so that the eight lanes of a 128-bit read group (rows n .. n + 7, one piece) fall on eight
// different bank quads; V row i at 16 KiB + 512 i, plain.
constexpr int kRawHalfBytes = kBlock * kHeadDim * 2;
constexpr int kRawSlotBytes = 2 * kRawHalfBytes;
// After the slots: each slot's 32 row positions (INT_MAX for a row without a token).
constexpr int kRawPosBytes = kBlock * 4;
constexpr int kRawLdsPerSlot = kRawSlotBytes + kRawPosBytes;
// Slots where the launch has the LDS to spare (4 x 32 KiB).
constexpr int kRawSlots = 4;

// DMA of block t0's K and V rows into `slot`: 2 x 16 KiB, 4 x 1 KiB per wavefront each.
// Lane l resolves row l % 32 once (raw_row) and the DMA lanes fetch their rows' pointers
// from it; lanes 0..31 of wavefront 0 also store the rows' positions at `pos_table`. Every
// lane issues (a row without a token copies the query row; its score and P are masked and
// its V operand is replaced by zeros), so every wavefront counts 8 loads per block.
__device__ __forceinline__ void raw_stage_block(const AttnArgs& a, const Task& t,
                                                const RawTask& r, int head, int t0, int end,
                                                int wave, int lane, uint32_t slot,
                                                int* pos_table) {
  const uint16_t *kp, *vp;
  const int row_pos = raw_row(a, t, r, head, t0 + (lane & 31), end, kp, vp);
  if (wave == 0 && lane < 32) pos_table[lane] = row_pos;
  kp = kp ? kp : a.query;
  vp = vp ? vp : a.query;
  // All eight sources first (the shuffles complete together), then the eight DMAs.
  const uint16_t* src[8];
  const int piece = lane & 31;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 2 * (4 * i + wave) + (lane >> 5);
    src[2 * i] = shfl_ptr(kp, row) + 8 * (piece ^ (row & 7));
    src[2 * i + 1] = shfl_ptr(vp, row) + 8 * piece;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int seg = 4 * i + wave;
    dma_dwordx4(src[2 * i], slot + 1024 * seg);
    dma_dwordx4(src[2 * i + 1], slot + kRawHalfBytes + 1024 * seg);
  }
}

// Wait until at most `ahead` blocks (8 loads each) of this wavefront are still in flight
// and its LDS stores (the position tables) are done, then meet the workgroup: every
// wavefront's share of the oldest block has landed.
__device__ __forceinline__ void raw_wait_blocks(int ahead) {
  switch (ahead) {
    case 0: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
  }
}

// The BF16 branch with each block's K and V rows staged in an LDS ring of `slots` (<= 4)
// slots by DMA, up to `slots` blocks in flight. The arithmetic is raw_block's, block for
// block: the same bits. The block loop is not unrolled: a launch runs this code cold, so its
// size, not its instruction count, sets the time of the first block. Every thread of the
// workgroup calls this; `lds` holds slots x kRawLdsPerSlot bytes. `row0`: the task's first row
// of the workgroup's RT row tiles (a task of more rows can be served 16 rows at a time: a row's
// bits do not depend on the rows beside it).
template <int RT, bool kDirect = false>
__device__ __forceinline__ void raw_block_staged(const AttnArgs& a, int task, int head, int split,
                                                 uint8_t* lds, int slots, int row0 = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  RawSetup<RT> s;
  if (!raw_setup<RT, false>(a, task, head, split, n, g, s)) return;
  s.row0 = row0;
  State<RT, 4> st;
  state_init(st);
  const uint32_t base = lds_addr(lds);
  int* pos_tables = reinterpret_cast<int*>(lds + kRawSlotBytes * slots);
  const int nblk = s.begin < s.end ? cdiv(s.end - s.begin, kBlock) : 0;
  int issued = 0;
  // Top the ring up (all slots at the first block, then the slot block b - 1 freed).
  auto top_up = [&](int b) {
#pragma unroll 1
    for (; issued < nblk && issued < b + slots; ++issued)
      raw_stage_block(a, s.t, s.r, head, s.begin + kBlock * issued, s.end, wave, lane,
                      base + kRawSlotBytes * (issued % slots),
                      pos_tables + kBlock * (issued % slots));
  };
  top_up(0);
  // The query rows are requested after the first blocks and consumed here, before the block
  // loop: the compiler counts only its own loads, so a wait for them placed inside the loop
  // would also wait for the DMA of later blocks; here it waits for the blocks in flight,
  // which landed about when the rows did.
  raw_load_query(a, head, n, g, s);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int m = 0; m < 8; ++m) asm volatile("" ::"v"(s.qb[rt][m]));
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    top_up(b);
    raw_wait_blocks(issued - b - 1);
    const uint8_t* slot = lds + kRawSlotBytes * (b % slots);
    f32x4 sc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const u32x4 kd = *reinterpret_cast<const u32x4*>(
            slot + (16 * tt + n) * 512 + 16 * ((8 * g + m) ^ (n & 7)));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[rt][tt] = mfma16x16x32(kd, s.qb[rt][m], sc[rt][tt]);
      }
    // Positions of the lane's eight tokens (4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3) from
    // the slot's table; INT_MAX marks a row without a token, which fails every mask as
    // raw_block's `live` does.
    const int* table = pos_tables + kBlock * (b % slots);
    const int4 p_lo = *reinterpret_cast<const int4*>(table + 4 * g);
    const int4 p_hi = *reinterpret_cast<const int4*>(table + 16 + 4 * g);
    const int pos[8] = {p_lo.x, p_lo.y, p_lo.z, p_lo.w, p_hi.x, p_hi.y, p_hi.z, p_hi.w};
    bool live[8];
    uint2 vq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = tau(g, e);
      live[e] = pos[e] != 0x7fffffff;
      const uint2 v = *reinterpret_cast<const uint2*>(slot + kRawHalfBytes + tok * 512 +
                                                      32 * n + 8 * wave);
      vq[e] = live[e] ? v : make_uint2(0u, 0u);
    }
    raw_block_tail(st, sc, s, vq, pos, live, a.scale_log2, g);
    if (issued < nblk) barrier_lds();  // every wavefront has read the slot refilled next
  }
  raw_finish<RT, kDirect>(a, s, head, split, st, n, g, wave);
}

}  // namespace oscar
