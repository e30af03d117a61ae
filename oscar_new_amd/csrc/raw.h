// The BF16 branch of the split-KV attention (sink, recent ring and current tokens), shared by
// the attention_partials entry point and the fused pre-attention kernel.
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel` with IS_RAW true: raw
// positions = sink + recent window + causal current tokens, kernels.py:421-470).
//
// MI355X design: a workgroup is 4 independent wavefronts on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16); each owns every 4th 32-token block of the split and keeps its
// own online-softmax state, merged once through LDS at the end. Scores are computed
// transposed (S^T = K Q^T), so the MFMA output layout (lane holds 4 consecutive tokens of
// one query row) is the A-operand layout of the P*V MFMA with no shuffle in between.
#pragma once

#include "attention.h"

namespace oscar {

constexpr float kRescale = 8.0f;  // lazy-max slack, log2 units
constexpr int kBlock = 32;        // tokens per wavefront iteration

// Per-lane token of element e of the PV k-group g: 4 consecutive tokens of each 16-token
// QK tile, matching the transposed-score output layout.
__device__ __forceinline__ int tau(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

// ---------------------------------------------------------------- softmax state

template <int RT>
struct State {
  float m[RT];      // running max (log2 units) of query row n + 16 rt
  float psum[RT];   // sum p over this lane's tokens
  f32x4 o[RT][16];  // PV accumulators: tile j holds dims 16n + j
};

template <int RT>
__device__ __forceinline__ void state_init(State<RT>& st) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st.m[rt] = -INFINITY;
    st.psum[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) st.o[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// Lazy running max. Each lane first checks its own 8 scores against m + 2^8 (no cross-lane
// traffic); only if some lane of the wavefront sees a larger score is the row max reduced
// across the 4 lane groups and the accumulators rescaled. Between updates p <= 2^8.
template <int RT, int kTiles>
__device__ __forceinline__ void update_max(State<RT>& st, const float (&s2)[RT][8], int g) {
  float lm[RT];
  bool need = false;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float v = s2[rt][0];
#pragma unroll
    for (int e = 1; e < 8; ++e) v = fmaxf(v, s2[rt][e]);
    lm[rt] = v;
    need |= v > st.m[rt] + kRescale;
  }
  if (__any(need)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v = lm[rt];
      v = fmaxf(v, __shfl_xor(v, 16, kWave));
      v = fmaxf(v, __shfl_xor(v, 32, kWave));
      const float mn = fmaxf(st.m[rt], v);
      const float alpha = mn == -INFINITY ? 1.0f : exp2f(st.m[rt] - mn);
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
}

// ---------------------------------------------------------------- epilogue

// Merge the 4 wavefront states through LDS and write normalized partials + LSE: per row tile,
// every wavefront publishes its scaled accumulators at once, then each thread sums one
// (row, 16 dims) over the four wavefronts in wavefront order.
template <int RT>
constexpr int finish_lds_bytes() {
  return 4 * 16 * kHeadDim * 4 + (2 * 4 + 3) * RT * 16 * 4;
}

// kDirect: the normalized rows go to a.direct_out as bf16 (and the LSE to a.direct_lse): the
// bits merge_paths gives a row whose history branch is empty.
template <int RT, bool kDirect = false>
__device__ void finish(const AttnArgs& a, const Task& t, int head, int split, State<RT>& st,
                       uint8_t* lds) {
  typedef float OutWave[16][kHeadDim];
  OutWave* s_o = reinterpret_cast<OutWave*>(lds);
  typedef float StatWave[RT * 16];
  StatWave* s_m = reinterpret_cast<StatWave*>(lds + 4 * 16 * kHeadDim * 4);
  StatWave* s_p = s_m + 4;
  float* s_max = reinterpret_cast<float*>(s_p + 4);
  float* s_den = s_max + RT * 16;
  float* s_lse = s_den + RT * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st.psum[rt] += __shfl_xor(st.psum[rt], 16, kWave);
    st.psum[rt] += __shfl_xor(st.psum[rt], 32, kWave);
    if (g == 0) {
      s_m[wave][n + 16 * rt] = st.m[rt];
      s_p[wave][n + 16 * rt] = st.psum[rt];
    }
  }
  __syncthreads();
  if (threadIdx.x < RT * 16) {
    const int row = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_m[w][row]);
    float den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (s_m[w][row] != -INFINITY) den += exp2f(s_m[w][row] - mx) * s_p[w][row];
    s_max[row] = mx;
    s_den[row] = den;
    s_lse[row] = den > 0.f ? (mx + log2f(den)) * kLn2 : -INFINITY;
  }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (rt > 0) __syncthreads();  // the previous tile's sums have been read
    // Lane (g, n) holds dims 16n + tile of rows 4g + v.
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * rt + 4 * g + v;
      const float mw = s_m[wave][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - s_max[row]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<f32x4*>(&s_o[wave][4 * g + v][16 * n + 4 * c]) =
            f32x4{st.o[rt][4 * c][v] * f, st.o[rt][4 * c + 1][v] * f, st.o[rt][4 * c + 2][v] * f,
                  st.o[rt][4 * c + 3][v] * f};
    }
    __syncthreads();
    const int row16 = threadIdx.x >> 4, dq = threadIdx.x & 15;
    const int row = 16 * rt + row16;
    const RowInfo ri = row_info(a, t, head, row);
    if (ri.valid) {
      const float den = fmaxf(s_den[row], 1.0e-30f);
      const int64_t orow = (ri.token * a.hq + ri.qhead) * a.splits + split;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = 16 * dq + 4 * c;
        const f32x4 sum = *reinterpret_cast<const f32x4*>(&s_o[0][row16][d]) +
                          *reinterpret_cast<const f32x4*>(&s_o[1][row16][d]) +
                          *reinterpret_cast<const f32x4*>(&s_o[2][row16][d]) +
                          *reinterpret_cast<const f32x4*>(&s_o[3][row16][d]);
        if constexpr (kDirect) {
          const int64_t out_row = ri.token * a.hq + ri.qhead;
          *reinterpret_cast<uint2*>(a.direct_out + out_row * kHeadDim + d) =
              make_uint2(pack_bf16x2(sum[0] / den, sum[1] / den),
                         pack_bf16x2(sum[2] / den, sum[3] / den));
        } else {
          *reinterpret_cast<float4*>(a.partials + orow * kHeadDim + d) =
              make_float4(sum[0] / den, sum[1] / den, sum[2] / den, sum[3] / den);
        }
      }
    }
  }
  if (threadIdx.x < RT * 16) {
    const RowInfo ri = row_info(a, t, head, threadIdx.x);
    if constexpr (kDirect) {
      if (ri.valid && a.direct_lse) a.direct_lse[ri.token * a.hq + ri.qhead] = s_lse[threadIdx.x];
    } else {
      if (ri.valid) a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] = s_lse[threadIdx.x];
    }
  }
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

// K rows of the block's two 16-token score tiles (A operands) and V rows of this lane's eight
// tokens (B operands of P*V), with the positions that mask them.
struct RawBlock {
  u32x4 kd[2][8];
  u32x4 vd[8][2];
  int pos[8];
  bool live[8];
};

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

__device__ __forceinline__ void raw_load_v(const AttnArgs& a, const Task& t, const RawTask& r,
                                           int head, int t0, int end, int g, int n,
                                           u32x4 (&vd)[8][2], int (&pos)[8], bool (&live)[8]) {
  const uint16_t* vp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    vp[e] = raw_token(a, t, r, head, t0 + tau(g, e), end, 1, pos[e]);
    live[e] = vp[e] != nullptr;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    vd[e][0] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n) : u32x4{0u, 0u, 0u, 0u};
    vd[e][1] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n + 8)
                     : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void raw_load_block(const AttnArgs& a, const Task& t, const RawTask& r,
                                               int head, int t0, int end, int g, int n,
                                               RawBlock& b) {
  raw_load_k(a, t, r, head, t0, end, g, n, b.kd);
  raw_load_v(a, t, r, head, t0, end, g, n, b.vd, b.pos, b.live);
}

// One workgroup of the BF16 branch: (task, kv head, split).
// `smem`: finish_lds_bytes<RT>() bytes of 16-byte aligned LDS. kLean: the block's K rows are
// loaded, scored, and only then its V rows (no prefetch; fewer registers, for a workgroup
// role inside a launch whose other roles need two workgroups per CU). Same arithmetic, same
// bits as the prefetching form.
template <int RT, bool kDirect = false, bool kLean = false>
__device__ __forceinline__ void raw_block(const AttnArgs& a, int task, int head, int split,
                                          uint8_t* smem) {
  Task t;
  if (!read_task(a, t, task)) return;
  // The owner page (block-table column 0) is requested together with the request's
  // metadata rows: both depend only on the task row.
  const int first = a.table_columns > 0 ? a.table[static_cast<int64_t>(t.req) * a.table_stride]
                                        : -1;
  RawTask r;
  r.high = t.sink_len + t.prefix - t.recent_begin;
  r.win = -1;
  if (first >= 0) {
    const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
    r.win = owner * (a.L.page_bytes / 2) + static_cast<int64_t>(head) * kHeadDim;
  }
  int begin, end;
  split_range(r.high + t.qlen, a.block_n, a.splits, split, begin, end);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;

  // Unrotated query as B operand of S^T = K Q^T; k-step m covers d = 64g + 8m .. +7.
  u32x4 qb[RT][8];
  int qi_row[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const RowInfo ri = row_info(a, t, head, n + 16 * rt);
    qi_row[rt] = ri.qi;
#pragma unroll
    for (int m = 0; m < 8; ++m) qb[rt][m] = u32x4{0u, 0u, 0u, 0u};
    if (ri.valid) {
      const uint16_t* qp = a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 64 * g;
#pragma unroll
      for (int m = 0; m < 8; ++m) qb[rt][m] = *reinterpret_cast<const u32x4*>(qp + 8 * m);
    }
  }
  State<RT> st;
  state_init(st);

  // A wavefront's blocks are t0 = begin + 32 w, + 128, ...; the K/V rows of the next block
  // are requested before the current block is computed, so a wavefront with two blocks (a
  // decode step's 133 BF16 tokens over four wavefronts) still waits one memory round trip.
  // (Two row tiles (RT = 2) leave no registers for the second block: loaded in turn.)
  constexpr bool kPrefetch = RT == 1 && !kLean;
  RawBlock cur, nxt;
  int t0 = begin + kBlock * wave;
  if (kPrefetch && t0 < end) raw_load_block(a, t, r, head, t0, end, g, n, cur);
  for (; t0 < end; t0 += 4 * kBlock) {
    const bool more = kPrefetch && t0 + 4 * kBlock < end;
    if (more) raw_load_block(a, t, r, head, t0 + 4 * kBlock, end, g, n, nxt);
    if (!kPrefetch && !kLean) raw_load_block(a, t, r, head, t0, end, g, n, cur);
    if (kLean) raw_load_k(a, t, r, head, t0, end, g, n, cur.kd);
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
          sc[rt][tt] = mfma16x16x32(cur.kd[tt][m], qb[rt][m], sc[rt][tt]);
    if (kLean) raw_load_v(a, t, r, head, t0, end, g, n, cur.vd, cur.pos, cur.live);
    float s2[RT][8];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool ok = cur.live[e] && cur.pos[e] <= t.prefix + qi_row[rt];
        s2[rt][e] = ok ? sc[rt][e >> 2][e & 3] * a.scale_log2 : -INFINITY;
      }
    update_max<RT, 16>(st, s2, g);
    u32x4 ap[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = s2[rt][e] == -INFINITY ? 0.f : exp2f(s2[rt][e] - st.m[rt]);
        st.psum[rt] += p[e];
      }
#pragma unroll
      for (int f = 0; f < 4; ++f) ap[rt][f] = pack_bf16x2(p[2 * f], p[2 * f + 1]);
    }
#pragma unroll
    for (int tile = 0; tile < 16; ++tile) {
      const uint32_t sel = (tile & 1) ? 0x07060302u : 0x05040100u;
      u32x4 bv;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        bv[f] = __builtin_amdgcn_perm(cur.vd[2 * f + 1][tile >> 3][(tile & 7) >> 1],
                                      cur.vd[2 * f][tile >> 3][(tile & 7) >> 1], sel);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st.o[rt][tile] = mfma16x16x32(ap[rt], bv, st.o[rt][tile]);
    }
    if (more) cur = nxt;
  }
  finish<RT, kDirect>(a, t, head, split, st, smem);
}

}  // namespace oscar
