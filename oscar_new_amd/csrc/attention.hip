// Split-KV paged decode attention over the INT2 history and the BF16 sink/ring/current
// window, on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel`, `attention_partials`).
// Semantics kept: one workgroup per (task, kv head, split); history positions
// [min(S, prefix), max(sink_len, prefix - R)); raw positions sink + recent window + causal
// current tokens; per-split normalized output and natural-log LSE; live rows of an empty
// split get 0 / -inf; inactive programs write nothing.
//
// MI355X design (not a translation of the Triton tiling):
//   * a workgroup is 4 independent wavefronts; each owns every 4th aligned 32-token block
//     of the split and keeps its own online-softmax state, so the KV loop has no barrier.
//     The four states are merged once, through LDS, at the end;
//   * scores are computed transposed (S^T = K Q^T): the MFMA output layout (lane holds 4
//     consecutive tokens of one query row) is then exactly the A-operand layout of the
//     P*V MFMA -- no cross-lane shuffle between the two products;
//   * INT2 history is never dequantized element-wise. A 2-bit code c placed in the mantissa
//     of a bf16 with exponent 2^7 is the exact value 128 + 4^s c (s = field position), so
//     one AND+OR turns packed codes into MFMA operands. Scale and zero are folded out:
//     q.k = s_k (q.c) + z_k sum(q);  sum_t p_t v_t = sum_t (p_t s_v) c_t + sum_t p_t z_v.
//     The 128 offsets are cancelled by an MFMA accumulator initialisation (QK) and by an
//     extra MFMA against a constant-128 operand (PV);
//   * the softmax maximum is updated lazily (only when a block raises it by > 2^8), so the
//     common block does no accumulator rescaling;
//   * each wavefront issues the loads of its next block before computing the current one.
#include "common.h"

namespace oscar {
namespace {

constexpr uint32_t kMagic = 0x43004300u;  // bf16 pair (128, 128)
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescale = 8.0f;  // log2 units
constexpr int kSlot = 160, kVector = 68;
constexpr int kBlock = 32;  // tokens per wavefront iteration

struct AttnArgs {
  const uint16_t* query;
  int64_t qs0, qs1;
  const uint16_t* key;
  int64_t ks0, ks1;
  const uint16_t* value;
  int64_t vs0, vs1;
  const uint8_t* history;
  int64_t history_bytes;
  const uint16_t* window;
  int64_t window_elems;
  const int32_t* qstarts;
  const int32_t* seq_lens;
  const int32_t* table;
  int64_t table_stride, table_columns;
  const int32_t* counts;
  const int32_t* tasks;
  const int32_t* task_count;
  float* partials;
  float* lse;
  int64_t n;
  Layout L;
  int32_t g, hq, qt, splits, block_n;
  float scale_log2;
  uint32_t mask[3];  // 0x00030003 << 2s, s = 0..2: code-field masks (see and_or)
};

struct Task {
  int req, qoff, qstart, qlen, prefix, sink_len, recent_begin;
};

__device__ __forceinline__ bool read_task(const AttnArgs& a, Task& t) {
  const int task = blockIdx.x;
  if (task >= a.task_count[0]) return false;
  t.req = a.tasks[2 * task];
  t.qoff = a.tasks[2 * task + 1];
  t.qstart = a.qstarts[t.req];
  const int qend = min(a.qstarts[t.req + 1], a.counts[1]);
  t.qlen = qend - t.qstart;
  t.prefix = a.seq_lens[t.req] - t.qlen;
  t.sink_len = min(a.L.sink, t.prefix);
  t.recent_begin = max(t.sink_len, t.prefix - a.L.recent);
  return true;
}

// kernels.py:368-370: every split covers ceil(ceil(len / BN) / splits) tiles of BN tokens.
__device__ __forceinline__ void split_range(int length, int block_n, int splits, int split,
                                            int& begin, int& end) {
  length = max(length, 0);
  const int per = cdiv(cdiv(length, block_n), splits);
  begin = split * per * block_n;
  end = min((split + 1) * per * block_n, length);
}

struct RowInfo {
  bool valid;
  int qi, qhead;
  int64_t token;
};

__device__ __forceinline__ RowInfo row_info(const AttnArgs& a, const Task& t, int head, int row) {
  RowInfo r;
  r.qi = t.qoff + row / a.g;
  r.token = static_cast<int64_t>(t.qstart) + r.qi;
  r.valid = row < a.qt * a.g && r.qi < t.qlen && r.token >= 0 && r.token < a.n;
  r.qhead = head * a.g + row % a.g;
  return r;
}

__device__ __forceinline__ uint32_t half16(const u32x4 (&raw)[8], int x) {
  return (raw[x >> 3][(x & 7) >> 1] >> (16 * (x & 1))) & 0xffffu;
}

// Per-lane token of element e of the PV k-group g: 4 consecutive tokens of each 16-token
// QK tile, matching the transposed-score output layout.
__device__ __forceinline__ int tau(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

// Scale of code field j' (0..7) inside a magic bf16 pair: 4^(j' % 3).
__device__ __forceinline__ float field_scale_inv(int jp) {
  const int s = jp % 3;
  return s == 0 ? 1.0f : (s == 1 ? 0.25f : 0.0625f);
}

// (a & mask) | magic in ONE v_and_or_b32. gfx9 VOP3 reads at most one scalar or literal
// operand, so the masks arrive as kernel arguments (SGPRs, see AttnArgs::mask) and magic is
// a VGPR the compiler cannot fold (opaque_magic). Plain C, not asm: VALU results feeding
// MFMA operands must stay visible to the compiler's hazard tracking.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  return (a & mask) | magic;
}

__device__ __forceinline__ uint32_t opaque_magic() {
  return static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(kMagic), 0xe4, 0xf, 0xf, false));
}

// One 16-code K dword -> the A operands of two consecutive k-steps (8 bf16 each).
// D-dword j' holds (128 + 4^s c_{j'}, 128 + 4^s c_{8+j'}), s = j' % 3.
__device__ __forceinline__ void codes_to_steps(uint32_t w, const uint32_t (&mk)[3],
                                               uint32_t magic, u32x4& s0, u32x4& s1) {
  const uint32_t w6 = w >> 6, w12 = w >> 12;
  s0[0] = and_or(w, mk[0], magic);
  s0[1] = and_or(w, mk[1], magic);
  s0[2] = and_or(w, mk[2], magic);
  s0[3] = and_or(w6, mk[0], magic);
  s1[0] = and_or(w6, mk[1], magic);
  s1[1] = and_or(w6, mk[2], magic);
  s1[2] = and_or(w12, mk[0], magic);
  s1[3] = and_or(w12, mk[1], magic);
}

__device__ __forceinline__ float h16(_Float16 h) { return static_cast<float>(h); }
__device__ __forceinline__ _Float16 lo16(uint32_t x) {
  return __builtin_bit_cast(_Float16, static_cast<uint16_t>(x & 0xffffu));
}
__device__ __forceinline__ _Float16 hi16(uint32_t x) {
  return __builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> 16));
}

// ---------------------------------------------------------------- softmax state

template <int RT>
struct State {
  float m[RT];      // running max (log2 units) of query row n + 16 rt
  float psum[RT];   // sum p over this lane's tokens
  float zsum[RT];   // sum p * z_v over this lane's tokens (history only)
  f32x4 o[RT][17];  // PV accumulators (tile 16: sum p s_v * 128, history only)
};

template <int RT>
__device__ __forceinline__ void state_init(State<RT>& st) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st.m[rt] = -INFINITY;
    st.psum[rt] = 0.f;
    st.zsum[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < 17; ++t) st.o[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
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
      st.zsum[rt] *= alpha;
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

// Merge the 4 wavefront states through LDS and write normalized partials + LSE.
// LDS bytes finish() needs for RT row tiles.
template <int RT>
constexpr int finish_lds_bytes() {
  return 4 * RT * 16 * 16 * 16 + (3 * 4 + 3) * RT * 16 * 4;
}

template <int RT, bool kHist>
__device__ void finish(const AttnArgs& a, const Task& t, int head, int split, State<RT>& st,
                       uint8_t* lds) {
  typedef f32x4 RedRow[16];
  typedef RedRow RedWave[RT * 16];
  RedWave* s_red = reinterpret_cast<RedWave*>(lds);
  typedef float StatWave[RT * 16];
  StatWave* s_m = reinterpret_cast<StatWave*>(lds + 4 * RT * 16 * 16 * 16);
  StatWave* s_p = s_m + 4;
  StatWave* s_z = s_p + 4;
  float* s_max = reinterpret_cast<float*>(s_z + 4);
  float* s_den = s_max + RT * 16;
  float* s_lse = s_den + RT * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st.psum[rt] += __shfl_xor(st.psum[rt], 16, kWave);
    st.psum[rt] += __shfl_xor(st.psum[rt], 32, kWave);
    st.zsum[rt] += __shfl_xor(st.zsum[rt], 16, kWave);
    st.zsum[rt] += __shfl_xor(st.zsum[rt], 32, kWave);
    if (g == 0) {
      s_m[wave][n + 16 * rt] = st.m[rt];
      s_p[wave][n + 16 * rt] = st.psum[rt];
      s_z[wave][n + 16 * rt] = st.zsum[rt];
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
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * rt + 4 * g + v;
      const float mw = s_m[wave][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - s_max[row]);
      if (kHist) {
        const float zs = s_z[wave][row];
        const float w128 = st.o[rt][16][v];
#pragma unroll
        for (int tt = 0; tt < 16; ++tt)
          st.o[rt][tt][v] = ((st.o[rt][tt][v] - w128) * field_scale_inv(tt & 7) + zs) * f;
      } else {
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) st.o[rt][tt][v] *= f;
      }
    }
  }
  // Lane (g, n) holds dims 16n + tile; chunk c gathers tiles 4c..4c+3 of every wavefront.
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        s_red[wave][16 * rt + 4 * g + v][n] =
            f32x4{st.o[rt][4 * c][v], st.o[rt][4 * c + 1][v], st.o[rt][4 * c + 2][v],
                  st.o[rt][4 * c + 3][v]};
    __syncthreads();
    for (int idx = threadIdx.x; idx < RT * 16 * 16; idx += kThreads) {
      const int row = idx >> 4, nn = idx & 15;
      const RowInfo ri = row_info(a, t, head, row);
      if (ri.valid) {
        const f32x4 sum = s_red[0][row][nn] + s_red[1][row][nn] + s_red[2][row][nn] +
                          s_red[3][row][nn];
        const float den = fmaxf(s_den[row], 1.0e-30f);
        const int64_t orow = (ri.token * a.hq + ri.qhead) * a.splits + split;
        *reinterpret_cast<float4*>(a.partials + orow * kHeadDim + 16 * nn + 4 * c) =
            make_float4(sum[0] / den, sum[1] / den, sum[2] / den, sum[3] / den);
      }
    }
    __syncthreads();
  }
  if (threadIdx.x < RT * 16) {
    const RowInfo ri = row_info(a, t, head, threadIdx.x);
    if (ri.valid) a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] = s_lse[threadIdx.x];
  }
}

// ---------------------------------------------------------------- history branch

// Per-wavefront LDS pipeline: kStages buffers of one 32-token block each (32 x 160-byte
// records, compact). One query row tile (decode): 3 stages, 2 workgroups per CU. Two row
// tiles (MTP verification, more registers, 1 workgroup per CU): 5 stages. Blocks arrive by direct-to-LDS DMA (global_load_lds_dwordx4), five
// 16-byte loads per lane per block, so staging costs no VGPRs. kStages - 1 blocks are in
// flight while the wavefront computes the oldest one.
constexpr int kBlockBytes = kBlock * kSlot;      // 5120
constexpr int kDmaPerBlock = kBlockBytes / 1024;  // 16 B x 64 lanes per instruction

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One 16-byte-per-lane direct-to-LDS load: lane l writes LDS bytes [lds + 16 l, +16).
// Issued through asm so the compiler does not serialize every later LDS read behind all
// outstanding DMA (it cannot tell pipeline stages apart); ordering is by the explicit
// vmcnt waits below. M0 holds the LDS base; one wait state separates its write from the DMA.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "{m0}"(lds_addr), "v"(src)
               : "memory");
}

// LDS DMA is issued by asm (see dma16), so waits are explicit.
#define OSCAR_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")
#define OSCAR_WAIT_LDS() asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory")

// The byte offsets of the kernel blocks a workgroup reads (in 32-byte units, or kNoBlock)
// are resolved once, into LDS, by the whole workgroup. The KV loop then reads one LDS word
// per block: no vector-memory load whose wait would also drain the in-flight LDS DMA, and
// little scalar arithmetic.
constexpr int kTableCache = 2048;  // kernel blocks (262144 tokens at 128 per block)
constexpr uint32_t kNoBlock = 0xffffffffu;

typedef __attribute__((address_space(3))) const uint32_t* lds_u32_ptr_t;

// Offset (32-byte units) of kernel block kb of this request/head, or kNoBlock.
__device__ __forceinline__ uint32_t kernel_block_offset(const AttnArgs& a, const Task& t, int head,
                                                        int kb) {
  if (kb < 0 || kb >= a.table_columns) return kNoBlock;
  const int blk = a.table[static_cast<int64_t>(t.req) * a.table_stride + kb];
  if (blk < 0) return kNoBlock;
  const uint32_t page = fastdiv(static_cast<uint32_t>(blk), a.L.bpp_div);
  const uint32_t inpage = static_cast<uint32_t>(blk) - page * a.L.bpp;
  const int64_t off = static_cast<int64_t>(page) * a.L.page_bytes +
                      (static_cast<int64_t>(inpage) * a.L.bk * a.L.kv_heads + head) * kSlot;
  // The whole kernel block must lie inside the history buffer.
  if (off + static_cast<int64_t>(a.L.bk) * a.L.kv_heads * kSlot > a.history_bytes) return kNoBlock;
  return static_cast<uint32_t>(off >> 5);
}

template <int RT>
__device__ __forceinline__ void hist_compute(const AttnArgs& a, const uint8_t* blk, int t0,
                                             int p_lo, int p_hi, int n, int g,
                                             const uint32_t (&mk)[3], uint32_t magic,
                                             const u32x4 (&qb)[RT][8], const float (&corr)[RT],
                                             const float (&qsum)[RT], State<RT>& st) {
  // S^T tiles (tokens 0-15, 16-31): the two MFMA chains alternate so that every dependent
  // accumulation has an independent MFMA between it and its predecessor.
  const u32x4 kc0 = *reinterpret_cast<const u32x4*>(blk + n * kSlot + 16 * g);
  const u32x4 kc1 = *reinterpret_cast<const u32x4*>(blk + (16 + n) * kSlot + 16 * g);
  f32x4 sc[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) sc[rt][tt] = f32x4{-corr[rt], -corr[rt], -corr[rt], -corr[rt]};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    u32x4 a0, a1, b0, b1;
    codes_to_steps(kc0[w], mk, magic, a0, a1);
    codes_to_steps(kc1[w], mk, magic, b0, b1);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      sc[rt][0] = mfma16x16x32(a0, qb[rt][2 * w], sc[rt][0]);
      sc[rt][1] = mfma16x16x32(b0, qb[rt][2 * w], sc[rt][1]);
      sc[rt][0] = mfma16x16x32(a1, qb[rt][2 * w + 1], sc[rt][0]);
      sc[rt][1] = mfma16x16x32(b1, qb[rt][2 * w + 1], sc[rt][1]);
    }
  }
  // Records of this lane's 8 tokens tau(g, 0..7): one base, constant offsets.
  const uint8_t* rec = blk + 4 * g * kSlot;
  uint32_t ksz[8], vsz[8], vc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int off = (e < 4 ? e : 12 + e) * kSlot;
    ksz[e] = *reinterpret_cast<const uint32_t*>(rec + off + 64);
    vsz[e] = *reinterpret_cast<const uint32_t*>(rec + off + kVector + 64);
    vc[e] = *reinterpret_cast<const uint32_t*>(rec + off + kVector + 4 * n);
  }
  // Only the first/last block of a split is partial. There, tokens outside [p_lo, p_hi)
  // get score -inf (p = 0 exactly: every block overlaps the split, so the running max is
  // finite) and zeroed V scale/zero (their bytes may hold NaN patterns).
  const bool full = t0 >= p_lo && t0 + kBlock <= p_hi;
  uint32_t okmask = 0xffu;
  if (!full) {
    okmask = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool ok = static_cast<uint32_t>(t0 + tau(g, e) - p_lo) <
                      static_cast<uint32_t>(p_hi - p_lo);
      okmask |= ok ? (1u << e) : 0u;
      vsz[e] = ok ? vsz[e] : 0u;
    }
  }
  // Scores in log2 units: (s_k (q.c) + z_k sum(q)) * scale * log2(e).
  float s2[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float qs = qsum[rt] * a.scale_log2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float qc = sc[rt][e >> 2][e & 3] * a.scale_log2;
      s2[rt][e] = fmaf(h16(lo16(ksz[e])), qc, h16(hi16(ksz[e])) * qs);
    }
  }
  if (!full) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 8; ++e) s2[rt][e] = (okmask >> e) & 1u ? s2[rt][e] : -INFINITY;
  }
  update_max<RT, 17>(st, s2, g);
  u32x4 aw[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = __builtin_amdgcn_exp2f(s2[rt][e] - st.m[rt]);
      st.psum[rt] += p[e];
      st.zsum[rt] = fmaf(p[e], h16(hi16(vsz[e])), st.zsum[rt]);
    }
#pragma unroll
    for (int f = 0; f < 4; ++f)
      aw[rt][f] = pack_bf16x2(p[2 * f] * h16(lo16(vsz[2 * f])),
                              p[2 * f + 1] * h16(lo16(vsz[2 * f + 1])));
  }
  u32x4 zlo, zhi;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    zlo[f] = __builtin_amdgcn_perm(vc[2 * f + 1], vc[2 * f], 0x05040100u);
    zhi[f] = __builtin_amdgcn_perm(vc[2 * f + 1], vc[2 * f], 0x07060302u);
  }
#pragma unroll
  for (int tile = 0; tile < 16; ++tile) {
    const int jp = tile & 7;
    const int sh = 6 * (jp / 3);
    const uint32_t mask = mk[jp % 3];
    u32x4 bv;
#pragma unroll
    for (int f = 0; f < 4; ++f) bv[f] = and_or((tile < 8 ? zlo[f] : zhi[f]) >> sh, mask, magic);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) st.o[rt][tile] = mfma16x16x32(aw[rt], bv, st.o[rt][tile]);
  }
  const u32x4 b128 = u32x4{magic, magic, magic, magic};
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) st.o[rt][16] = mfma16x16x32(aw[rt], b128, st.o[rt][16]);
}

// Rotated query as the B operand of S^T = K Q^T, in the k order produced by codes_to_steps,
// each element pre-divided by its field scale 4^s; corr = 128 * sum(B), qsum = sum(q).
template <int RT>
__device__ __forceinline__ void hist_query(const AttnArgs& a, const Task& t, int head, int n,
                                           int g, u32x4 (&qb)[RT][8], float (&corr)[RT],
                                           float (&qsum)[RT]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const RowInfo ri = row_info(a, t, head, n + 16 * rt);
    u32x4 raw[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) raw[c] = u32x4{0u, 0u, 0u, 0u};
    if (ri.valid) {
      const uint16_t* qp = a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 64 * g;
#pragma unroll
      for (int c = 0; c < 8; ++c) raw[c] = *reinterpret_cast<const u32x4*>(qp + 8 * c);
    }
    float cs = 0.f, qs = 0.f;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int w = m >> 1, half = m & 1;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int jp = 4 * half + f;
        const float sc = field_scale_inv(jp);
        const float lo = bf16_to_float(half16(raw, 16 * w + jp));
        const float hi = bf16_to_float(half16(raw, 16 * w + 8 + jp));
        const float slo = lo * sc, shi = hi * sc;  // exact: power-of-two scaling
        qb[rt][m][f] = float_to_bf16(slo) | (float_to_bf16(shi) << 16);
        cs += slo + shi;
        qs += lo + hi;
      }
    }
    cs += __shfl_xor(cs, 16, kWave);
    cs += __shfl_xor(cs, 32, kWave);
    qs += __shfl_xor(qs, 16, kWave);
    qs += __shfl_xor(qs, 32, kWave);
    corr[rt] = 128.0f * cs;
    qsum[rt] = qs;
  }
}

template <int RT>
__global__ __launch_bounds__(kThreads, 3 - RT) void history_kernel(const AttnArgs a) {
  constexpr int kStages = RT == 1 ? 3 : 5;
  static_assert(4 * kStages * kBlockBytes >= finish_lds_bytes<RT>(), "epilogue LDS alias");
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * kStages * kBlockBytes];
  __shared__ uint32_t s_off[kTableCache];
  Task t;
  if (!read_task(a, t)) return;
  const int head = blockIdx.y, split = blockIdx.z;
  int begin, end;
  split_range(t.recent_begin - t.sink_len, a.block_n, a.splits, split, begin, end);
  const int p_lo = max(t.sink_len + begin, 0), p_hi = t.sink_len + end;
  const int kb_first = p_lo >> a.L.bk_shift;
  if (p_lo < p_hi) {
    const int nkb = min(((p_hi - 1) >> a.L.bk_shift) - kb_first + 1, kTableCache);
    for (int j = threadIdx.x; j < nkb; j += kThreads)
      s_off[j] = kernel_block_offset(a, t, head, kb_first + j);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;

  u32x4 qb[RT][8];
  float corr[RT], qsum[RT];
  State<RT> st;
  state_init(st);
  const uint32_t magic = opaque_magic();
  const uint32_t mk[3] = {a.mask[0], a.mask[1], a.mask[2]};

  if (p_lo >= p_hi) hist_query<RT>(a, t, head, n, g, qb, corr, qsum);
  if (p_lo < p_hi) {
    const int first = p_lo >> 5;
    const int nblk = ((p_hi - 1) >> 5) - first + 1;
    const uint32_t tok_bytes = static_cast<uint32_t>(a.L.kv_heads) * kSlot;
    // DMA piece i of this lane: 16 bytes of record c / 10, bytes 16 * (c % 10), c = 64 i + lane.
    uint32_t goff[kDmaPerBlock];
#pragma unroll
    for (int i = 0; i < kDmaPerBlock; ++i) {
      const int c = i * 64 + lane;
      goff[i] = static_cast<uint32_t>((c / 10) * tok_bytes + (c % 10) * 16);
    }
    uint8_t* wbuf = smem + wave * (kStages * kBlockBytes);
    const uint32_t wbuf_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)wbuf));
    const uint32_t in_kb_mask = static_cast<uint32_t>(a.L.bk - 1);
    int valid_mask = 0;
    // Always five loads per block (a safe in-bounds dummy block when out of range) so the
    // number of loads younger than any block is a constant: 5 * (kStages - 1).
    auto issue = [&](int ib, int stage) {
      const uint8_t* base = a.history;
      bool ok = false;
      if (ib < nblk) {
        const int t0 = (first + ib) << 5;
        const int local = (t0 >> a.L.bk_shift) - kb_first;
        uint32_t off32 = uniform(((lds_u32_ptr_t)s_off)[min(local, kTableCache - 1)]);
        if (local >= kTableCache) off32 = kernel_block_offset(a, t, head, t0 >> a.L.bk_shift);
        if (off32 != kNoBlock) {
          ok = true;
          base = a.history + (static_cast<uint64_t>(off32) << 5) +
                 (static_cast<uint32_t>(t0) & in_kb_mask) * tok_bytes;
        }
      }
      valid_mask = ok ? (valid_mask | (1 << stage)) : (valid_mask & ~(1 << stage));
      OSCAR_WAIT_LDS();
      const uint32_t lds = wbuf_lds + stage * kBlockBytes;
#pragma unroll
      for (int i = 0; i < kDmaPerBlock; ++i) dma16(base + goff[i], lds + i * 1024);
    };
#pragma unroll
    for (int k = 0; k < kStages - 1; ++k) issue(wave + 4 * k, k);
    // The query loads overlap the first blocks' DMA latency. The compiler does not see
    // the asm DMA, so its own wait for these loads cannot drain them (vmcnt counts in
    // order; it waits for the query loads, which are the youngest).
    hist_query<RT>(a, t, head, n, g, qb, corr, qsum);
    int stage = 0;
    for (int ib = wave; ib < nblk; ib += 4) {
      issue(ib + 4 * (kStages - 1), stage == 0 ? kStages - 1 : stage - 1);
      OSCAR_WAIT_VM(kDmaPerBlock * (kStages - 1));
      if (valid_mask & (1 << stage)) {
        hist_compute<RT>(a, wbuf + stage * kBlockBytes, (first + ib) << 5, p_lo, p_hi, n, g,
                         mk, magic, qb, corr, qsum, st);
      }
      stage = stage == kStages - 1 ? 0 : stage + 1;
    }
    OSCAR_WAIT_VM(0);
  }
  __syncthreads();  // the epilogue reuses the pipeline's LDS
  finish<RT, true>(a, t, head, split, st, smem);
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
  const int wi = pos < a.L.sink ? pos : a.L.sink + pos % a.L.ring;
  const int64_t off = r.win + (static_cast<int64_t>(wi) * 2 + kv) * a.L.kv_heads * kHeadDim;
  if (off + kHeadDim > a.window_elems) return nullptr;
  return a.window + off;
}

template <int RT>
__global__ __launch_bounds__(kThreads) void raw_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[finish_lds_bytes<RT>()];
  Task t;
  if (!read_task(a, t)) return;
  const int head = blockIdx.y, split = blockIdx.z;
  RawTask r;
  r.high = t.sink_len + t.prefix - t.recent_begin;
  r.win = -1;
  if (a.table_columns > 0) {
    const int first = a.table[static_cast<int64_t>(t.req) * a.table_stride];
    if (first >= 0) {
      const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
      r.win = owner * (a.L.page_bytes / 2) + static_cast<int64_t>(head) * kHeadDim;
    }
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

  for (int t0 = begin + kBlock * wave; t0 < end; t0 += 4 * kBlock) {
    f32x4 sc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      int pos;
      const uint16_t* kp = raw_token(a, t, r, head, t0 + 16 * tt + n, end, 0, pos);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const u32x4 kv = kp ? *reinterpret_cast<const u32x4*>(kp + 64 * g + 8 * m)
                            : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[rt][tt] = mfma16x16x32(kv, qb[rt][m], sc[rt][tt]);
      }
    }
    const uint16_t* vp[8];
    int pos[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vp[e] = raw_token(a, t, r, head, t0 + tau(g, e), end, 1, pos[e]);
    float s2[RT][8];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool ok = vp[e] != nullptr && pos[e] <= t.prefix + qi_row[rt];
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
    u32x4 vd[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      vd[e][0] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n) : u32x4{0u, 0u, 0u, 0u};
      vd[e][1] = vp[e] ? *reinterpret_cast<const u32x4*>(vp[e] + 16 * n + 8)
                       : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int tile = 0; tile < 16; ++tile) {
      const uint32_t sel = (tile & 1) ? 0x07060302u : 0x05040100u;
      u32x4 bv;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        bv[f] = __builtin_amdgcn_perm(vd[2 * f + 1][tile >> 3][(tile & 7) >> 1],
                                      vd[2 * f][tile >> 3][(tile & 7) >> 1], sel);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st.o[rt][tile] = mfma16x16x32(ap[rt], bv, st.o[rt][tile]);
    }
  }
  finish<RT, false>(a, t, head, split, st, smem);
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_attention_partials(
    const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* key, int64_t k_s0,
    int64_t k_s1, int64_t k_s2, const void* value, int64_t v_s0, int64_t v_s1, int64_t v_s2,
    const void* history, int64_t history_bytes, const void* window, int64_t window_elems,
    const int32_t* qstarts, const int32_t* seq_lens, const int32_t* block_tables,
    int64_t table_stride, int64_t table_columns, const int32_t* counts, const int32_t* tasks,
    const int32_t* task_count, int64_t n, int64_t hq, int64_t programs, int32_t splits,
    int32_t block_n, int32_t query_tile, int32_t max_query_len, float scale, int32_t raw,
    const oscar_layout* layout, float* partials, float* lse, void* stream) {
  using namespace oscar;
  AttnArgs a{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  const int64_t h = a.L.kv_heads;
  if (n < 0 || hq <= 0 || hq % h || programs < 1 || splits < 1 || splits > 65535 ||
      block_n < 1 || query_tile < 1 || table_columns < 0 || programs > (1ll << 31) - 1)
    return OSCAR_E_SHAPE;
  const int64_t g = hq / h;
  const int64_t qrows = (max_query_len > 0 && max_query_len < query_tile ? max_query_len
                                                                         : query_tile) * g;
  if (qrows > 32) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!query || !qstarts || !seq_lens || !block_tables || !counts || !tasks || !task_count ||
      !partials || !lse)
    return OSCAR_E_NULL;
  auto aligned16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (q_s2 != 1 || q_s0 % 8 || q_s1 % 8 || !aligned16(query) || !aligned16(partials))
    return OSCAR_E_ALIGN;
  if (raw) {
    if (!key || !value || !window) return OSCAR_E_NULL;
    if (k_s2 != 1 || v_s2 != 1 || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 ||
        !aligned16(key) || !aligned16(value) || !aligned16(window))
      return OSCAR_E_ALIGN;
  } else {
    if (!history) return OSCAR_E_NULL;
    if (!aligned16(history)) return OSCAR_E_ALIGN;
    if (history_bytes < 32 * h * 160) return OSCAR_E_SHAPE;  // smaller than one 32-token block
  }
  a.query = static_cast<const uint16_t*>(query);
  a.qs0 = q_s0;
  a.qs1 = q_s1;
  a.key = static_cast<const uint16_t*>(key);
  a.ks0 = k_s0;
  a.ks1 = k_s1;
  a.value = static_cast<const uint16_t*>(value);
  a.vs0 = v_s0;
  a.vs1 = v_s1;
  a.history = static_cast<const uint8_t*>(history);
  a.history_bytes = history ? history_bytes : 0;
  a.window = static_cast<const uint16_t*>(window);
  a.window_elems = window ? window_elems : 0;
  a.qstarts = qstarts;
  a.seq_lens = seq_lens;
  a.table = block_tables;
  a.table_stride = table_stride;
  a.table_columns = table_columns;
  a.counts = counts;
  a.tasks = tasks;
  a.task_count = task_count;
  a.partials = partials;
  a.lse = lse;
  a.n = n;
  a.g = static_cast<int32_t>(g);
  a.hq = static_cast<int32_t>(hq);
  a.qt = query_tile;
  a.splits = splits;
  a.block_n = block_n;
  a.scale_log2 = scale * kLog2e;
  a.mask[0] = 0x00030003u;
  a.mask[1] = 0x000c000cu;
  a.mask[2] = 0x00300030u;
  const dim3 grid(static_cast<unsigned>(programs), static_cast<unsigned>(h),
                  static_cast<unsigned>(splits));
  hipStream_t s = as_stream(stream);
  if (raw) {
    if (qrows <= 16)
      hipLaunchKernelGGL(raw_kernel<1>, grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL(raw_kernel<2>, grid, dim3(kThreads), 0, s, a);
  } else {
    if (qrows <= 16)
      hipLaunchKernelGGL(history_kernel<1>, grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL(history_kernel<2>, grid, dim3(kThreads), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}
