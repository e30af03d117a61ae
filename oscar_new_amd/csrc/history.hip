// Split-KV paged decode attention over the INT2 history, on gfx950 FP4 x FP8 MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel` with IS_RAW false; the
// history tile loop kernels.py:385-420 and its packed-vector load kernels.py:205-219).
// Semantics kept: one workgroup per (task, kv head, split); history positions
// [sink_len, recent_begin) split into ceil(ceil(len / BN) / splits) tiles per split; scores
// scaled by `scale`; per-split normalized output and natural-log LSE; live rows of an empty
// split get 0 / -inf; inactive programs write nothing.
//
// MI355X design:
//   * A 2-bit code c in a zero-padded nibble is the FP4 (e2m1) value c/2, exactly, so packed
//     codes become MFMA operands with one AND (even codes) or SHIFT+AND (odd codes) per 8
//     codes; nothing is dequantized element-wise. Scale s and zero z are folded out:
//       q.k = s_k (q.c) + z_k sum(q);   sum_t p_t v_t = sum_t (p_t s_v,t) c_t + sum_t p_t z_v,t.
//   * The other operand is FP8 (OCP e4m3): the rotated query as a sum of kQTerms FP8 terms
//     after a power-of-two row scaling, and p_t s_v,t as hi + lo with an E8M0 scale per
//     (query row, chunk) applied by the MFMA itself.
//   * Every wavefront streams its own 64-token chunks (chunks w, w + 4, ... of the split)
//     through a private two-stage LDS ring and keeps its own online-softmax state, so the
//     token loop has no workgroup barrier. The four states are merged once at the end.
//   * Scores are computed transposed (S^T = K Q^T): a lane holds one query row and 16 of the
//     chunk's tokens, so softmax statistics are lane-local and the lane's probabilities are
//     directly its bytes of the P*V A operand (16 tokens hi, the same 16 tokens lo). The V
//     codes reach the B operand in token-major order through ds_read_b64_tr_b4, with each
//     lane supplying the LDS row of the token that its P bytes hold.
//   * Records arrive by direct-to-LDS DMA (global_load_lds_dwordx4, nine 16-byte loads per
//     lane per chunk, SGPR base + per-lane offset): bytes 0..143 of each 160-byte record
//     (the last 16 bytes are slot padding), 144 bytes apart, 4 bytes past a 16-byte
//     boundary so that V codes (record byte 68) are 8-byte aligned for the transposed reads.
//   * Block-table entries of the split are resolved to byte offsets once, into LDS.
#include <type_traits>

#include "attention.h"
#include "dma.h"
#include "finish.h"
#include "layer.h"
#include "pre.h"

namespace oscar {
namespace {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2* lds_i32x2_ptr_t;

constexpr int kChunk = 64;                       // tokens per wavefront iteration
constexpr int kPieces = 9;                       // 16-byte pieces staged per record
constexpr int kRec = 16 * kPieces;               // 144: LDS record stride
constexpr int kSkew = 4;                         // record base offset: V codes 8-aligned
constexpr int kStageBytes = kChunk * kRec + 16;  // 9232
constexpr int kDma = kChunk * kPieces / 64;      // 9 loads of 16 bytes per lane per chunk
constexpr int kRingBytes = 4 * 2 * kStageBytes;  // two stages per wavefront
constexpr int kTableCache = 256;                 // kernel blocks whose offsets live in LDS
constexpr float kTheta = 8.0f;                   // lazy-max slack, log2 units
constexpr int kQTerms = 2;
constexpr uint32_t kNoBlock = 0xffffffffu;

static_assert(kDma * 64 == kChunk * kPieces, "a chunk image is whole DMA instructions");
static_assert(kStageBytes % 16 == 0, "stages stay 16-byte aligned");

// ---------------------------------------------------------------- number formats

// Packed 2-bit codes -> FP4 nibbles: codes 0, 2, 4, .. (even) or 1, 3, 5, .. (odd) of a dword.
__device__ __forceinline__ int32_t even_codes(uint32_t w) {
  return static_cast<int32_t>(w & 0x33333333u);
}
__device__ __forceinline__ int32_t odd_codes(uint32_t w) {
  return static_cast<int32_t>((w >> 2) & 0x33333333u);
}

// S^T tile += K (FP4, A) x Q (FP8, B); K = 128 head dims.
__device__ __forceinline__ f32x4 mfma_qk(const i32x8& k4, const i32x8& q8, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k4, q8, c, 4, 0, 0, 0, 0, 0);
}
// O tile += 2^(sa - 127) P (FP8, A) x V (FP4, B); K = 64 tokens x {hi, lo}.
__device__ __forceinline__ f32x4 mfma_pv(const i32x8& p8, const i32x8& v4, f32x4 c, int sa) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(p8, v4, c, 0, 4, 0, sa, 0, 127);
}

// Four floats -> four e4m3 bytes (round to nearest even).
__device__ __forceinline__ uint32_t fp8x4(float x0, float x1, float x2, float x3) {
  const int v = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, v, true));
}
// Rounds x to e4m3 bytes and leaves the (exact) residual x - rounded in x.
__device__ __forceinline__ uint32_t fp8x4_take(float (&x)[4]) {
  const uint32_t b = fp8x4(x[0], x[1], x[2], x[3]);
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(b), false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(b), true);
  x[0] -= lo[0];
  x[1] -= lo[1];
  x[2] -= hi[0];
  x[3] -= hi[1];
  return b;
}

__device__ __forceinline__ float h16lo(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x & 0xffffu)));
}
__device__ __forceinline__ float h16hi(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> 16)));
}

// ---------------------------------------------------------------- paging

// Offset (32-byte units) of kernel block kb of this request/head, or kNoBlock
// (kernels.py:392-399: block table column -> physical page and block within the page).
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

// ---------------------------------------------------------------- kernel

// Token held by byte e (0..15) of the P operand of lane group g: the score-layout token of
// element e of the lane's four 16-token QK tiles.
__host__ __device__ constexpr int p_token(int g, int e) { return 16 * (e >> 2) + 4 * g + (e & 3); }

// Operand index maps (fixed by the f8f6f4 MFMA operand layouts on gfx950):
//   FP8 operand: lane (row l%16, group G = l/16) byte e holds k = 32 G + e.
//   FP4 operand: lane group G nibble i holds k = 64 (G&1) + 16 (G>>1) + 32 (i/16) + i%16.
// QK (k = head dim within a 128-dim half h): K lane group G reads code dwords 8h + 2G and
// 8h + 2G + 1 (d = 128h + 32G .. +31) and emits [even, odd, even, odd] nibble dwords, so
// B byte e of lane group G holds q[d], d = 128h + 64 (e/16) + 16 G + sigma(e%16),
// sigma(j) = 2 (j%8) + j/8.
// PV (k = token x term): A lane group g bytes 0..15 are P_hi of tokens p_token(g, 0..15),
// bytes 16..31 P_lo of the same tokens. B lane group G nibbles 0..15 are then k = 64 (G&1) +
// 16 (G>>1) + i = bytes 16 (G>>1) + i of A group 2 (G&1), and nibbles 16..31 the same bytes of
// A group 2 (G&1) + 1: lane n of B group G supplies the LDS row of token p_token(2 (G&1), n)
// to the first transposed read and p_token(2 (G&1) + 1, n) to the second. One E8M0 scale per
// query row covers all four scale blocks: the scale of k block kb is read from lane group kb,
// while an FP8 lane group G holds its bytes 0..15 in block G / 2 and 16..31 in block 2 + G / 2.
// LDS of one general-kernel workgroup.
template <int RT>
struct HistoryLds {
  uint8_t ring[kRingBytes] __attribute__((aligned(16)));
  uint32_t off[kTableCache];
  float red[3][4][RT * 16];  // per wavefront: row max, sum p, sum p z_v
};

// One (task, kv head, split) unit of the general kernel; the whole workgroup calls it.
// `st`: the launch's split length (launch_split_tokens).
template <int RT>
__device__ __forceinline__ void history_unit(const AttnArgs& a, int task, int head, int split,
                                             int st, HistoryLds<RT>& lds) {
  uint8_t* s_ring = lds.ring;
  uint32_t* s_off = lds.off;
  auto& s_red = lds.red;
  static_assert(RT * 16 * 512 <= 2 * kStageBytes, "query staging fits wavefront 3's stages");
  static_assert(2 * kQTerms * 64 * 32 <= 2 * kStageBytes, "query operands fit as well");
  static_assert(4 * 16 * 256 * 4 <= kRingBytes, "the epilogue merge fits the ring");

  Task t;
  if (!read_task(a, t, task)) return;
  const int length = t.recent_begin - t.sink_len;
  const int nsplit = history_splits(a, length, st);
  if (split >= nsplit) {
    write_unused_split(a, t, head, split);
    return;
  }
  int p_lo, p_hi;
  history_positions(a, t, length, nsplit, split, st, p_lo, p_hi);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int first = p_lo >> 6;
  const int nchunk = p_lo < p_hi ? ((p_hi - 1) >> 6) - first + 1 : 0;
  const int nmine = nchunk > wave ? (nchunk - wave + 3) >> 2 : 0;  // chunks wave + 4 j
  const int kb_first = p_lo >> a.L.bk_shift;

  // ---- DMA plan: 16-byte piece c = 64 i + lane of a chunk is record c / 9, bytes
  // 16 (c % 9); records of one head are tok_bytes apart in the kernel block.
  const uint32_t tok_bytes = static_cast<uint32_t>(a.L.kv_heads) * kSlot;
  uint32_t voff[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int c = 64 * i + lane;
    voff[i] = static_cast<uint32_t>(c / kPieces) * tok_bytes + 16 * (c % kPieces);
  }
  const uint32_t my_ring = lds_addr(s_ring) + wave * 2 * kStageBytes;
  const uint32_t in_kb_mask = static_cast<uint32_t>(a.L.bk - 1);
  uint32_t valid_bits = 0;
  // This wavefront's chunk j -> its ring stage s.
  auto issue = [&](int j, int s) {
    const int t0 = (first + wave + 4 * j) << 6;
    const int local = (t0 >> a.L.bk_shift) - kb_first;
    uint32_t off32 = s_off[min(local, kTableCache - 1)];
    if (local >= kTableCache) off32 = kernel_block_offset(a, t, head, t0 >> a.L.bk_shift);
    off32 = uniform(off32);
    const uint8_t* base = a.history;
    const bool ok = off32 != kNoBlock;
    if (ok)
      base = a.history + (static_cast<uint64_t>(off32) << 5) +
             (static_cast<uint32_t>(t0) & in_kb_mask) * tok_bytes;
    valid_bits = ok ? (valid_bits | (1u << s)) : (valid_bits & ~(1u << s));
    const uint32_t lds = my_ring + s * kStageBytes + kSkew;
#pragma unroll
    for (int i = 0; i < kDma; ++i) dma_x4_stream(base, voff[i], lds + 1024 * i);
  };

  // ---- query rows -> LDS (wavefront 3's stages, whose first chunks are issued once the
  // query has been converted). 16-byte piece p of row r sits at position r * 32 +
  // (p ^ (r & 31)), so the column reads below spread over all banks.
  uint8_t* q_lds = s_ring + 6 * kStageBytes;
  {
    const uint32_t q_base = lds_addr(q_lds);
#pragma unroll
    for (int i = 0; i < 2 * RT; ++i) {
      const int slot = (wave * 2 * RT + i) * 64 + lane;
      const int row = slot >> 5, piece = (slot & 31) ^ (row & 31);
      const RowInfo ri = row_info(a, t, head, row);
      const uint16_t* src =
          ri.valid ? a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 8 * piece : a.query;
      dma_dwordx4(src, q_base + 1024 * (wave * 2 * RT + i));
    }
  }
  // Kernel-block offsets of the split. The wait for these loads also covers the query DMA
  // issued before them (vector-memory loads complete in order).
  if (nchunk > 0) {
    const int nkb = min(((p_hi - 1) >> a.L.bk_shift) - kb_first + 1, kTableCache);
    for (int j = threadIdx.x; j < nkb; j += kThreads)
      s_off[j] = kernel_block_offset(a, t, head, kb_first + j);
  }
  OSCAR_WAIT_VM(0);
  __syncthreads();
  if (wave < 3) {
    if (nmine > 0) issue(0, 0);
    if (nmine > 1) issue(1, 1);
  }

  // ---- query -> FP8 B operands (kQTerms terms) with a per-row power-of-two scaling,
  // converted cooperatively: wavefront w builds operand dwords 2w, 2w + 1 of every lane.
  // Those dwords hold q[row n][d], d = 128h + 64 (w/2) + 16g + 2i + (w&1), i = 0..7.
  i32x8 qb[RT][2][kQTerms];
  // Raw score r = s_k acc + z_k qs2 (acc = sum_d q'_d c_d / 2, q' = q mult); the score in
  // log2 units is r fq.
  float fq[RT], qs2[RT], qmult[RT];
  float qx[RT][2][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * rt + n;
    const bool live = row_info(a, t, head, row).valid;
    float mx = 0.f, qs = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int piece = 16 * h + 8 * (wave >> 1) + 2 * g;  // 8 bf16 per piece
      const u32x4 r0 = *reinterpret_cast<const u32x4*>(q_lds + row * 512 +
                                                       16 * (piece ^ (row & 31)));
      const u32x4 r1 = *reinterpret_cast<const u32x4*>(q_lds + row * 512 +
                                                       16 * ((piece + 1) ^ (row & 31)));
      const uint32_t w[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t bits = (wave & 1) ? (w[i] >> 16) : (w[i] & 0xffffu);
        const float x = live ? bf16_to_float(bits) : 0.f;
        qx[rt][h][i] = x;
        mx = fmaxf(mx, fabsf(x));
        qs += x;
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    qs += __shfl_xor(qs, 16, kWave);
    qs += __shfl_xor(qs, 32, kWave);
    if (g == 0) {
      s_red[0][wave][row] = mx;
      s_red[1][wave][row] = qs;
    }
  }
  barrier_lds();  // partial row max / sum published; the query rows are in registers
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * rt + n;
    const float mx = fmaxf(fmaxf(s_red[0][0][row], s_red[0][1][row]),
                           fmaxf(s_red[0][2][row], s_red[0][3][row]));
    const float qs = (s_red[1][0][row] + s_red[1][1][row]) + (s_red[1][2][row] + s_red[1][3][row]);
    // mult = 2^(134 - eb): the row max lands in [128, 256).
    const uint32_t eb = max((__float_as_uint(mx) >> 23) & 0xffu, 7u);
    qmult[rt] = __uint_as_float((261u - eb) << 23);
    fq[rt] = 2.0f * a.scale_log2 / qmult[rt];  // FP4 holds c/2
    qs2[rt] = 0.5f * qs * qmult[rt];
  }
  // Operand exchange area (aliases the query rows): [h][term][lane][8 dwords] per row tile.
  uint32_t* q_ops = reinterpret_cast<uint32_t*>(q_lds);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (rt > 0) barrier_lds();  // the previous tile's operands have been read
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        float v[4] = {qx[rt][h][4 * f] * qmult[rt], qx[rt][h][4 * f + 1] * qmult[rt],
                      qx[rt][h][4 * f + 2] * qmult[rt], qx[rt][h][4 * f + 3] * qmult[rt]};
#pragma unroll
        for (int term = 0; term < kQTerms; ++term)
          q_ops[((h * kQTerms + term) * 64 + lane) * 8 + 2 * wave + f] = fp8x4_take(v);
      }
    barrier_lds();
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int term = 0; term < kQTerms; ++term) {
        const u32x4* src = reinterpret_cast<const u32x4*>(q_ops + ((h * kQTerms + term) * 64 + lane) * 8);
        const u32x4 lo = src[0], hi = src[1];
        qb[rt][h][term] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                                (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
  }
  barrier_lds();  // everyone is done with the query staging area (wavefront 3's stages)
  if (wave == 3) {
    if (nmine > 0) issue(0, 0);
    if (nmine > 1) issue(1, 1);
  }

  // ---- per-lane LDS offsets inside a stage (record r starts at kSkew + 144 r)
  // QK A operand: token 16 tt + n, code dwords 8h + 2g, +1.
  const int k_off = kSkew + kRec * n + 8 * g;
  // Scale|zero of token p_token(g, e): K at record byte 64, V at 132.
  const int sz_off = kSkew + kRec * 4 * g + 64;
  // Transposed V reads: rows p_token(2 (g&1), n) and p_token(2 (g&1) + 1, n), codes at 68.
  const int v_off = kSkew + kRec * (16 * (n >> 2) + (n & 3)) + kRec * 8 * (g & 1) + kVector;

  float m[RT], psum[RT], zsum[RT];
  f32x4 o[RT][16];  // o[rt][2c + par]: rows 4g + v, dim 32c + 2n + par (units of c/2)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = -INFINITY;
    psum[rt] = 0.f;
    zsum[rt] = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c) o[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // One chunk from ring stage S (compile-time, so every LDS offset is an immediate).
  auto process = [&](int j, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    const uint8_t* st = s_ring + wave * 2 * kStageBytes + S * kStageBytes;
    // Scores S^T = K Q^T: four 16-token tiles.
    f32x4 acc[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      i32x8 kf[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const uint32_t* kp = reinterpret_cast<const uint32_t*>(st + k_off + 16 * kRec * tt + 32 * h);
        const uint32_t w0 = kp[0], w1 = kp[1];  // 4-byte aligned: two dword reads
        kf[tt] = i32x8{even_codes(w0), odd_codes(w0), even_codes(w1), odd_codes(w1), 0, 0, 0, 0};
      }
#pragma unroll
      for (int term = 0; term < kQTerms; ++term)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[rt][tt] = mfma_qk(kf[tt], qb[rt][h][term], acc[rt][tt]);
    }
    // Scale|zero of this lane's 16 tokens.
    uint32_t ksz[16], vsz[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int off = sz_off + kRec * (16 * (e >> 2) + (e & 3));
      ksz[e] = *reinterpret_cast<const uint32_t*>(st + off);
      vsz[e] = *reinterpret_cast<const uint32_t*>(st + off + kVector);
    }
    float r2[RT][16];  // raw scores (-inf: masked)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        r2[rt][e] = fmaf(h16lo(ksz[e]), acc[rt][e >> 2][e & 3], h16hi(ksz[e]) * qs2[rt]);
    // Only the first/last chunk of a split (or one whose kernel block is unmapped) is
    // partial: its tokens outside [p_lo, p_hi) get score -inf and a zero V scale/zero (the
    // bytes of unwritten slots may hold NaN patterns).
    const int t0 = (first + wave + 4 * j) << 6;
    const bool ok_block = (valid_bits >> S) & 1u;
    if (!(ok_block && t0 >= p_lo && t0 + kChunk <= p_hi)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const bool ok = ok_block && static_cast<uint32_t>(t0 + p_token(g, e) - p_lo) <
                                        static_cast<uint32_t>(p_hi - p_lo);
        vsz[e] = ok ? vsz[e] : 0u;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) r2[rt][e] = ok ? r2[rt][e] : -INFINITY;
      }
    }
    // Lazy running max: rescale only when a score exceeds the row max by more than 2^8.
    float lm[RT];
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v = r2[rt][0];
#pragma unroll
      for (int e = 1; e < 16; ++e) v = fmaxf(v, r2[rt][e]);
      lm[rt] = v * fq[rt];
      need |= lm[rt] > m[rt] + kTheta;
    }
    if (__any(need)) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float v = max_xor32(max_xor16(lm[rt]));
        const float mn = fmaxf(m[rt], v);
        const float alpha = mn == -INFINITY ? 1.0f : exp2f(m[rt] - mn);
        m[rt] = mn;
        psum[rt] *= alpha;
        zsum[rt] *= alpha;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const float av = __shfl(alpha, 4 * g + v4, kWave);  // accumulator row 4g + v4
#pragma unroll
          for (int c = 0; c < 16; ++c) o[rt][c][v4] *= av;
        }
      }
    }
    // Probabilities -> P operands: p s_v as FP8 hi + lo, one E8M0 scale per query row.
    i32x8 pa[RT];
    int sa[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float nm = m[rt] == -INFINITY ? 0.f : -m[rt];
      float av[16];
      float amax = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = __builtin_amdgcn_exp2f(fmaf(r2[rt][e], fq[rt], nm));
        psum[rt] += p;
        zsum[rt] = fmaf(p, h16hi(vsz[e]), zsum[rt]);
        av[e] = p * h16lo(vsz[e]);
        amax = fmaxf(amax, av[e]);
      }
      amax = max_xor32(max_xor16(amax));
      // mult = 2^(133 - eb) puts the row max in [64, 128); the MFMA scales back by
      // 2^(eb - 133) = E8M0 byte eb - 6.
      const uint32_t eb = max(__float_as_uint(amax) >> 23, 7u);
      const float mult = __uint_as_float((260u - eb) << 23);
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float x[4] = {av[4 * f] * mult, av[4 * f + 1] * mult, av[4 * f + 2] * mult,
                      av[4 * f + 3] * mult};
        hi[f] = fp8x4_take(x);
        lo[f] = fp8x4(x[0], x[1], x[2], x[3]);
      }
      pa[rt] = i32x8{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3],
                     (int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
      sa[rt] = static_cast<int>(eb) - 6;
    }
    // O += P V over the chunk's 64 tokens, 32 dims (16 dim pairs) per transposed read pair.
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const i32x2 r0 = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off + 8 * c));
      const i32x2 r1 =
          __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off + 4 * kRec + 8 * c));
      const i32x8 be = i32x8{even_codes(r0[0]), even_codes(r0[1]), even_codes(r1[0]),
                             even_codes(r1[1]), 0, 0, 0, 0};
      const i32x8 bo = i32x8{odd_codes(r0[0]), odd_codes(r0[1]), odd_codes(r1[0]),
                             odd_codes(r1[1]), 0, 0, 0, 0};
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        o[rt][2 * c] = mfma_pv(pa[rt], be, o[rt][2 * c], sa[rt]);
        o[rt][2 * c + 1] = mfma_pv(pa[rt], bo, o[rt][2 * c + 1], sa[rt]);
      }
    }
  };

  // ---- token loop: wait for chunk j, consume it, refill its stage with chunk j + 2.
  for (int j = 0; j < nmine; ++j) {
    if (j + 1 < nmine)
      OSCAR_WAIT_VM(kDma);  // chunk j landed; chunk j + 1 may still be in flight
    else
      OSCAR_WAIT_VM(0);
    if (j & 1)
      process(j, std::integral_constant<int, 1>());
    else
      process(j, std::integral_constant<int, 0>());
    if (j + 2 < nmine) {
      OSCAR_WAIT_LGKM();  // every read of this stage has completed
      issue(j + 2, j & 1);
    }
  }

  // ---- epilogue: merge the four wavefront states, then write normalized partials + LSE.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    psum[rt] = sum_xor32(sum_xor16(psum[rt]));
    zsum[rt] = sum_xor32(sum_xor16(zsum[rt]));
    if (g == 0) {
      s_red[0][wave][16 * rt + n] = m[rt];
      s_red[1][wave][16 * rt + n] = psum[rt];
      s_red[2][wave][16 * rt + n] = zsum[rt];
    }
  }
  __syncthreads();  // every chunk consumed; the ring is free for the merge
  float* s_o = reinterpret_cast<float*>(s_ring);  // [wave][row][256], one row tile at a time
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (rt > 0) __syncthreads();
    // This wavefront's weight per accumulator row, against the merged max.
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * rt + 4 * g + v;
      const float mx = fmaxf(fmaxf(s_red[0][0][row], s_red[0][1][row]),
                             fmaxf(s_red[0][2][row], s_red[0][3][row]));
      const float mw = s_red[0][wave][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - mx);
      float* dst = s_o + (wave * 16 + 4 * g + v) * 256 + 2 * n;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *reinterpret_cast<float2*>(dst + 32 * c) =
            make_float2(o[rt][2 * c][v] * f, o[rt][2 * c + 1][v] * f);
    }
    __syncthreads();
    // Thread -> (row, dims 4 (tid % 16) + 64 q4): 16 threads read 256 contiguous bytes.
    const int row16 = threadIdx.x >> 4, d0 = 4 * (threadIdx.x & 15);
    const int row = 16 * rt + row16;
    const RowInfo ri = row_info(a, t, head, row);
    if (ri.valid) {
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_red[0][w][row]);
      float den = 0.f, zs = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float mw = s_red[0][w][row];
        const float f = mw == -INFINITY ? 0.f : exp2f(mw - mx);
        den = fmaf(f, s_red[1][w][row], den);
        zs = fmaf(f, s_red[2][w][row], zs);
      }
      const float inv = 1.0f / fmaxf(den, 1.0e-30f);
      float* out = a.partials + ((ri.token * a.hq + ri.qhead) * a.splits + split) * kHeadDim + d0;
      const float4* so = reinterpret_cast<const float4*>(s_o + row16 * 256 + d0);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 x0 = so[16 * q4], x1 = so[16 * 256 / 4 + 16 * q4];
        const float4 x2 = so[2 * 16 * 256 / 4 + 16 * q4], x3 = so[3 * 16 * 256 / 4 + 16 * q4];
        const float4 r = make_float4((2.0f * ((x0.x + x1.x) + (x2.x + x3.x)) + zs) * inv,
                                     (2.0f * ((x0.y + x1.y) + (x2.y + x3.y)) + zs) * inv,
                                     (2.0f * ((x0.z + x1.z) + (x2.z + x3.z)) + zs) * inv,
                                     (2.0f * ((x0.w + x1.w) + (x2.w + x3.w)) + zs) * inv);
        *reinterpret_cast<float4*>(out + 64 * q4) = r;
      }
      if ((threadIdx.x & 15) == 0)
        a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] =
            den > 0.f ? (mx + log2f(den)) * kLn2 : -INFINITY;
    }
  }
}

template <int RT>
__global__ __launch_bounds__(kThreads, 3 - RT) void history_kernel(const AttnArgs a) {
  __shared__ HistoryLds<RT> lds;
  const int st = launch_split_tokens<kThreads>(a, static_cast<int>(gridDim.x));
  history_unit<RT>(a, blockIdx.x, blockIdx.y, blockIdx.z, st, lds);
}

// ---------------------------------------------------------------- 17-32 rows: two row groups

// Tasks of 17-32 query rows (MTP: 4 query tokens x 6 query heads = 24 rows). Two row groups of
// 16 rows share every chunk: with S streams (S = 4: eight wavefronts, one workgroup per CU;
// S = 2: four wavefronts, two workgroups per CU), wavefront w streams chunks (w % S) + S j and
// computes the rows 16 (w / S) .. + 15 of them, so each chunk is copied into LDS once (by the
// group-0 wavefront of its stream, three stages per stream) and read by two wavefronts, and
// every SIMD holds two wavefronts (a wavefront keeps one 16-row tile, about 210 registers,
// instead of 464 for two tiles, whose single wavefront per SIMD left the VALU half idle). A
// workgroup barrier per chunk publishes the chunk to the second wavefront of its stream and
// frees the stage of the chunk before; with two workgroups per CU those barriers are
// independent, so one workgroup's MFMAs meet the other's softmax. A row's arithmetic is the
// general kernel's with one row tile; the lazy-max rescale is decided per wavefront, so its
// bits depend on the 16-row grouping and the stream count, not on the launch form (grid or
// work queue, which take the same stream count for the same task count).
constexpr int kThreadsW8 = 512;
constexpr int kStagesW8 = 3;

// kWaves 8: four streams x two row groups; kWaves 4: two streams x two row groups, in under
// 80 KB of LDS with the work queue's task lists (two workgroups per CU).
template <int kWaves>
struct HistoryLdsW8 {
  uint8_t ring[(kWaves / 2) * kStagesW8 * kStageBytes] __attribute__((aligned(16)));
  uint8_t qstage[32 * 512] __attribute__((aligned(16)));  // query rows, then operand images
  uint32_t off[kTableCache];
  float red[3][8][16];  // per wavefront (or query stream): row max, sum p, sum p z_v of 16 rows
};
static_assert(8 * 16 * 128 * 4 <= sizeof(HistoryLdsW8<8>::ring), "half the merge fits the ring");
static_assert(4 * 16 * 128 * 4 <= sizeof(HistoryLdsW8<4>::ring), "half the merge fits the ring");
static_assert(2 * 2 * kQTerms * 64 * 32 <= 32 * 512, "both groups' operand images fit");

// `st`: the launch's split length (launch_split_tokens).
template <int kWaves>
__device__ __forceinline__ void history_unit_w8(const AttnArgs& a, int task, int head, int split,
                                                int st, HistoryLdsW8<kWaves>& lds) {
  constexpr int kStreams = kWaves / 2;
  constexpr int kT = kWaves * kWave;
  uint8_t* s_ring = lds.ring;
  uint32_t* s_off = lds.off;
  auto& s_red = lds.red;
  Task t;
  if (!read_task(a, t, task)) return;
  const int length = t.recent_begin - t.sink_len;
  const int nsplit = history_splits(a, length, st);
  if (split >= nsplit) {
    write_unused_split(a, t, head, split);
    return;
  }
  int p_lo, p_hi;
  history_positions(a, t, length, nsplit, split, st, p_lo, p_hi);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int stream = wave % kStreams, rg = wave / kStreams;
  const int n = lane & 15, g = lane >> 4;
  const int first = p_lo >> 6;
  const int nchunk = p_lo < p_hi ? ((p_hi - 1) >> 6) - first + 1 : 0;
  // chunks stream + kStreams j
  const int nmine = nchunk > stream ? (nchunk - stream + kStreams - 1) / kStreams : 0;
  const int nmax = (nchunk + kStreams - 1) / kStreams;  // stream 0's count
  const int kb_first = p_lo >> a.L.bk_shift;

  // ---- DMA plan (as in the general kernel); the group-0 wavefront of a stream issues.
  const uint32_t tok_bytes = static_cast<uint32_t>(a.L.kv_heads) * kSlot;
  uint32_t voff[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int c = 64 * i + lane;
    voff[i] = static_cast<uint32_t>(c / kPieces) * tok_bytes + 16 * (c % kPieces);
  }
  const uint32_t my_ring = lds_addr(s_ring) + stream * kStagesW8 * kStageBytes;
  const uint32_t in_kb_mask = static_cast<uint32_t>(a.L.bk - 1);
  // Offset (32-byte units) of the kernel block of this stream's chunk j, or kNoBlock.
  auto block_of = [&](int j) {
    const int t0 = (first + stream + kStreams * j) << 6;
    const int local = (t0 >> a.L.bk_shift) - kb_first;
    uint32_t off32 = s_off[min(local, kTableCache - 1)];
    if (local >= kTableCache) off32 = kernel_block_offset(a, t, head, t0 >> a.L.bk_shift);
    return static_cast<uint32_t>(uniform(static_cast<int>(off32)));
  };
  auto issue = [&](int j, int s) {
    const int t0 = (first + stream + kStreams * j) << 6;
    const uint32_t off32 = block_of(j);
    const uint8_t* base = a.history;
    if (off32 != kNoBlock)
      base = a.history + (static_cast<uint64_t>(off32) << 5) +
             (static_cast<uint32_t>(t0) & in_kb_mask) * tok_bytes;
    const uint32_t l = my_ring + s * kStageBytes + kSkew;
#pragma unroll
    for (int i = 0; i < kDma; ++i) dma_x4_stream(base, voff[i], l + 1024 * i);
  };

  // ---- query rows -> LDS: 32 rows, piece p of row r at r * 32 + (p ^ (r & 31)).
  uint8_t* q_lds = lds.qstage;
  {
    constexpr int kQPer = 16 / kWaves;  // 1 KiB DMAs per wavefront
    const uint32_t q_base = lds_addr(q_lds);
#pragma unroll
    for (int i = 0; i < kQPer; ++i) {
      const int slot = (wave * kQPer + i) * 64 + lane;
      const int row = slot >> 5, piece = (slot & 31) ^ (row & 31);
      const RowInfo ri = row_info(a, t, head, row);
      const uint16_t* src =
          ri.valid ? a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 8 * piece : a.query;
      dma_dwordx4(src, q_base + 1024 * (wave * kQPer + i));
    }
  }
  if (nchunk > 0) {
    const int nkb = min(((p_hi - 1) >> a.L.bk_shift) - kb_first + 1, kTableCache);
    for (int j = threadIdx.x; j < nkb; j += kT)
      s_off[j] = kernel_block_offset(a, t, head, kb_first + j);
  }
  OSCAR_WAIT_VM(0);
  __syncthreads();
  if (rg == 0) {
    if (nmine > 0) issue(0, 0);
    if (nmine > 1) issue(1, 1);
  }

  // ---- query -> FP8 B operands of this wavefront's 16 rows (row group rg), converted by the
  // group's wavefronts in four query streams: stream qs builds operand dwords 2 qs, 2 qs + 1
  // of every lane (four wavefronts: one stream each; two: streams w and w + 2).
  i32x8 qb[2][kQTerms];
  float fq, qs2, qmult;
  constexpr int kQStreams = 4 / kStreams;
  float qx[kQStreams][2][8];
  {
    const int row = 16 * rg + n;
    const bool live = row_info(a, t, head, row).valid;
#pragma unroll
    for (int k = 0; k < kQStreams; ++k) {
      const int qsid = stream + kStreams * k;
      float mx = 0.f, qsum = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int piece = 16 * h + 8 * (qsid >> 1) + 2 * g;
        const u32x4 r0 = *reinterpret_cast<const u32x4*>(q_lds + row * 512 + 16 * (piece ^ (row & 31)));
        const u32x4 r1 =
            *reinterpret_cast<const u32x4*>(q_lds + row * 512 + 16 * ((piece + 1) ^ (row & 31)));
        const uint32_t w[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t bits = (qsid & 1) ? (w[i] >> 16) : (w[i] & 0xffffu);
          const float x = live ? bf16_to_float(bits) : 0.f;
          qx[k][h][i] = x;
          mx = fmaxf(mx, fabsf(x));
          qsum += x;
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      qsum += __shfl_xor(qsum, 16, kWave);
      qsum += __shfl_xor(qsum, 32, kWave);
      if (g == 0) {
        s_red[0][4 * rg + qsid][n] = mx;
        s_red[1][4 * rg + qsid][n] = qsum;
      }
    }
  }
  barrier_lds();  // partial row max / sum published; the query rows are in registers
  {
    const int w0 = 4 * rg;
    const float mx = fmaxf(fmaxf(s_red[0][w0][n], s_red[0][w0 + 1][n]),
                           fmaxf(s_red[0][w0 + 2][n], s_red[0][w0 + 3][n]));
    const float qsum = (s_red[1][w0][n] + s_red[1][w0 + 1][n]) + (s_red[1][w0 + 2][n] + s_red[1][w0 + 3][n]);
    const uint32_t eb = max((__float_as_uint(mx) >> 23) & 0xffu, 7u);
    qmult = __uint_as_float((261u - eb) << 23);
    fq = 2.0f * a.scale_log2 / qmult;  // FP4 holds c/2
    qs2 = 0.5f * qsum * qmult;
  }
  // Operand images [rg][h][term][lane][8 dwords] (alias the query rows, now in registers).
  uint32_t* q_ops = reinterpret_cast<uint32_t*>(q_lds) + rg * (2 * kQTerms * 64 * 8);
#pragma unroll
  for (int k = 0; k < kQStreams; ++k) {
    const int qsid = stream + kStreams * k;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        float v[4] = {qx[k][h][4 * f] * qmult, qx[k][h][4 * f + 1] * qmult,
                      qx[k][h][4 * f + 2] * qmult, qx[k][h][4 * f + 3] * qmult};
#pragma unroll
        for (int term = 0; term < kQTerms; ++term)
          q_ops[((h * kQTerms + term) * 64 + lane) * 8 + 2 * qsid + f] = fp8x4_take(v);
      }
  }
  barrier_lds();
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int term = 0; term < kQTerms; ++term) {
      const u32x4* src = reinterpret_cast<const u32x4*>(q_ops + ((h * kQTerms + term) * 64 + lane) * 8);
      const u32x4 lo = src[0], hi = src[1];
      qb[h][term] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                          (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }

  // ---- per-lane LDS offsets inside a stage (as in the general kernel)
  const int k_off = kSkew + kRec * n + 8 * g;
  const int sz_off = kSkew + kRec * 4 * g + 64;
  const int v_off = kSkew + kRec * (16 * (n >> 2) + (n & 3)) + kRec * 8 * (g & 1) + kVector;

  float m = -INFINITY, psum = 0.f, zsum = 0.f;
  f32x4 o[16];  // o[2c + par]: rows 4g + v, dim 32c + 2n + par (units of c/2)
#pragma unroll
  for (int c = 0; c < 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One chunk from ring stage S (compile-time, so every LDS offset is an immediate).
  auto process = [&](int j, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    const uint8_t* st = s_ring + stream * kStagesW8 * kStageBytes + S * kStageBytes;
    f32x4 acc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      i32x8 kf[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const uint32_t* kp = reinterpret_cast<const uint32_t*>(st + k_off + 16 * kRec * tt + 32 * h);
        const uint32_t w0 = kp[0], w1 = kp[1];
        kf[tt] = i32x8{even_codes(w0), odd_codes(w0), even_codes(w1), odd_codes(w1), 0, 0, 0, 0};
      }
#pragma unroll
      for (int term = 0; term < kQTerms; ++term)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt] = mfma_qk(kf[tt], qb[h][term], acc[tt]);
    }
    uint32_t ksz[16], vsz[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int off = sz_off + kRec * (16 * (e >> 2) + (e & 3));
      ksz[e] = *reinterpret_cast<const uint32_t*>(st + off);
      vsz[e] = *reinterpret_cast<const uint32_t*>(st + off + kVector);
    }
    float r2[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) r2[e] = fmaf(h16lo(ksz[e]), acc[e >> 2][e & 3], h16hi(ksz[e]) * qs2);
    const int t0 = (first + stream + kStreams * j) << 6;
    const bool ok_block = block_of(j) != kNoBlock;
    if (!(ok_block && t0 >= p_lo && t0 + kChunk <= p_hi)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const bool ok = ok_block && static_cast<uint32_t>(t0 + p_token(g, e) - p_lo) <
                                        static_cast<uint32_t>(p_hi - p_lo);
        vsz[e] = ok ? vsz[e] : 0u;
        r2[e] = ok ? r2[e] : -INFINITY;
      }
    }
    float lm = r2[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) lm = fmaxf(lm, r2[e]);
    lm *= fq;
    if (__any(lm > m + kTheta)) {
      const float v = max_xor32(max_xor16(lm));
      const float mn = fmaxf(m, v);
      const float alpha = mn == -INFINITY ? 1.0f : exp2f(m - mn);
      m = mn;
      psum *= alpha;
      zsum *= alpha;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const float av = __shfl(alpha, 4 * g + v4, kWave);  // accumulator row 4g + v4
#pragma unroll
        for (int c = 0; c < 16; ++c) o[c][v4] *= av;
      }
    }
    const float nm = m == -INFINITY ? 0.f : -m;
    float av[16];
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(fmaf(r2[e], fq, nm));
      psum += p;
      zsum = fmaf(p, h16hi(vsz[e]), zsum);
      av[e] = p * h16lo(vsz[e]);
      amax = fmaxf(amax, av[e]);
    }
    amax = max_xor32(max_xor16(amax));
    const uint32_t eb = max(__float_as_uint(amax) >> 23, 7u);
    const float mult = __uint_as_float((260u - eb) << 23);
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      float x[4] = {av[4 * f] * mult, av[4 * f + 1] * mult, av[4 * f + 2] * mult,
                    av[4 * f + 3] * mult};
      hi[f] = fp8x4_take(x);
      lo[f] = fp8x4(x[0], x[1], x[2], x[3]);
    }
    const i32x8 pa = i32x8{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3],
                           (int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
    const int sa = static_cast<int>(eb) - 6;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const i32x2 r0 = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off + 8 * c));
      const i32x2 r1 =
          __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off + 4 * kRec + 8 * c));
      const i32x8 be = i32x8{even_codes(r0[0]), even_codes(r0[1]), even_codes(r1[0]),
                             even_codes(r1[1]), 0, 0, 0, 0};
      const i32x8 bo = i32x8{odd_codes(r0[0]), odd_codes(r0[1]), odd_codes(r1[0]),
                             odd_codes(r1[1]), 0, 0, 0, 0};
      o[2 * c] = mfma_pv(pa, be, o[2 * c], sa);
      o[2 * c + 1] = mfma_pv(pa, bo, o[2 * c + 1], sa);
    }
  };

  // ---- token loop: every wavefront takes the same number of barriers (nmax, stream 0's
  // chunk count). Iteration j: the group-0 wavefront waits for its chunk j (chunk j + 1 may
  // still be in flight), the barrier publishes it to both wavefronts of the stream and tells
  // every wavefront that chunk j - 1 is consumed, so its stage takes chunk j + 2.
  auto step = [&](int j, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    if (rg == 0 && j < nmine) {
      if (j + 1 < nmine)
        OSCAR_WAIT_VM(kDma);
      else
        OSCAR_WAIT_VM(0);
    }
    barrier_lds();
    if (rg == 0 && j + 2 < nmine) issue(j + 2, (S + 2) % kStagesW8);
    if (j < nmine) process(j, stage_tag);
  };
  for (int j = 0; j < nmax; j += kStagesW8) {
    step(j, std::integral_constant<int, 0>());
    if (j + 1 < nmax) step(j + 1, std::integral_constant<int, 1>());
    if (j + 2 < nmax) step(j + 2, std::integral_constant<int, 2>());
  }

  // ---- epilogue: merge the four stream wavefronts of each row group, 128 dims at a time.
  psum = sum_xor32(sum_xor16(psum));
  zsum = sum_xor32(sum_xor16(zsum));
  barrier_lds();  // every chunk consumed; the ring is free for the merge
  if (g == 0) {
    s_red[0][wave][n] = m;
    s_red[1][wave][n] = psum;
    s_red[2][wave][n] = zsum;
  }
  barrier_lds();
  float* s_o = reinterpret_cast<float*>(s_ring);  // [wave][row 0..15][128]
  const int tid = threadIdx.x;
  constexpr int kPasses = 512 / kT;  // 32 rows x 16 threads
  RowInfo ri[kPasses];
  float mx[kPasses], den[kPasses], zs[kPasses], inv[kPasses];
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int row32 = (tid >> 4) + pass * (kT >> 4);
    const int rgx = row32 >> 4, r16 = row32 & 15;
    ri[pass] = row_info(a, t, head, row32);
    mx[pass] = -INFINITY;
    den[pass] = 0.f;
    zs[pass] = 0.f;
#pragma unroll
    for (int w = 0; w < kStreams; ++w) mx[pass] = fmaxf(mx[pass], s_red[0][kStreams * rgx + w][r16]);
#pragma unroll
    for (int w = 0; w < kStreams; ++w) {
      const float mw = s_red[0][kStreams * rgx + w][r16];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - mx[pass]);
      den[pass] = fmaf(f, s_red[1][kStreams * rgx + w][r16], den[pass]);
      zs[pass] = fmaf(f, s_red[2][kStreams * rgx + w][r16], zs[pass]);
    }
    inv[pass] = 1.0f / fmaxf(den[pass], 1.0e-30f);
  }
  const int d0 = 4 * (tid & 15);
#pragma unroll
  for (int hd = 0; hd < 2; ++hd) {
    if (hd > 0) barrier_lds();  // the first half has been read
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 4 * g + v;
      float mxr = s_red[0][kStreams * rg][row];
#pragma unroll
      for (int w = 1; w < kStreams; ++w) mxr = fmaxf(mxr, s_red[0][kStreams * rg + w][row]);
      const float mw = s_red[0][wave][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - mxr);
      float* dst = s_o + (wave * 16 + row) * 128 + 2 * n;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<float2*>(dst + 32 * c) =
            make_float2(o[2 * (4 * hd + c)][v] * f, o[2 * (4 * hd + c) + 1][v] * f);
    }
    barrier_lds();
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      if (!ri[pass].valid) continue;
      const int row32 = (tid >> 4) + pass * (kT >> 4);
      const int rgx = row32 >> 4, r16 = row32 & 15;
      float* out = a.partials +
                   ((ri[pass].token * a.hq + ri[pass].qhead) * a.splits + split) * kHeadDim +
                   128 * hd + d0;
      const float4* so =
          reinterpret_cast<const float4*>(s_o + ((kStreams * rgx) * 16 + r16) * 128 + d0);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float4 x[kStreams];
#pragma unroll
        for (int w = 0; w < kStreams; ++w) x[w] = so[w * 16 * 128 / 4 + 16 * q];
        float4 acc;
        if constexpr (kStreams == 4) {
          acc = make_float4((x[0].x + x[1].x) + (x[2].x + x[3].x), (x[0].y + x[1].y) + (x[2].y + x[3].y),
                            (x[0].z + x[1].z) + (x[2].z + x[3].z), (x[0].w + x[1].w) + (x[2].w + x[3].w));
        } else {
          acc = make_float4(x[0].x + x[1].x, x[0].y + x[1].y, x[0].z + x[1].z, x[0].w + x[1].w);
        }
        const float4 r = make_float4((2.0f * acc.x + zs[pass]) * inv[pass],
                                     (2.0f * acc.y + zs[pass]) * inv[pass],
                                     (2.0f * acc.z + zs[pass]) * inv[pass],
                                     (2.0f * acc.w + zs[pass]) * inv[pass]);
        *reinterpret_cast<float4*>(out + 64 * q) = r;
      }
      if (hd == 0 && (tid & 15) == 0)
        a.lse[(ri[pass].token * a.hq + ri[pass].qhead) * a.splits + split] =
            den[pass] > 0.f ? (mx[pass] + log2f(den[pass])) * kLn2 : -INFINITY;
    }
  }
  barrier_lds();  // the merge area is read before the next unit's DMA reuses the ring
}

template <int kWaves>
__global__ __launch_bounds__(kWaves * kWave, 8 / kWaves) void history_w8_kernel(const AttnArgs a) {
  __shared__ HistoryLdsW8<kWaves> lds;
  const int st = launch_split_tokens<kWaves * kWave>(a, static_cast<int>(gridDim.x));
  history_unit_w8<kWaves>(a, blockIdx.x, blockIdx.y, blockIdx.z, st, lds);
}

// The 17-32-row kernel as a work queue (token-bounded splits, one workgroup per CU): a grid of
// (task, kv head, split) workgroups is mostly empty when lengths are ragged (a request of L
// history tokens uses ceil(L / split_tokens) of the split slots), and with one workgroup per
// CU every empty workgroup holds a CU while it reads its task and exits. Here each
// workgroup lists the units of every task (split counts from the task rows, an exclusive
// scan in LDS), then takes units from a device counter until none are left: full splits
// first, then each task's last (shorter) split. A unit is computed exactly as in the grid
// form (the same bits). The split slots a task does not use get their -inf LSE from the
// workgroups in task-stride order. The counters (next unit, finished workgroups) are zero at
// launch; the last workgroup to finish sets them to zero again, so graph replays reuse them.
// Launches that overlap on one device must not share counters.
constexpr int kQueueTasks = 2048;  // task rows the workgroup lists in LDS (eight wavefronts)

// kRoles (four wavefronts): the step's pre-attention roles `pre` run as units of the queue,
// each with the role code of the other launches (the same bits): the BF16 branch of each
// (task, kv head), in two units of 16 rows, is claimed before any history unit (it is the
// longest unit); the K/V store quads, short, are claimed after the last history unit, where
// they fill the queue's tail (first: 2.3 us slower per c4 step). A role borrows the unit's LDS
// (the ring and the query stage) and ends with a barrier.
template <int kWaves, int kTasks, bool kRoles>
__device__ __forceinline__ void history_queue_body(const AttnArgs& a, int32_t* counters,
                                                   int32_t programs, const PreArgs* pre) {
  constexpr int kT = kWaves * kWave;
  __shared__ HistoryLdsW8<kWaves> lds;
  __shared__ int32_t s_full[kTasks + 1];  // full splits of the tasks before t
  __shared__ int32_t s_nsplit[kTasks];
  __shared__ int16_t s_used[kTasks];      // tasks in use, in order
  __shared__ int32_t s_part[2][kT];            // per-thread sums, then their exclusive scan
  __shared__ int32_t s_total[2];               // full splits, tasks in use
  __shared__ int32_t s_claim;
  const int heads = a.L.kv_heads;
  // Split counts (the launch's split length, or under the device rule the length derived from
  // the task lengths read in the same pass), then two exclusive scans (full splits, tasks in
  // use) over thread chunks.
  __shared__ int64_t s_wave_total[kT / kWave];
  int64_t hist = 0;
  for (int task = threadIdx.x; task < programs; task += kT) {
    Task t;
    const int len = read_task(a, t, task) ? max(t.recent_begin - t.sink_len, 0) : -1;
    s_nsplit[task] = len;
    hist += max(len, 0);
  }
  int st = a.split_tokens;
  if (st < 0) {
    hist = wave_sum_i64(hist);
    if ((threadIdx.x & (kWave - 1)) == 0) s_wave_total[threadIdx.x / kWave] = hist;
    __syncthreads();
    int64_t total = 0;
#pragma unroll
    for (int w = 0; w < kT / kWave; ++w) total += s_wave_total[w];
    const int count = max(min(a.task_count[0], programs), 0);
    st = device_split_tokens(total, count, heads, -st, false);
  }
  for (int task = threadIdx.x; task < programs; task += kT) {
    const int len = s_nsplit[task];
    s_nsplit[task] = len >= 0 ? history_splits(a, len, st) : 0;
  }
  __syncthreads();
  const int per = (programs + kT - 1) / kT;
  const int lo_t = min(static_cast<int>(threadIdx.x) * per, programs);
  const int hi_t = min(lo_t + per, programs);
  int fsum = 0, usum = 0;
  for (int task = lo_t; task < hi_t; ++task) {
    const int ns = s_nsplit[task];
    fsum += max(ns - 1, 0);
    usum += ns > 0;
  }
  s_part[0][threadIdx.x] = fsum;
  s_part[1][threadIdx.x] = usum;
  __syncthreads();
  if (threadIdx.x < 2) {
    int acc = 0;
    for (int i = 0; i < kT; ++i) {
      const int x = s_part[threadIdx.x][i];
      s_part[threadIdx.x][i] = acc;
      acc += x;
    }
    s_total[threadIdx.x] = acc;
  }
  __syncthreads();
  int fbase = s_part[0][threadIdx.x], ubase = s_part[1][threadIdx.x];
  for (int task = lo_t; task < hi_t; ++task) {
    const int ns = s_nsplit[task];
    s_full[task] = fbase;
    fbase += max(ns - 1, 0);
    if (ns > 0) s_used[ubase++] = static_cast<int16_t>(task);
  }
  if (threadIdx.x == 0) s_full[programs] = s_total[0];
  __syncthreads();
  const int full = s_total[0], used = s_total[1];
  // Roles: the BF16 branch of each (task, kv head) in two 16-row halves, then the K/V quads.
  const int64_t roles = kRoles ? 2 * static_cast<int64_t>(pre->raw_wgs) + pre->kv_wgs : 0;
  const int64_t units = (static_cast<int64_t>(full) + used) * heads + roles;
  for (;;) {
    if (threadIdx.x == 0) s_claim = atomicAdd(&counters[0], 1);
    __syncthreads();
    int64_t u = s_claim;
    __syncthreads();  // every lane has read the claim (and the previous unit is done)
    if (u >= units) break;
    if constexpr (kRoles) {
      const int64_t bf = 2 * static_cast<int64_t>(pre->raw_wgs);
      const int64_t hist_units = units - roles;
      if (u < bf || u >= bf + hist_units) {
        uint8_t* role_lds = reinterpret_cast<uint8_t*>(&lds);
        if (u < bf) {
          const int r = static_cast<int>(u);
          const int th = r >> 1;  // (task, kv head) as in the pre-attention launch
          raw_block_staged<1>(pre->attn, th / heads, th % heads, 0, role_lds, 2, 16 * (r & 1));
        } else {
          kv_store_role(*pre, static_cast<int>(u - bf - hist_units), role_lds);
        }
        __syncthreads();  // the role's LDS is free for the next unit
        continue;
      }
      u -= bf;
    }
    const int head = static_cast<int>(u % heads);
    const int k = static_cast<int>(u / heads);
    int task, split;
    if (k < full) {
      // The task that holds full split k: the last one whose first full split is <= k.
      int lo = 0, hi = programs - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_full[mid] <= k)
          lo = mid;
        else
          hi = mid - 1;
      }
      task = lo;
      split = k - s_full[task];
    } else {
      task = s_used[k - full];
      split = s_nsplit[task] - 1;
    }
    history_unit_w8<kWaves>(a, task, head, split, st, lds);
  }
  // Unused split slots: LSE -inf for the rows of every task in use.
  for (int task = blockIdx.x; task < programs; task += gridDim.x) {
    const int ns = s_nsplit[task];
    if (ns <= 0) continue;
    Task t;
    if (!read_task(a, t, task)) continue;
    for (int head = 0; head < heads; ++head) write_unused_splits<kT>(a, t, head, ns, a.splits);
  }
  if (threadIdx.x == 0) {
    if (atomicAdd(&counters[1], 1) == static_cast<int>(gridDim.x) - 1) {
      atomicExch(&counters[0], 0);
      atomicExch(&counters[1], 0);
    }
  }
}

template <int kWaves, int kTasks>
__global__ __launch_bounds__(kWaves * kWave, 8 / kWaves) void history_queue_kernel(
    const AttnArgs a, int32_t* counters, int32_t programs) {
  history_queue_body<kWaves, kTasks, false>(a, counters, programs, nullptr);
}

// The MTP step's history launch: the work queue with the pre-attention roles as its first
// units (the counterpart of history_pre_kernel for 17-32 query rows per task).
static_assert(2 * kRawLdsPerSlot <= sizeof(HistoryLdsW8<4>::ring) + sizeof(HistoryLdsW8<4>::qstage),
              "a BF16 role's two ring slots fit the unit's ring and query stage");
static_assert(16 * kHeadDim * 2 <= sizeof(HistoryLdsW8<4>::ring), "the K/V store role's tile fits");
__global__ __launch_bounds__(4 * kWave, 2) void history_queue_pre_kernel(const AttnArgs a,
                                                                         const PreArgs p,
                                                                         int32_t* counters,
                                                                         int32_t programs) {
  history_queue_body<4, kQueueTasks4, true>(a, counters, programs, &p);
}

// ---------------------------------------------------------------- paired-token kernel

// Up to 8 query rows (decode with G <= 8): each QK MFMA covers two 16-token sets on the two
// 64-wide halves of k (block-diagonal operands), so 12 of the 16 score columns are live
// instead of 6 and every lane carries 8 scores of a chunk instead of 16.
//   * Pair tile pt (0, 1) of a chunk: A row i holds token X = 32 pt + i in k < 64 and token
//     Y = 32 pt + 16 + i in k >= 64, 64 head dims per MFMA (block b = dims 64 b .. +63); the
//     query is column j < 8 (row j, k < 64 live) and column j + 8 (row j, k >= 64 live).
//   * Score lane (j, g) holds tokens 32 pt + 16 (j >= 8) + 4 g + v of query row j % 8; lanes
//     j and j ^ 8 share a row, its running max and the row's E8M0 scale of the P operand.
//   * P * V is the 16-row MFMA of the general kernel: P row j (< 8) takes its own 8 tokens
//     and those of lane j + 8 (one row_ror:8 DPP move per dword).
// Operand index maps (f8f6f4 layouts):
//   FP4 A lane (i, G) nibble v: k = 64 (G&1) + 16 (G>>1) + 32 (v/16) + v%16; with raw code
//   dwords 4b + 2 (G>>1) + {0, 1} emitted [even, odd, even, odd] its head dim is
//   64 b + 32 (G>>1) + 16 (v/16) + s(v%16), s(t) = 2 (t%8) + t/8.
//   FP8 B lane (j, G) byte e: k = 32 G + e, live when (j < 8) == (G < 2); head dim
//   64 b + 32 (e/16) + 16 (G&1) + s(e%16). Dword d of it holds dims
//   64 b + 32 (d/4) + 16 (G&1) + 8 (d%2) + ((d/2)%2) + {0, 2, 4, 6}.
//   PV: A lane (j, G) byte e (< 16 hi, +16 lo) is token T(G, e) = 32 ((e/4)%2) + 16 (e/8) +
//   4 G + e%4; B lane group G reads token rows T(2 (G&1), i) and T(2 (G&1) + 1, i).
__host__ __device__ constexpr int pair_token(int ga, int e) {
  return 32 * ((e >> 2) & 1) + 16 * (e >> 3) + 4 * ga + (e & 3);
}
// LDS record slot of chunk token t in the paired kernel: token bits 2-3 XOR bits 4-5 (its own
// inverse). With 144-byte records, tokens 16 apart share banks; a transposed V read takes
// tokens t, t + 16, t + 32 and t + 48 at once, which this map spreads over four bank groups
// (4-way conflicts become 2-way, the floor for this stride). The DMA places token
// pair_slot(r) in slot r, so the copy itself is unchanged.
__host__ __device__ constexpr int pair_slot(int t) { return t ^ (((t >> 4) & 3) << 2); }
static_assert(pair_slot(pair_slot(45)) == 45 && pair_slot(21) == 17, "pair_slot is an involution");
static_assert(kDeviceUnitTasks * 4 <= kRingBytes, "the unit resolver's task list fits the ring");

// kMode 0: the history branch alone (attention_partials).
// kMode 1: the two-launch step's history launch (finish.h): the grid has one more z slice
// (window stores, padded rows), unused split slots are left unwritten (the merge reads only
// the task's splits), and the workgroup that completes a (task, head) finishes its rows.
// kMode 2: the one-launch layer step (layer.h): as 1, and the workgroups also rotate the query
// (a.query is the unrotated query), store the step's INT2 slots, share the BF16 branch, and
// the finisher stores the windows; padded rows are cleared by split 0 of each program.
// kMode 3: as 0, behind `role_slices` z slices of pre-attention roles (pre.h: the BF16 branch
// and the K/V INT2 store of the step), which dispatch first and run beside the history stream.
// kMode 4: as 3, and each workgroup rotates its task's query rows by R_k itself (a.query is
// the unrotated query), with the operands and k order of the rotate entry point (same bits).
// kMode 5: as 3, and q rotation roles of the same launch (pre.h q_rotate_role) write the
// rotated query into a.query: every wavefront requests its first chunks, then wavefront 3
// waits for the roles' tile count and copies the task's rotated rows.
template <int kMode>
__device__ __forceinline__ void history_pair_body(const AttnArgs& a, const FinishArgs* fin,
                                                  const LayerArgs* lay,
                                                  const PreArgs* pre = nullptr,
                                                  int role_slices = 0) {
  constexpr bool kFinish = kMode == 1 || kMode == 2;
  if constexpr (kMode == 1) {
    if (static_cast<int>(blockIdx.z) == a.splits) {
      finish_extra(*fin, blockIdx.y);
      return;
    }
  }
  if constexpr (kMode == 2) {
    if (blockIdx.y == 0 && blockIdx.z == 0) clear_padded_rows(*fin, blockIdx.x);
  }
  __shared__ __attribute__((aligned(16))) uint8_t s_ring[kRingBytes];
  __shared__ uint32_t s_off[kTableCache];
  __shared__ float s_red[3][4][8];  // per wavefront: row max, sum p, sum p z_v
  static_assert(8 * 512 + 4 * 2 * 8 * 16 * 4 <= 2 * kStageBytes,
                "query rows and operand images fit wavefront 3's stages");
  static_assert(4 * 8 * 256 * 4 <= kRingBytes, "the epilogue merge fits the ring");
  static_assert(kFinishLdsBytes <= kRingBytes, "the finisher fits the ring");
  static_assert(kLayerRingBytes <= kRingBytes, "the layer-step finisher fits the ring");
  static_assert(16 * kStageRowBytes + 4 * 2 * 8 * 16 * 4 <= 2 * kStageBytes,
                "the layer step's 16-row staging tile and operand images fit wavefront 3's stages");
  static_assert(16 * kHeadDim * 2 <= kRingBytes, "the K/V store role's tile fits the ring");
  if constexpr (kMode == 3 || kMode == 4 || kMode == 5) {
    const int z = blockIdx.z;
    if (z < role_slices) {
      if (z == 0) {
        raw_block_staged<1>(pre->attn, blockIdx.x, blockIdx.y, 0, s_ring,
                            kRingBytes / kRawLdsPerSlot);
      } else {
        int r = ((z - 1) * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x)) *
                    static_cast<int>(gridDim.y) + static_cast<int>(blockIdx.y);
        if constexpr (kMode == 5) {
          if (r < pre->q_wgs) {
            q_rotate_role(*pre, r, s_ring);
            return;
          }
          r -= pre->q_wgs;
        }
        if (r < pre->kv_wgs) kv_store_role(*pre, r, s_ring);
      }
      return;
    }
  }

  // Layer step: R_k^T operands of the query rotation are requested first (they depend on
  // nothing), so that they arrive with the task metadata.
  u32x4 rb[4][8];
  if constexpr (kMode == 2) load_rt_tiles(lay->rk_t, rb);
  if constexpr (kMode == 4) load_rt_tiles(pre->rk_t, rb);

  Task t;
  const int head = blockIdx.y;
  int split = static_cast<int>(blockIdx.z) - role_slices, nsplit, st = a.split_tokens;
  if (!kFinish && a.split_tokens < 0) {
    // Device rule: this workgroup slot computes unit u of the step's (task, split) units
    // (task-major, the split length derived from the step's lengths); slots past the last
    // unit compute nothing. The last split of a task marks the task's unused split slots
    // (LSE -inf) for the split merges. The ring is free until the first DMA.
    DeviceUnit du;
    const int u = split * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x);
    if (!device_unit<kThreads>(a, static_cast<int>(gridDim.x), u,
                               reinterpret_cast<int*>(s_ring), du))
      return;
    t = du.t;
    split = du.split;
    nsplit = du.nsplit;
    st = du.split_tokens;
    if (split == nsplit - 1) write_unused_splits<kThreads>(a, t, head, nsplit, a.splits);
  } else {
    if (!read_task(a, t, blockIdx.x)) return;
    nsplit = history_splits(a, t.recent_begin - t.sink_len, st);
    if (split >= nsplit) {
      if constexpr (!kFinish) write_unused_split(a, t, head, split);
      return;
    }
  }
  const int length = t.recent_begin - t.sink_len;
  int p_lo, p_hi;
  history_positions(a, t, length, nsplit, split, st, p_lo, p_hi);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int first = p_lo >> 6;
  const int nchunk = p_lo < p_hi ? ((p_hi - 1) >> 6) - first + 1 : 0;
  const int nmine = nchunk > wave ? (nchunk - wave + 3) >> 2 : 0;  // chunks wave + 4 j
  const int kb_first = p_lo >> a.L.bk_shift;

  // ---- DMA plan (as in the general kernel, record slot r holding token pair_slot(r)).
  const uint32_t tok_bytes = static_cast<uint32_t>(a.L.kv_heads) * kSlot;
  uint32_t voff[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int c = 64 * i + lane;
    voff[i] = static_cast<uint32_t>(pair_slot(c / kPieces)) * tok_bytes + 16 * (c % kPieces);
  }
  const uint32_t my_ring = lds_addr(s_ring) + wave * 2 * kStageBytes;
  const uint32_t in_kb_mask = static_cast<uint32_t>(a.L.bk - 1);
  uint32_t valid_bits = 0;
  auto issue = [&](int j, int s) {
    const int t0 = (first + wave + 4 * j) << 6;
    const int local = (t0 >> a.L.bk_shift) - kb_first;
    uint32_t off32 = s_off[min(local, kTableCache - 1)];
    if (local >= kTableCache) off32 = kernel_block_offset(a, t, head, t0 >> a.L.bk_shift);
    off32 = uniform(off32);
    const uint8_t* base = a.history;
    const bool ok = off32 != kNoBlock;
    if (ok)
      base = a.history + (static_cast<uint64_t>(off32) << 5) +
             (static_cast<uint32_t>(t0) & in_kb_mask) * tok_bytes;
    valid_bits = ok ? (valid_bits | (1u << s)) : (valid_bits & ~(1u << s));
    const uint32_t lds = my_ring + s * kStageBytes + kSkew;
#pragma unroll
    for (int i = 0; i < kDma; ++i) dma_x4_stream(base, voff[i], lds + 1024 * i);
  };

  // ---- query rows -> LDS: piece p of row r at r * 32 + (p ^ r), in an area of their own
  // (the FP8 operand images [b][term][r][h][d] replace them once every wavefront has read
  // them), so that every wavefront requests its first chunks at once. Layer step: 16 staged
  // rows in wavefront 3's stages, the query rows 0..7 and, in the workgroups that store them,
  // the current key rows (8..11) and value rows (12..15) of the task's tokens, and the images
  // in the finisher's LDS (free until the end), so that they outlive wavefront 3's stages.
  __shared__ __attribute__((aligned(16))) uint8_t s_q[kMode == 2 ? 16 : 8 * 512];
  static_assert(4 * 2 * 8 * 16 * 4 <= 8 * 512, "the images fit the query rows' area");
  uint8_t* q_lds = kMode == 2 ? s_ring + 6 * kStageBytes : s_q;
  __shared__ __attribute__((aligned(16))) uint8_t s_fin[kMode == 2 ? kLayerFinBytes : 16];
  static_assert(kMode != 2 || 4 * 2 * 8 * 16 * 4 <= kLayerFinBytes, "images fit s_fin");
  uint32_t* q_img = reinterpret_cast<uint32_t*>(kMode == 2 ? s_fin : s_q);
  bool stores_k = false, stores_v = false;
  const int nraw = min(kRawSplits, nsplit);
  if constexpr (kMode == 2) {
    stores_k = split == 4 % nsplit;
    stores_v = split == 5 % nsplit;
  }
  if constexpr (kMode != 5) {
    const int slot = wave * 64 + lane;
    const int row = slot >> 5, piece = (slot & 31) ^ row;
    const RowInfo ri = row_info(a, t, head, row);
    const uint16_t* src =
        ri.valid ? a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 8 * piece : a.query;
    dma_dwordx4(src, lds_addr(q_lds) + 1024 * wave);
    if constexpr (kMode == 2) {
      // Rows 8 + i (keys) and 12 + i (values) of current token i < min(qlen, 4).
      const int row2 = 8 + row, i = row & 3;
      const bool is_v = row >= 4;
      const bool want = (is_v ? stores_v : stores_k) && i < t.qlen;
      const int64_t token = static_cast<int64_t>(t.qstart) + t.qoff + i;
      const int piece2 = (slot & 31) ^ (row2 & 31);
      const uint16_t* src2 =
          want ? (is_v ? a.value + token * a.vs0 + head * a.vs1
                       : a.key + token * a.ks0 + head * a.ks1) + 8 * piece2
               : a.query;
      dma_dwordx4(src2, lds_addr(q_lds) + 4096 + 1024 * wave);
    }
  }
  if (nchunk > 0) {
    const int nkb = min(((p_hi - 1) >> a.L.bk_shift) - kb_first + 1, kTableCache);
    for (int j = threadIdx.x; j < nkb; j += kThreads)
      s_off[j] = kernel_block_offset(a, t, head, kb_first + j);
  }
  OSCAR_WAIT_VM(0);
  __syncthreads();
  if constexpr (kMode == 5) {
    // Every wavefront requests its first chunks, then wavefront 3 waits for the rotated rows
    // and copies them (its wait for the copy also covers its first chunks).
    if (nmine > 0) issue(0, 0);
    if (nmine > 1) issue(1, 1);
    if (wave == 3) {
      for (int poll = 0;; ++poll) {
        const int done = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(pre->qsync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (done >= pre->q_wgs) break;
        if (poll == kQSyncPolls) {
          __hip_atomic_store(pre->qsync + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(8);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int slot = i * 64 + lane;
        const int row = slot >> 5, piece = (slot & 31) ^ row;
        const RowInfo ri = row_info(a, t, head, row);
        const uint16_t* src =
            ri.valid ? a.query + ri.token * a.qs0 + ri.qhead * a.qs1 + 8 * piece : a.query;
        dma_dwordx4_coherent(src, lds_addr(q_lds) + 1024 * i);
      }
      OSCAR_WAIT_VM(0);
    }
    barrier_lds();  // the rotated rows are in LDS
  } else if (kMode != 2 || wave < 3) {
    if (nmine > 0) issue(0, 0);
    if (nmine > 1) issue(1, 1);
  }

  // ---- layer step: rotate the staged rows in place (rows 0..7 and the key rows by R_k, the
  // value rows by R_v), the bits of the rotate entry point. The BF16 branch's wavefront keeps
  // the unrotated query rows (its B operand) in registers.
  const bool raw_wave = kMode == 2 && wave == 3 && split < nraw;
  u32x4 qraw[8];
  if constexpr (kMode == 2) {
    u32x4 aop[8];
    load_stage_a(q_lds, aop);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      qraw[m] = u32x4{0u, 0u, 0u, 0u};
      if (raw_wave && n < 8)
        qraw[m] = *reinterpret_cast<const u32x4*>(q_lds + n * 512 + 16 * ((8 * g + m) ^ n));
    }
    barrier_lds();  // every operand is in registers; the rotated rows replace the staged ones
    rotate_stage(aop, rb, q_lds, 0, stores_k ? 12 : 8);
    if (stores_v) {
      load_rt_tiles(lay->rv_t, rb);
      rotate_stage(aop, rb, q_lds, 12, 16);
    }
    barrier_lds();
  }
  if constexpr (kMode == 4) {
    // Rows 0..7 are staged; rows 8..15 of the tile are zero operands (never written back).
    u32x4 aop[8];
#pragma unroll
    for (int m = 0; m < 8; ++m)
      aop[m] = n < 8 ? *reinterpret_cast<const u32x4*>(q_lds + n * kStageRowBytes +
                                                       16 * ((4 * m + g) ^ n))
                     : u32x4{0u, 0u, 0u, 0u};
    barrier_lds();  // every operand is in registers; the rotated rows replace the staged ones
    rotate_stage(aop, rb, q_lds, 0, 8);
    barrier_lds();
  }

  // ---- row statistics (every wavefront, redundantly): lane l reduces row l / 8 over dims
  // 32 (l % 8) .. +31; the row's power-of-two multiplier puts its max |q| in [128, 256).
  float qmult_l, qsum_l;
  {
    const int row = lane >> 3;
    const bool live = row_info(a, t, head, row).valid;
    float mx = 0.f, qs = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int piece = 4 * (lane & 7) + k;
      const u32x4 w = *reinterpret_cast<const u32x4*>(q_lds + row * 512 + 16 * (piece ^ row));
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const float lo = live ? bf16_to_float(w[x] & 0xffffu) : 0.f;
        const float hi = live ? bf16_to_float(w[x] >> 16) : 0.f;
        mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
        qs += lo + hi;
      }
    }
    mx = fmaxf(mx, dpp<kDppQuadXor1>(mx));
    mx = fmaxf(mx, dpp<kDppQuadXor2>(mx));
    mx = fmaxf(mx, dpp<kDppRowHalfMirror>(mx));
    qs += dpp<kDppQuadXor1>(qs);
    qs += dpp<kDppQuadXor2>(qs);
    qs += dpp<kDppRowHalfMirror>(qs);
    const uint32_t eb = max((__float_as_uint(mx) >> 23) & 0xffu, 7u);
    qmult_l = __uint_as_float((261u - eb) << 23);
    qsum_l = qs;
  }
  // This lane's score row j % 8: FP4 holds c / 2, the score in log2 units is r fq.
  const int my_row = n & 7;
  const float qmult = __shfl(qmult_l, 8 * my_row, kWave);
  const float fq = 2.0f * a.scale_log2 / qmult;
  const float qs2 = 0.5f * __shfl(qsum_l, 8 * my_row, kWave) * qmult;

  // ---- operand images: wavefront w converts head-dim block b = w. Item (r, h, d) = dword d
  // of the live B operand of row r, k half h: FP8 terms of 4 dims, term 1 the residual.
  u32x4 wq[2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int item = 64 * it + lane;
    const int r = item >> 4, h = (item >> 3) & 1, d = item & 7;
    const int piece = 8 * wave + 4 * (d >> 2) + 2 * h + (d & 1);
    wq[it] = *reinterpret_cast<const u32x4*>(q_lds + r * 512 + 16 * (piece ^ r));
  }
  if constexpr (kMode != 2) barrier_lds();  // every wavefront has read the rows the images replace
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int item = 64 * it + lane;
    const int r = item >> 4, h = (item >> 3) & 1, d = item & 7;
    const float mult = __shfl(qmult_l, 8 * r, kWave);
    const bool live = row_info(a, t, head, r).valid;  // padding rows stage the wrong bytes
    const u32x4 w = wq[it];
    const bool odd = (d >> 1) & 1;
    float v[4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
      v[x] = live ? bf16_to_float(odd ? (w[x] >> 16) : (w[x] & 0xffffu)) * mult : 0.f;
    const uint32_t t0 = fp8x4_take(v);
    const uint32_t t1 = fp8x4(v[0], v[1], v[2], v[3]);
    q_img[((wave * 2 + 0) * 8 + r) * 16 + h * 8 + d] = t0;
    q_img[((wave * 2 + 1) * 8 + r) * 16 + h * 8 + d] = t1;
  }
  barrier_lds();
  i32x8 qb[4][kQTerms];
  auto load_qb = [&]() {
    const bool live = (n < 8) == (g < 2);
    const int h = g & 1;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int term = 0; term < kQTerms; ++term) {
        const u32x4* src =
            reinterpret_cast<const u32x4*>(q_img + ((b * 2 + term) * 8 + my_row) * 16 + h * 8);
        const u32x4 lo = src[0], hi = src[1];
        qb[b][term] = live ? i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                                   (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]}
                           : i32x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
  };
  // The layer step loads them after its BF16-branch share (fewer registers live there).
  if constexpr (kMode != 2) load_qb();
  // Layer step: wavefront i keeps the rotated key / value row of current token i (if this
  // workgroup stores it) before wavefront 3's stages are reused.
  const int kv_rows = min(t.qlen, 4);
  const bool do_k = stores_k && wave < kv_rows, do_v = stores_v && wave < kv_rows;
  float kx[4], vx[4];
  if constexpr (kMode == 2) {
    if (do_k) stage_row_floats(q_lds, 8 + wave, kx);
    if (do_v) stage_row_floats(q_lds, 12 + wave, vx);
  }
  if constexpr (kMode == 2) {
    barrier_lds();  // everyone is done with wavefront 3's stages
    if (wave == 3) {
      if (nmine > 0) issue(0, 0);
      if (nmine > 1) issue(1, 1);
    }
  }
  if constexpr (kMode == 2) {
    // INT2 store of the step's own key / value rows (store_int2 semantics), then this split's
    // share of the BF16 branch, while the first chunks are in flight.
    const int64_t token = static_cast<int64_t>(t.qstart) + t.qoff + wave;
    if (do_k) store_int2_row(a, *lay, token, head, false, kx);
    if (do_v) store_int2_row(a, *lay, token, head, true, vx);
    if (raw_wave) {
      const int first_blk =
          a.table_columns > 0 ? a.table[static_cast<int64_t>(t.req) * a.table_stride] : -1;
      RawTask r;
      r.high = t.sink_len + t.prefix - t.recent_begin;
      r.win = -1;
      if (first_blk >= 0) {
        const int64_t owner = fastdiv(static_cast<uint32_t>(first_blk), a.L.bpp_div);
        r.win = owner * (a.L.page_bytes / 2) + static_cast<int64_t>(head) * kHeadDim;
      }
      raw_share(a, *lay, t, r, head, split, nraw, qraw);
    }
    load_qb();
  }

  // ---- per-lane LDS offsets inside a stage (token t's record starts at kSkew + 144
  // pair_slot(t))
  const int side = n >> 3;  // 0: X tokens, 1: Y tokens of each pair tile
  // QK A operand: token i + 16 (G&1) + 32 pt of the pair tile, code dwords 4b + 2 (G>>1), +1.
  int k_off[2];
#pragma unroll
  for (int pt = 0; pt < 2; ++pt)
    k_off[pt] = kSkew + kRec * pair_slot(n + 16 * (g & 1) + 32 * pt) + 8 * (g >> 1);
  // Scale|zero of this lane's score tokens 32 h + 16 side + 4 g + v (v < 4: bits 0-1 are
  // left alone by pair_slot, so v stays an immediate offset).
  int sz_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    sz_off[h] = kSkew + kRec * pair_slot(32 * h + 16 * side + 4 * g) + 64;
  // Transposed V reads: token rows T(2 (g&1), n) and T(2 (g&1) + 1, n) = T(2 (g&1), n) + 4.
  int v_off[2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
    v_off[r] = kSkew + kRec * pair_slot(pair_token(2 * (g & 1), n) + 4 * r) + kVector;

  float m = -INFINITY, psum = 0.f, zsum = 0.f;
  f32x4 o[16];  // o[2c + par]: rows 4g + v, dim 32c + 2n + par (units of c/2)
#pragma unroll
  for (int c = 0; c < 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](int j, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    const uint8_t* st = s_ring + wave * 2 * kStageBytes + S * kStageBytes;
    // Scores: two pair tiles, four head-dim blocks, kQTerms query terms.
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      i32x8 kf[2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        const uint32_t* kp = reinterpret_cast<const uint32_t*>(st + k_off[pt] + 16 * b);
        const uint32_t w0 = kp[0], w1 = kp[1];
        kf[pt] = i32x8{even_codes(w0), odd_codes(w0), even_codes(w1), odd_codes(w1), 0, 0, 0, 0};
      }
#pragma unroll
      for (int term = 0; term < kQTerms; ++term)
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) acc[pt] = mfma_qk(kf[pt], qb[b][term], acc[pt]);
    }
    uint32_t ksz[8], vsz[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int off = sz_off[e >> 2] + kRec * (e & 3);
      ksz[e] = *reinterpret_cast<const uint32_t*>(st + off);
      vsz[e] = *reinterpret_cast<const uint32_t*>(st + off + kVector);
    }
    float r2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r2[e] = fmaf(h16lo(ksz[e]), acc[e >> 2][e & 3], h16hi(ksz[e]) * qs2);
    const int t0 = (first + wave + 4 * j) << 6;
    const bool ok_block = (valid_bits >> S) & 1u;
    if (!(ok_block && t0 >= p_lo && t0 + kChunk <= p_hi)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = 32 * (e >> 2) + 16 * side + 4 * g + (e & 3);
        const bool ok = ok_block && static_cast<uint32_t>(t0 + tok - p_lo) <
                                        static_cast<uint32_t>(p_hi - p_lo);
        vsz[e] = ok ? vsz[e] : 0u;
        r2[e] = ok ? r2[e] : -INFINITY;
      }
    }
    // Lazy running max, shared by the lanes of a row: j, j ^ 8 and all four lane groups.
    float lm = r2[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) lm = fmaxf(lm, r2[e]);
    lm *= fq;
    if (__any(lm > m + kTheta)) {
      float v = fmaxf(lm, dpp<kDppRowRor8>(lm));
      v = max_xor32(max_xor16(v));
      const float mn = fmaxf(m, v);
      const float alpha = mn == -INFINITY ? 1.0f : exp2f(m - mn);
      m = mn;
      psum *= alpha;
      zsum *= alpha;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const float av = __shfl(alpha, 4 * g + v4, kWave);  // accumulator row 4g + v4
#pragma unroll
        for (int c = 0; c < 16; ++c) o[c][v4] *= av;
      }
    }
    // P operand: p s_v as FP8 hi + lo with one E8M0 scale per query row (the scale of k
    // block kb comes from lane group kb, while FP8 lane group G holds its hi bytes in block
    // G / 2 and its lo bytes in block 2 + G / 2, so a per-lane scale would mix rows' data).
    const float nm = m == -INFINITY ? 0.f : -m;
    float av[8];
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(fmaf(r2[e], fq, nm));
      psum += p;
      zsum = fmaf(p, h16hi(vsz[e]), zsum);
      av[e] = p * h16lo(vsz[e]);
      amax = fmaxf(amax, av[e]);
    }
    amax = max_xor32(max_xor16(fmaxf(amax, dpp<kDppRowRor8>(amax))));
    const uint32_t eb = max(__float_as_uint(amax) >> 23, 7u);
    const float mult = __uint_as_float((260u - eb) << 23);
    const int sa = static_cast<int>(eb) - 6;
    uint32_t hi[2], lo[2];
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      float x[4] = {av[4 * pt] * mult, av[4 * pt + 1] * mult, av[4 * pt + 2] * mult,
                    av[4 * pt + 3] * mult};
      hi[pt] = fp8x4_take(x);
      lo[pt] = fp8x4(x[0], x[1], x[2], x[3]);
    }
    const i32x8 pa = i32x8{(int)hi[0], (int)hi[1], (int)dpp_u32<kDppRowRor8>(hi[0]),
                           (int)dpp_u32<kDppRowRor8>(hi[1]), (int)lo[0], (int)lo[1],
                           (int)dpp_u32<kDppRowRor8>(lo[0]), (int)dpp_u32<kDppRowRor8>(lo[1])};
    // O += P V over the chunk's 64 tokens, 32 dims (16 dim pairs) per transposed read pair.
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const i32x2 r0 =
          __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off[0] + 8 * c));
      const i32x2 r1 =
          __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(st + v_off[1] + 8 * c));
      const i32x8 be = i32x8{even_codes(r0[0]), even_codes(r0[1]), even_codes(r1[0]),
                             even_codes(r1[1]), 0, 0, 0, 0};
      const i32x8 bo = i32x8{odd_codes(r0[0]), odd_codes(r0[1]), odd_codes(r1[0]),
                             odd_codes(r1[1]), 0, 0, 0, 0};
      o[2 * c] = mfma_pv(pa, be, o[2 * c], sa);
      o[2 * c + 1] = mfma_pv(pa, bo, o[2 * c + 1], sa);
    }
  };

  // ---- token loop, two chunks (one per ring stage) per iteration: wait for chunk j,
  // consume it, refill its stage with chunk j + 2.
  int j = 0;
  for (; j + 1 < nmine; j += 2) {
    OSCAR_WAIT_VM(kDma);
    process(j, std::integral_constant<int, 0>());
    if (j + 2 < nmine) {
      OSCAR_WAIT_LGKM();
      issue(j + 2, 0);
      OSCAR_WAIT_VM(kDma);
    } else {
      OSCAR_WAIT_VM(0);
    }
    process(j + 1, std::integral_constant<int, 1>());
    if (j + 3 < nmine) {
      OSCAR_WAIT_LGKM();
      issue(j + 3, 1);
    }
  }
  if (j < nmine) {
    OSCAR_WAIT_VM(0);
    process(j, std::integral_constant<int, 0>());
  }

  // ---- epilogue: row totals over the lanes of a row, then the four wavefront states.
  // Lane indices are recomputed here (mbcnt) so that none stays live across the token loop.
  const int el = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
  const int etid = wave * 64 + el, en = el & 15, eg = el >> 4;
  psum += dpp<kDppRowRor8>(psum);
  zsum += dpp<kDppRowRor8>(zsum);
  psum = sum_xor32(sum_xor16(psum));
  zsum = sum_xor32(sum_xor16(zsum));
  if (el < 8) {
    s_red[0][wave][el] = m;
    s_red[1][wave][el] = psum;
    s_red[2][wave][el] = zsum;
  }
  __syncthreads();  // every chunk consumed; the ring is free for the merge
  float* s_o = reinterpret_cast<float*>(s_ring);  // [wave][row 0..7][256]
  if (eg < 2) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 4 * eg + v;
      const float mx = fmaxf(fmaxf(s_red[0][0][row], s_red[0][1][row]),
                             fmaxf(s_red[0][2][row], s_red[0][3][row]));
      const float mw = s_red[0][wave][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - mx);
      float* dst = s_o + (wave * 8 + row) * 256 + 2 * en;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *reinterpret_cast<float2*>(dst + 32 * c) =
            make_float2(o[2 * c][v] * f, o[2 * c + 1][v] * f);
    }
  }
  __syncthreads();
  // Thread -> (row, dims 4 (tid % 32) + 128 q): 32 threads write 512 contiguous bytes.
  const int row = etid >> 5, d0 = 4 * (etid & 31);
  const RowInfo ri = row_info(a, t, head, row);
  if (ri.valid) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_red[0][w][row]);
    float den = 0.f, zs = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = s_red[0][w][row];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - mx);
      den = fmaf(f, s_red[1][w][row], den);
      zs = fmaf(f, s_red[2][w][row], zs);
    }
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    float* out = a.partials + ((ri.token * a.hq + ri.qhead) * a.splits + split) * kHeadDim + d0;
    const float4* so = reinterpret_cast<const float4*>(s_o + row * 256 + d0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float4 x0 = so[32 * q], x1 = so[8 * 256 / 4 + 32 * q];
      const float4 x2 = so[2 * 8 * 256 / 4 + 32 * q], x3 = so[3 * 8 * 256 / 4 + 32 * q];
      const float4 r = make_float4((2.0f * ((x0.x + x1.x) + (x2.x + x3.x)) + zs) * inv,
                                   (2.0f * ((x0.y + x1.y) + (x2.y + x3.y)) + zs) * inv,
                                   (2.0f * ((x0.z + x1.z) + (x2.z + x3.z)) + zs) * inv,
                                   (2.0f * ((x0.w + x1.w) + (x2.w + x3.w)) + zs) * inv);
      if constexpr (kFinish)
        store_coherent(out + 128 * q, r);
      else
        *reinterpret_cast<float4*>(out + 128 * q) = r;
    }
    if ((etid & 31) == 0) {
      float* dst = a.lse + (ri.token * a.hq + ri.qhead) * a.splits + split;
      const float l = den > 0.f ? (mx + log2f(den)) * kLn2 : -INFINITY;
      if constexpr (kFinish)
        store_coherent(dst, l);
      else
        *dst = l;
    }
  }
  if constexpr (kFinish) {
    __shared__ int s_flag;
    int32_t* counter = fin->counters + static_cast<int64_t>(blockIdx.x) * a.L.kv_heads + head;
    if (finish_arrive(counter, nsplit, &s_flag)) {
      if constexpr (kMode == 1) {
        finish_task8(*fin, a, t, head, nsplit, s_ring);
      } else {
        finish_layer8(*fin, *lay, a, t, head, nsplit, nraw, s_ring, s_fin);
        // Every split of the task, and so every read of its window, is done.
        store_window_request(fin->p.win, t.req, head);
      }
    }
  }
}

__global__ __launch_bounds__(kThreads, 2) void history_pair_kernel(const AttnArgs a) {
  history_pair_body<0>(a, nullptr, nullptr);
}

struct HistoryFinishArgs {
  AttnArgs a;
  FinishArgs f;
};

__global__ __launch_bounds__(kThreads, 2) void history_pair_finish_kernel(const HistoryFinishArgs h) {
  history_pair_body<1>(h.a, &h.f, nullptr);
}

struct LayerStepArgs {
  AttnArgs a;
  FinishArgs f;
  LayerArgs l;
};

__global__ __launch_bounds__(kThreads, 2) void layer_step_kernel(const LayerStepArgs h) {
  history_pair_body<2>(h.a, &h.f, &h.l);
}

struct HistoryPreArgs {
  AttnArgs a;
  PreArgs p;
  int32_t role_slices;
};

__global__ __launch_bounds__(kThreads, 2) void history_pre_kernel(const HistoryPreArgs h) {
  history_pair_body<3>(h.a, nullptr, nullptr, &h.p, h.role_slices);
}
__global__ __launch_bounds__(kThreads, 2) void history_pre_rot_kernel(const HistoryPreArgs h) {
  history_pair_body<4>(h.a, nullptr, nullptr, &h.p, h.role_slices);
}
__global__ __launch_bounds__(kThreads, 2) void history_pre_q_kernel(const HistoryPreArgs h) {
  history_pair_body<5>(h.a, nullptr, nullptr, &h.p, h.role_slices);
  if (threadIdx.x == 0)
    q_sync_leave(h.p.qsync, static_cast<int>(gridDim.x * gridDim.y * gridDim.z));
}

}  // namespace

hipError_t launch_history(const AttnArgs& a, dim3 grid, int rows, hipStream_t stream,
                          int32_t* queue) {
  if (rows <= 8) {
    hipLaunchKernelGGL(history_pair_kernel, grid, dim3(kThreads), 0, stream, a);
  } else if (rows <= 16) {
    hipLaunchKernelGGL(history_kernel<1>, grid, dim3(kThreads), 0, stream, a);
  } else {
    // Four-wavefront workgroups (two per CU) up to kQueueTasks4 task rows, eight-wavefront
    // ones above; the grid and queue forms take the same size, so they give the same bits.
    const bool four = static_cast<int64_t>(grid.x) <= kQueueTasks4;
    if (queue != nullptr && a.split_tokens != 0 &&
        static_cast<int64_t>(grid.x) <= kQueueTasks) {
      int device = 0, cus = 0;
      hipError_t e = hipGetDevice(&device);
      if (e == hipSuccess)
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
      if (e != hipSuccess) return e;
      const int64_t units = static_cast<int64_t>(grid.x) * grid.y * grid.z;
      const int64_t cap = (cus > 0 ? cus : 1) * (four ? 2 : 1);
      const unsigned wgs = static_cast<unsigned>(units < cap ? units : cap);
      if (four)
        hipLaunchKernelGGL((history_queue_kernel<4, kQueueTasks4>), dim3(wgs), dim3(4 * kWave), 0,
                           stream, a, queue, static_cast<int32_t>(grid.x));
      else
        hipLaunchKernelGGL((history_queue_kernel<8, kQueueTasks>), dim3(wgs), dim3(kThreadsW8), 0,
                           stream, a, queue, static_cast<int32_t>(grid.x));
    } else if (four) {
      hipLaunchKernelGGL(history_w8_kernel<4>, grid, dim3(4 * kWave), 0, stream, a);
    } else {
      hipLaunchKernelGGL(history_w8_kernel<8>, grid, dim3(kThreadsW8), 0, stream, a);
    }
  }
  return hipGetLastError();
}

hipError_t launch_history_queue_pre(const AttnArgs& a, const PreArgs& p, int32_t* queue,
                                    int32_t programs, hipStream_t stream) {
  int device = 0, cus = 0;
  hipError_t e = hipGetDevice(&device);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return e;
  const unsigned wgs = static_cast<unsigned>(2 * (cus > 0 ? cus : 1));  // two per CU
  hipLaunchKernelGGL(history_queue_pre_kernel, dim3(wgs), dim3(4 * kWave), 0, stream, a, p,
                     queue, programs);
  return hipGetLastError();
}

hipError_t launch_history_pre(const AttnArgs& a, const PreArgs& p, int role_slices, dim3 grid,
                              bool rotate_query, hipStream_t stream) {
  const HistoryPreArgs h{a, p, role_slices};
  if (p.qsync)
    hipLaunchKernelGGL(history_pre_q_kernel, grid, dim3(kThreads), 0, stream, h);
  else if (rotate_query)
    hipLaunchKernelGGL(history_pre_rot_kernel, grid, dim3(kThreads), 0, stream, h);
  else
    hipLaunchKernelGGL(history_pre_kernel, grid, dim3(kThreads), 0, stream, h);
  return hipGetLastError();
}

hipError_t launch_layer_step(const AttnArgs& a, const FinishArgs& f, const LayerArgs& l,
                             hipStream_t stream) {
  const LayerStepArgs h{a, f, l};
  const dim3 grid(static_cast<unsigned>(f.programs), static_cast<unsigned>(a.L.kv_heads),
                  static_cast<unsigned>(a.splits));
  hipLaunchKernelGGL(layer_step_kernel, grid, dim3(kThreads), 0, stream, h);
  return hipGetLastError();
}

hipError_t launch_history_finish(const AttnArgs& a, const FinishArgs& f, hipStream_t stream) {
  const HistoryFinishArgs h{a, f};
  const dim3 grid(static_cast<unsigned>(f.programs), static_cast<unsigned>(a.L.kv_heads),
                  static_cast<unsigned>(a.splits + 1));
  hipLaunchKernelGGL(history_pair_finish_kernel, grid, dim3(kThreads), 0, stream, h);
  return hipGetLastError();
}

}  // namespace oscar
