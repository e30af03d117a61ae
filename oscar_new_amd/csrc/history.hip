// Split-KV paged decode attention over the INT2 history, on gfx950 FP4 x FP8 MFMA
// (v_mfma_f32_16x16x128_f8f6f4).
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
//   * The other operand is FP8 (OCP e4m3): the rotated query as a sum of three FP8 terms
//     after a power-of-two row scaling (relative error ~2^-12), and p_t s_v,t as two terms
//     (hi + lo) with an E8M0 scale per (query row, 32 tokens) applied by the MFMA itself.
//   * A workgroup (4 wavefronts) walks its split in chunks of 128 tokens = 4 sub-blocks of
//     32. Wavefront w computes the scores of sub-block w (S^T = K Q^T: the MFMA output keeps
//     one query row per lane, so softmax statistics stay lane-local), publishes FP8
//     probabilities to LDS, and then every wavefront multiplies all 128 of them into its own
//     quarter of the head dimension (64 dims). The V codes of that quarter are transposed
//     on the way out of LDS by ds_read_b64_tr_b4. Each output dim has exactly one owner, so
//     the epilogue needs no cross-wavefront reduction of the accumulators.
//   * The running max is shared by the workgroup and updated lazily: only a chunk in which
//     some score exceeds it by more than 2^8 exchanges row maxima and rescales.
//   * Sub-blocks arrive by direct-to-LDS DMA (global_load_lds_dwordx4, five 16-byte loads per
//     lane per sub-block, SGPR base + per-lane offset) as 32 whole 160-byte records placed 4
//     bytes past a 16-byte boundary, which puts every V code row (record byte 68) on the
//     8-byte alignment the transposed reads need. Three chunks are in flight per workgroup.
#include "attention.h"

namespace oscar {
namespace {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(3))) i32x2* lds_i32x2_ptr_t;
typedef __attribute__((address_space(3))) const uint32_t* lds_u32_ptr_t;

constexpr int kSub = 32;                       // tokens per sub-block
constexpr int kSkew = 4;                       // image offset: V codes (byte 68) 8-aligned
constexpr int kSubBytes = kSub * kSlot + 16;   // 5136: 32 records + skew, 16-byte multiple
constexpr int kDmaPerSub = kSub * kSlot / 1024;  // 5 loads of 16 bytes per lane
constexpr int kStageBytes = 4 * kSubBytes;     // one 128-token chunk
constexpr int kStages = 3;
constexpr int kPRow = 144;                   // FP8 probability row: 128 tokens + 16 (banks)
constexpr float kTheta = 8.0f;               // lazy-max slack, log2 units
constexpr int kQTerms = 3;
constexpr int kTableCache = 2048;            // kernel blocks whose offsets are cached in LDS
constexpr uint32_t kNoBlock = 0xffffffffu;

static_assert(kDmaPerSub * 1024 == kSub * kSlot, "sub-block image is whole DMA instructions");

// ---------------------------------------------------------------- asm plumbing

// Direct-to-LDS loads are issued by asm so that the compiler does not serialize every LDS
// read behind all outstanding DMA (it cannot tell pipeline stages apart); ordering is by
// the explicit vmcnt waits below. M0 holds the LDS base (any dword address); one wait state
// separates its write from the DMA. Lane l writes LDS bytes [lds + 16 l, +16).
__device__ __forceinline__ void dma_x4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" : : "{m0}"(lds), "v"(voff), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma_dwordx4(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "{m0}"(lds), "v"(src)
               : "memory");
}
#define OSCAR_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")

// Workgroup barrier that waits for this wavefront's LDS traffic but not for its DMA.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)p));
}

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
// O tile += 2^(sa - 127) P (FP8, A) x V (FP4, B); K = 128 tokens; sa: this lane's E8M0 byte,
// the scale of row n over the 32 k of FP4 lane group g (sub-block g, see the index maps).
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

// Operand index maps (fixed by the f8f6f4 MFMA operand layouts on gfx950):
//   FP8 operand: lane (row l%16, group G = l/16) byte e holds k = 32 G + e.
//   FP4 operand: lane group G nibble i holds k = 64 (G&1) + 16 (G>>1) + 32 (i/16) + i%16.
//   E8M0 scale of lane (row m, group G) applies to the k of FP4 lane group G, i.e. to FP8
//   bytes e of lane group G' with 2 (e/16) + (G'>>1) = G.
// QK (k = head dim within a 128-dim half h): K lane group G reads code dwords 8h + 2G and
// 8h + 2G + 1 (d = 128h + 32G .. +31) and emits [even, odd, even, odd] nibble dwords, so
// B byte e of lane group G holds q[d], d = 128h + 64 (e/16) + 16 G + sigma(e%16),
// sigma(j) = 2 (j%8) + j/8. PV (k = token within the chunk): the scale blocks are made to
// coincide with sub-blocks -- FP4 lane group G nibble i is token 32 G + i (the transposed V
// read of lane group G, pass R, row j fetches token 16 R + j of sub-block G), so FP8 bytes
// 0-15 of lane group G' are tokens 16 G' + 0..15 and bytes 16-31 are tokens 64 + 16 G' + 0..15
// of the token-ordered P row.
template <int RT>
__global__ __launch_bounds__(kThreads, 3 - RT) void history_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_stage[kStages * kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t s_p[2][2][RT * 16 * kPRow];  // [buf][hi/lo]
  __shared__ int32_t s_scale[2][RT * 16][4];                                  // [buf][row][sub]
  __shared__ uint32_t s_flag[2][4];                                           // [buf][wave]
  __shared__ float s_red[3][4][RT * 16];  // row max / sum p / sum p z_v, per wavefront
  __shared__ uint32_t s_off[kTableCache];
  static_assert(RT * 16 * 512 <= kStageBytes, "query staging fits one stage");

  Task t;
  if (!read_task(a, t)) return;
  const int head = blockIdx.y, split = blockIdx.z;
  int begin, end;
  split_range(t.recent_begin - t.sink_len, a.block_n, a.splits, split, begin, end);
  const int p_lo = max(t.sink_len + begin, 0), p_hi = t.sink_len + end;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int first = p_lo >> 5;
  const int nblk = p_lo < p_hi ? ((p_hi - 1) >> 5) - first + 1 : 0;
  const int nchunk = (nblk + 3) >> 2;
  const int kb_first = p_lo >> a.L.bk_shift;
  // ---- DMA plan: 16-byte piece c = 64 i + lane of a sub-block is record c / 10, bytes
  // 16 (c % 10); records of one head are tok_bytes apart in the kernel block.
  const uint32_t tok_bytes = static_cast<uint32_t>(a.L.kv_heads) * kSlot;
  uint32_t voff[kDmaPerSub];
#pragma unroll
  for (int i = 0; i < kDmaPerSub; ++i) {
    const int c = 64 * i + lane;
    voff[i] = static_cast<uint32_t>(c / 10) * tok_bytes + 16 * (c % 10);
  }
  const uint32_t stage_lds = lds_addr(s_stage);
  const uint32_t in_kb_mask = static_cast<uint32_t>(a.L.bk - 1);
  uint32_t valid_bits = 0;
  // Chunk j, this wavefront's sub-block -> stage. Always 5 loads (an in-bounds dummy block
  // when out of range), so the number of loads younger than any chunk is a constant.
  auto issue = [&](int j, int stage) {
    const int ib = 4 * j + wave;
    const uint8_t* base = a.history;
    bool ok = false;
    if (ib < nblk) {
      const int t0 = (first + ib) << 5;
      const int local = (t0 >> a.L.bk_shift) - kb_first;
      uint32_t off32 = ((lds_u32_ptr_t)s_off)[min(local, kTableCache - 1)];
      if (local >= kTableCache) off32 = kernel_block_offset(a, t, head, t0 >> a.L.bk_shift);
      off32 = uniform(off32);
      if (off32 != kNoBlock) {
        ok = true;
        base = a.history + (static_cast<uint64_t>(off32) << 5) +
               (static_cast<uint32_t>(t0) & in_kb_mask) * tok_bytes;
      }
    }
    valid_bits = ok ? (valid_bits | (1u << stage)) : (valid_bits & ~(1u << stage));
    const uint32_t lds = stage_lds + stage * kStageBytes + wave * kSubBytes + kSkew;
#pragma unroll
    for (int i = 0; i < kDmaPerSub; ++i) dma_x4(base, voff[i], lds + 1024 * i);
  };

  // ---- query rows -> LDS, in the last stage (its first chunk is issued once the query has
  // been converted). 16-byte piece p of row r sits at position r * 32 + (p ^ (r & 31)), so
  // the column reads below spread over all banks. Issued before the block-table reads so
  // that the two latencies overlap.
  uint8_t* q_lds = s_stage + (kStages - 1) * kStageBytes;
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
  // Kernel-block offsets of the split. The compiler's wait for these loads also covers the
  // query DMA issued before them (vector-memory loads complete in order).
  if (nblk > 0) {
    const int nkb = min(((p_hi - 1) >> a.L.bk_shift) - kb_first + 1, kTableCache);
    for (int j = threadIdx.x; j < nkb; j += kThreads)
      s_off[j] = kernel_block_offset(a, t, head, kb_first + j);
  }
  OSCAR_WAIT_VM(0);
  __syncthreads();
  static_assert(kStages == 3, "the prologue and the loop's DMA waits assume 3 stages");
#pragma unroll
  for (int k = 0; k < kStages - 1; ++k) issue(k, k);

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
  static_assert(2 * kQTerms * 64 * 32 <= kStageBytes, "query operands fit one stage");

  // ---- per-lane LDS offsets (record t of a sub-block starts at kSkew + 160 t)
  // QK A operand: token 16 tt + n, code dwords 8h + 2g, +1.
  const int k_off = kSkew + kSlot * n + 8 * g;
  // Score-layout tokens of this lane: tok(e) = 16 (e/4) + 4g + e%4; K scale|zero at record
  // byte 64, V scale|zero at 132.
  const int sz_off = kSkew + kSlot * 4 * g + 64;
  // Transposed V reads: pass R fetches token 16 R + n of sub-block g (codes at byte 68).
  const int v_off0 = g * kSubBytes + kSkew + kVector + kSlot * n;
  const int v_off1 = v_off0 + 16 * kSlot;
  const int dcol = 16 * wave;  // byte offset of this wavefront's 64 dims in a V code row

  float m[RT], psum[RT], zsum[RT];
  f32x4 o[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = -INFINITY;
    psum[rt] = 0.f;
    zsum[rt] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  barrier_lds();  // everyone is done with the query staging area (the last stage)
  issue(kStages - 1, kStages - 1);

  // ---- per-chunk pieces. Chunk j lives in stage j % 3; its probabilities in buffer j & 1.
  // Scores of this wavefront's sub-block of chunk j: S^T = K Q^T, two 16-token tiles.
  auto qk = [&](int j, f32x4 (&acc)[RT][2]) {
    const uint8_t* mine = s_stage + (j % kStages) * kStageBytes + wave * kSubBytes;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) acc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      i32x8 kf[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const uint32_t* kp =
            reinterpret_cast<const uint32_t*>(mine + k_off + 16 * kSlot * tt + 32 * h);
        const uint32_t w0 = kp[0], w1 = kp[1];  // 4-byte aligned: two dword reads
        kf[tt] = i32x8{even_codes(w0), odd_codes(w0), even_codes(w1), odd_codes(w1), 0, 0, 0, 0};
      }
#pragma unroll
      for (int term = 0; term < kQTerms; ++term)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][tt] = mfma_qk(kf[tt], qb[rt][h][term], acc[rt][tt]);
    }
  };

  // Per-token state of the chunk being scored (this lane's 8 tokens).
  float r2[RT][8];   // scores, raw units (-inf: masked)
  float p[RT][8];    // probabilities against the shared max
  float lm[RT];      // lane max of r2 * fq (log2 units)
  uint32_t vsz[8];   // V scale | zero (zeroed when masked)

  // Scores of chunk j from acc; the lazy-max vote goes to s_flag[j & 1].
  auto score = [&](int j, const f32x4 (&acc)[RT][2]) {
    const uint8_t* mine = s_stage + (j % kStages) * kStageBytes + wave * kSubBytes;
    uint32_t ksz[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int off = sz_off + kSlot * (16 * (e >> 2) + (e & 3));
      ksz[e] = *reinterpret_cast<const uint32_t*>(mine + off);
      vsz[e] = *reinterpret_cast<const uint32_t*>(mine + off + kVector);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        r2[rt][e] = fmaf(h16lo(ksz[e]), acc[rt][e >> 2][e & 3], h16hi(ksz[e]) * qs2[rt]);
    // Only the first/last sub-block of a split (or one whose kernel block is unmapped) is
    // partial: its tokens outside [p_lo, p_hi) get score -inf and a zero V scale/zero (the
    // bytes of unwritten slots may hold NaN patterns).
    const int t0 = (first + 4 * j + wave) << 5;
    const bool sub_ok = (valid_bits >> (j % kStages)) & 1u;
    if (!(sub_ok && t0 >= p_lo && t0 + kSub <= p_hi)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = 16 * (e >> 2) + 4 * g + (e & 3);
        const bool ok = sub_ok && static_cast<uint32_t>(t0 + tok - p_lo) <
                                      static_cast<uint32_t>(p_hi - p_lo);
        vsz[e] = ok ? vsz[e] : 0u;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) r2[rt][e] = ok ? r2[rt][e] : -INFINITY;
      }
    }
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v = fmaxf(fmaxf(r2[rt][0], r2[rt][1]), fmaxf(r2[rt][2], r2[rt][3]));
      v = fmaxf(v, fmaxf(fmaxf(r2[rt][4], r2[rt][5]), fmaxf(r2[rt][6], r2[rt][7])));
      lm[rt] = v * fq[rt];
      need |= lm[rt] > m[rt] + kTheta;
    }
    s_flag[j & 1][wave] = __any(need) ? 1u : 0u;
  };

  // Probabilities of chunk j against the shared max -> FP8 hi/lo + E8M0 scale per
  // (row, sub-block) in buffer j & 1.
  auto publish = [&](int j) {
    const int buf = j & 1;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float nm = m[rt] == -INFINITY ? 0.f : -m[rt];
      float av[8];
      float amax = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[rt][e] = __builtin_amdgcn_exp2f(fmaf(r2[rt][e], fq[rt], nm));
        av[e] = p[rt][e] * h16lo(vsz[e]);
        amax = fmaxf(amax, fabsf(av[e]));
      }
      amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
      // mult = 2^(133 - eb) puts the block max in [64, 128); the MFMA scales back by
      // 2^(eb - 133) = E8M0 byte eb - 6.
      const uint32_t eb = max(__float_as_uint(amax) >> 23, 7u);
      const float mult = __uint_as_float((260u - eb) << 23);
      const int prow = (16 * rt + n) * kPRow + 32 * wave + 4 * g;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float x[4] = {av[4 * tt] * mult, av[4 * tt + 1] * mult, av[4 * tt + 2] * mult,
                      av[4 * tt + 3] * mult};
        const uint32_t hi = fp8x4_take(x);
        const uint32_t lo = fp8x4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<uint32_t*>(&s_p[buf][0][prow + 16 * tt]) = hi;
        *reinterpret_cast<uint32_t*>(&s_p[buf][1][prow + 16 * tt]) = lo;
      }
      s_scale[buf][16 * rt + n][wave] = static_cast<int32_t>(eb) - 6;
    }
  };

  // Row maxima agreed by the four wavefronts (each brings the max of its sub-block, lm);
  // the accumulators, which hold earlier chunks only, are rescaled to the new max.
  auto agree_max = [&]() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v = lm[rt];
      v = fmaxf(v, __shfl_xor(v, 16, kWave));
      v = fmaxf(v, __shfl_xor(v, 32, kWave));
      if (g == 0) s_red[0][wave][16 * rt + n] = v;
    }
    barrier_lds();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = 16 * rt + n;
      const float bm = fmaxf(fmaxf(s_red[0][0][row], s_red[0][1][row]),
                             fmaxf(s_red[0][2][row], s_red[0][3][row]));
      const float mn = fmaxf(m[rt], bm);
      const float alpha = mn == -INFINITY ? 1.0f : exp2f(m[rt] - mn);
      m[rt] = mn;
      psum[rt] *= alpha;
      zsum[rt] *= alpha;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float av = __shfl(alpha, 4 * g + v, kWave);  // accumulator row 4g + v
#pragma unroll
        for (int c = 0; c < 4; ++c) o[rt][c][v] *= av;
      }
    }
  };

  // Row sums of the published chunk.
  auto accumulate = [&]() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        psum[rt] += p[rt][e];
        zsum[rt] = fmaf(p[rt][e], h16hi(vsz[e]), zsum[rt]);
      }
  };

  // After the barrier that publishes chunk j: if some wavefront voted (a score above the
  // shared max + 2^8), agree on the new maxima and republish; then fold the chunk's
  // probabilities into the row sums.
  auto resolve = [&](int j) {
    const int buf = j & 1;
    if (uniform(s_flag[buf][0] | s_flag[buf][1] | s_flag[buf][2] | s_flag[buf][3])) {
      agree_max();
      publish(j);
      barrier_lds();
    }
    accumulate();
  };

  // O[:, 64 wave .. +63] += P V over chunk j's 128 tokens.
  auto pv = [&](int j) {
    const int buf = j & 1;
    const uint8_t* cb = s_stage + (j % kStages) * kStageBytes;
    i32x8 pa[RT][2];
    int sca[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int prow = (16 * rt + n) * kPRow + 16 * g;
#pragma unroll
      for (int term = 0; term < 2; ++term) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(&s_p[buf][term][prow]);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(&s_p[buf][term][prow + 64]);
        pa[rt][term] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                             (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
      sca[rt] = s_scale[buf][16 * rt + n][g];
    }
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int col = dcol + 8 * cc;
      const i32x2 r0 = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(cb + v_off0 + col));
      const i32x2 r1 = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2_ptr_t)(cb + v_off1 + col));
      const i32x8 be = i32x8{even_codes(r0[0]), even_codes(r0[1]), even_codes(r1[0]),
                             even_codes(r1[1]), 0, 0, 0, 0};
      const i32x8 bo = i32x8{odd_codes(r0[0]), odd_codes(r0[1]), odd_codes(r1[0]),
                             odd_codes(r1[1]), 0, 0, 0, 0};
#pragma unroll
      for (int term = 0; term < 2; ++term)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          o[rt][2 * cc] = mfma_pv(pa[rt][term], be, o[rt][2 * cc], sca[rt]);
          o[rt][2 * cc + 1] = mfma_pv(pa[rt][term], bo, o[rt][2 * cc + 1], sca[rt]);
        }
    }
  };

  // ---- software pipeline: iteration j multiplies chunk j into O while the QK MFMAs of
  // chunk j + 1 run; one barrier per chunk publishes chunk j + 1 and frees chunk j's stage.
  f32x4 acc[RT][2];
  if (nchunk > 0) {
    OSCAR_WAIT_VM(kDmaPerSub * (kStages - 1));  // own part of chunk 0 landed
    qk(0, acc);
    score(0, acc);  // (its vote is not needed: the max starts at -inf)
    agree_max();
    publish(0);
    barrier_lds();
    accumulate();
  }
  for (int j = 0; j < nchunk; ++j) {
    const bool more = j + 1 < nchunk;
    if (more) {
      OSCAR_WAIT_VM(kDmaPerSub * (kStages - 2));  // own part of chunk j + 1 landed
      qk(j + 1, acc);
    }
    pv(j);
    if (more) {
      score(j + 1, acc);
      publish(j + 1);
    }
    barrier_lds();  // chunk j + 1 published (and landed); everyone is done with chunk j
    issue(j + kStages, j % kStages);
    if (more) resolve(j + 1);
  }
  OSCAR_WAIT_VM(0);

  // ---- epilogue: row totals over lanes and wavefronts, then each wavefront writes its
  // 64 dims. Accumulator o[rt][2cc + par] lane (g, n) element v = row 16 rt + 4g + v,
  // dim 64 wave + 32 cc + 2n + par, in units of c/2 (FP4).
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    psum[rt] += __shfl_xor(psum[rt], 16, kWave);
    psum[rt] += __shfl_xor(psum[rt], 32, kWave);
    zsum[rt] += __shfl_xor(zsum[rt], 16, kWave);
    zsum[rt] += __shfl_xor(zsum[rt], 32, kWave);
    if (g == 0) {
      s_red[1][wave][16 * rt + n] = psum[rt];
      s_red[2][wave][16 * rt + n] = zsum[rt];
    }
  }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * rt + 4 * g + v;
      const RowInfo ri = row_info(a, t, head, row);
      if (!ri.valid) continue;
      const float den = s_red[1][0][row] + s_red[1][1][row] + s_red[1][2][row] + s_red[1][3][row];
      const float zs = s_red[2][0][row] + s_red[2][1][row] + s_red[2][2][row] + s_red[2][3][row];
      const float inv = 1.0f / fmaxf(den, 1.0e-30f);
      float* out = a.partials + ((ri.token * a.hq + ri.qhead) * a.splits + split) * kHeadDim +
                   64 * wave + 2 * n;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        *reinterpret_cast<float2*>(out + 32 * cc) =
            make_float2((2.0f * o[rt][2 * cc][v] + zs) * inv,
                        (2.0f * o[rt][2 * cc + 1][v] + zs) * inv);
    }
  }
  if (wave == 0 && g == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = 16 * rt + n;
      const RowInfo ri = row_info(a, t, head, row);
      if (!ri.valid) continue;
      const float den = s_red[1][0][row] + s_red[1][1][row] + s_red[1][2][row] + s_red[1][3][row];
      a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] =
          den > 0.f ? (m[rt] + log2f(den)) * kLn2 : -INFINITY;
    }
  }
}

}  // namespace

hipError_t launch_history(const AttnArgs& a, dim3 grid, int rows, hipStream_t stream) {
  if (rows <= 16)
    hipLaunchKernelGGL(history_kernel<1>, grid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(history_kernel<2>, grid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace oscar
