// Initial prefill: causal attention of each request over its own tokens (no history), the
// replacement of the reference's fused-infer call (oscar_ascend/backend.py:175-193).
//
// Flash layout for MI355X: a workgroup of 12 wavefronts (three per SIMD) serves 192 consecutive
// (query, head) rows of one request and one KV head (wavefront w: rows 16 w .. 16 w + 15, all
// 256 output dims) and streams the request's keys and values in 32-token blocks that its
// wavefronts share: each block is copied into LDS once by direct-to-LDS loads (four stages,
// three blocks in flight while one is computed, one barrier per block), so the K/V bytes a
// workgroup reads from L2 serve all of its 192 rows. The copies, 32 KiB per block and
// workgroup, are what bounds the kernel: 128-row workgroups took 16 % longer, and one block in
// flight 11 % longer. The arithmetic of every row is the BF16 branch's (raw.h: the same MFMA
// operands and k order, the same lazy max, p, sums and normalization), so the output, the LSE
// and the bits are those of the decode path (attention_partials raw + merges) for a request
// without history. Blocks past a workgroup's last query are not read (they are masked for
// every row). Workgroups run the longest spans (the last rows of requests) first. Requests
// with cached tokens (seq_len != query tokens) are not initial prefills: their rows are
// written as NaN (output and LSE), never silently wrong.
#include "dma.h"
#include "raw.h"

namespace oscar {
namespace {

constexpr int kWavesP = 12;                          // wavefronts per workgroup (3 per SIMD)
constexpr int kCopyWavesP = 8;                       // the ones that copy blocks and pair V
constexpr int kThreadsP = kWavesP * kWave;
constexpr int kPrefillRT = 1;                        // row tiles per wavefront
constexpr int kSpanRows = kWavesP * 16 * kPrefillRT;  // 192 rows per workgroup (at most)
constexpr int kRowBytes = kHeadDim * 2;              // 512 bytes per K or V row
constexpr int kBlockBytes = kBlock * kRowBytes;      // 16 KiB per K or V block
constexpr int kStageBytesP = 2 * kBlockBytes;        // K then V
constexpr int kDmaPerWave = kStageBytesP / 1024 / kCopyWavesP;  // 1 KiB per DMA, 4 per wavefront
constexpr int kStagesP = 4;                          // K/V blocks in LDS
constexpr int kAheadP = 3;                           // blocks in flight beyond the current one
// Paired V (the P*V B operands, built once per block by the whole workgroup): row r(d) of dim
// d holds 16 dwords, dword 4 g + f = (V[tau(g, 2 f + 1)][d] << 16) | V[tau(g, 2 f)][d]; rows
// are 64 bytes apart and ordered r(16 n + j) = 16 j + n, and the 16-byte column g of row r
// sits at column g ^ (r / 2 mod 4), so that the 8 lanes n = 0..7 of a read (rows 16 j + n, one
// column) hit 8 different bank quads. Four K/V stages and two pair buffers fill the 160 KiB.
constexpr int kPairRowBytes = 64;
constexpr int kPairBytes = kHeadDim * kPairRowBytes;  // 16 KiB per block
__device__ __forceinline__ uint32_t pair_pos(int r, int dword) {
  return r * kPairRowBytes + 16 * ((dword >> 2) ^ ((r >> 1) & 3)) + 4 * (dword & 3);
}

// LDS position of 16-byte chunk c of block row t: the chunk's low three bits are XOR-swizzled by
// the row's low three bits and the chunk's own bits 3-4, so that each group of 8 lanes the LDS
// serves together (a ds_read_b128 moves 128 bytes a clock) touches 8 different bank quads, both
// in a K read (8 rows, one chunk) and in a V read (one row, chunks 2 n + h). An involution.
__device__ __forceinline__ uint32_t chunk_pos(int t, int c) { return c ^ (t & 7) ^ ((c >> 3) & 3); }

struct PrefillArgs {
  const uint16_t* query;
  int64_t qs0, qs1;
  const uint16_t* key;
  int64_t ks0, ks1;
  const uint16_t* value;
  int64_t vs0, vs1;
  const int32_t* qstarts;
  const int32_t* seq_lens;
  const int32_t* counts;
  int64_t n;
  int32_t g, hq, kv_heads;
  // Rows per workgroup: kSpanRows, or 96 or 48 when a launch would have fewer workgroups
  // than CUs (one long request); the wavefronts past them only copy and pair blocks.
  int32_t span_rows;
  FastDiv g_div;
  float scale_log2;
  uint16_t* out;
  float* lse;
  // Continuation chunks (the chunk form): each request's sink and recent rows come from its
  // window page (block-table column 0's page), and the rows are written as fp32 partials.
  Layout L;
  const uint16_t* window;
  int64_t window_elems;
  const int32_t* table;
  int64_t table_stride, table_columns;
  float* partials;  // [n][hq][256]
  float* plse;      // [n][hq]
};

// The BF16 branch's raw index sequence of one request and KV head in the chunk form
// (raw.h raw_row): indices [0, sink_len) are the sink positions, [sink_len, high) the recent
// positions recent_begin.., then the current tokens prefix... `win`: element offset of the
// head's K row at window index 0 in the owner page, or -1 when the page does not lie wholly in
// the window buffer (the window rows are then masked; the decode path masks row by row, and
// the two agree whenever the buffer holds whole pages, as the layout's views do).
struct ChunkRows {
  int prefix, sink_len, recent_begin, high;
  int64_t win;
};

__device__ __forceinline__ ChunkRows chunk_rows(const PrefillArgs& a, int req, int seq, int qlen,
                                                int head) {
  ChunkRows c;
  c.prefix = seq - qlen;
  c.sink_len = min(a.L.sink, c.prefix);
  c.recent_begin = max(c.sink_len, c.prefix - a.L.recent);
  c.high = c.sink_len + c.prefix - c.recent_begin;
  c.win = -1;
  const int first = a.table_columns > 0 ? a.table[static_cast<int64_t>(req) * a.table_stride] : -1;
  if (first >= 0) {
    const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
    const int64_t win = owner * (a.L.page_bytes / 2) + static_cast<int64_t>(head) * kHeadDim;
    // Last row read: V of window index sink + ring - 1.
    const int64_t last = win + (static_cast<int64_t>(a.L.sink + a.L.ring - 1) * 2 + 1) *
                                   a.L.kv_heads * kHeadDim + kHeadDim;
    if (last <= a.window_elems) c.win = win;
  }
  return c;
}

// K (kv 0) or V row of raw index ns (0 <= ns < high + qlen): a window row or a current token;
// a masked window row (no window page) reads the request's first current token instead.
__device__ __forceinline__ const uint16_t* chunk_row(const PrefillArgs& a, const ChunkRows& c,
                                                     int64_t qstart, int head, int ns, int kv) {
  if (ns >= c.high || c.win < 0) {
    const int64_t ci = qstart + max(ns - c.high, 0);
    return kv ? a.value + ci * a.vs0 + head * a.vs1 : a.key + ci * a.ks0 + head * a.ks1;
  }
  const int pos = ns < c.sink_len ? ns : c.recent_begin + ns - c.sink_len;
  const int lap = static_cast<int>(fastdiv(static_cast<uint32_t>(pos), a.L.ring_div));
  const int wi = pos < a.L.sink ? pos : a.L.sink + pos - lap * a.L.ring;
  return a.window + c.win + (static_cast<int64_t>(wi) * 2 + kv) * a.L.kv_heads * kHeadDim;
}

// Copies block b of (K, V) rows into `stage`: wavefront w < 8 issues DMAs 4 w .. 4 w + 3, DMA i
// covering K (i < 16) or V rows 2 (i mod 16), + 1. Lane l writes row t = 2 (i mod 16) + l / 32
// at position l mod 32, fetching the chunk chunk_pos maps there. Every lane issues its copy
// (the stage waits count 4 DMAs per copying wavefront; the others have none): rows at or past the request's token count copy
// its last row instead; they are masked for every query row, so their p is exactly 0 and their
// products add exact zeros, as the decode path's zero rows do. `kb`/`vb`: the request's row 0
// of this head's keys and values; `kstride`/`vstride`: bytes per token.
__device__ __forceinline__ void prefill_copy_block(const uint8_t* kb, const uint8_t* vb,
                                                   uint32_t kstride, uint32_t vstride, int qlen,
                                                   int b, uint8_t* stage) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave >= kCopyWavesP) return;
  const int last = qlen - 1 - kBlock * b;  // rows past it copy the request's last row
  const int64_t block_row = static_cast<int64_t>(kBlock) * b;
  const uint8_t* kbase = kb + block_row * kstride;
  const uint8_t* vbase = vb + block_row * vstride;
#pragma unroll
  for (int k = 0; k < kDmaPerWave; ++k) {
    const int i = kDmaPerWave * wave + k;  // is_v = i >> 4 is wave-uniform (waves 4..7: V)
    const int t = 2 * (i & 15) + (lane >> 5);
    const uint32_t row = static_cast<uint32_t>(min(t, last));
    const uint32_t chunk = 16u * chunk_pos(t, lane & 31);
    const uint32_t lds = lds_addr(stage + (i >> 4) * kBlockBytes + (i & 15) * 1024);
    if (i >> 4)
      dma_x4(vbase, row * vstride + chunk, lds);
    else
      dma_x4(kbase, row * kstride + chunk, lds);
  }
}

// The chunk form of prefill_copy_block: block b of the raw index sequence (rows at or past
// `end` copy raw index end - 1, a current token; they are masked for every query row), each
// lane's row from its own address (window page or current tokens).
__device__ __forceinline__ void chunk_copy_block(const PrefillArgs& a, const ChunkRows& c,
                                                 int64_t qstart, int head, int end, int b,
                                                 uint8_t* stage) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave >= kCopyWavesP) return;
#pragma unroll
  for (int k = 0; k < kDmaPerWave; ++k) {
    const int i = kDmaPerWave * wave + k;  // is_v = i >> 4 is wave-uniform
    const int t = 2 * (i & 15) + (lane >> 5);
    const int ns = min(kBlock * b + t, end - 1);
    const uint8_t* row = reinterpret_cast<const uint8_t*>(chunk_row(a, c, qstart, head, ns, i >> 4));
    const uint32_t lds = lds_addr(stage + (i >> 4) * kBlockBytes + (i & 15) * 1024);
    dma_dwordx4(row + 16u * chunk_pos(t, lane & 31), lds);
  }
}

// kChunk false: initial prefill (bf16 output rows and LSE; requests with cached tokens get
// NaN rows). kChunk true: the BF16 branch of continuation chunks (sink, recent and causal
// current keys; fp32 partial rows and LSE, as attention_partials raw with one split), with
// the same row arithmetic.
template <bool kChunk>
__global__ __launch_bounds__(kThreadsP) void prefill_flash_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_kv[kStagesP][kStageBytesP];
  __shared__ __attribute__((aligned(16))) uint8_t s_pair[2][kPairBytes];
  const int req = blockIdx.x, head = blockIdx.z;
  const int span = static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y);
  if (req >= a.counts[0]) return;
  const int64_t qstart = a.qstarts[req];
  const int64_t qend = min(static_cast<int64_t>(a.qstarts[req + 1]),
                           static_cast<int64_t>(a.counts[1]));
  const int qlen = static_cast<int>(qend - qstart);
  if (qlen <= 0) return;
  const int rows_req = qlen * a.g;
  const int row0 = span * a.span_rows;
  if (row0 >= rows_req) return;
  const int row_end = min(row0 + a.span_rows, rows_req);
  const int seq = a.seq_lens[req];
  // Initial prefill: a request with cached tokens is not one; chunk form: a request with
  // fewer tokens than query tokens is malformed. Their rows are NaN.
  const bool history = kChunk ? seq < qlen : seq != qlen;
  ChunkRows c{};
  if constexpr (kChunk) {
    if (!history) c = chunk_rows(a, req, seq, qlen, head);
  }
  const int high = kChunk ? c.high : 0;  // raw index of the first current token
  const int end = high + qlen;           // raw indices of the request
  // Raw indices below this are window rows without a window page (masked).
  const int masked_below = kChunk && c.win < 0 ? high : 0;
  // Rows past the grid's spans (a request with more query tokens than the caller's
  // max_query_len) are written as NaN by the last span's workgroup, like the rows of a
  // request with cached tokens, so that a wrong bound shows in the output.
  if (span == static_cast<int>(gridDim.y) - 1) {
    const int covered = static_cast<int>(gridDim.y) * a.span_rows;
    for (int row = covered + static_cast<int>(threadIdx.x >> 5); row < rows_req;
         row += kThreadsP / 32) {
      const int qi = static_cast<int>(fastdiv(static_cast<uint32_t>(row), a.g_div));
      const int qhead = head * a.g + (row - qi * a.g);
      const int64_t orow = (qstart + qi) * a.hq + qhead;
      if constexpr (kChunk) {
        float* dst = a.partials + orow * kHeadDim + 8 * (threadIdx.x & 31);
        *reinterpret_cast<float4*>(dst) = make_float4(NAN, NAN, NAN, NAN);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(NAN, NAN, NAN, NAN);
        if ((threadIdx.x & 31) == 0) a.plse[orow] = NAN;
      } else {
        *reinterpret_cast<u32x4*>(a.out + orow * kHeadDim + 8 * (threadIdx.x & 31)) =
            u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
        if (a.lse && (threadIdx.x & 31) == 0) a.lse[orow] = NAN;
      }
    }
  }
  const int q_last = static_cast<int>(fastdiv(static_cast<uint32_t>(row_end - 1), a.g_div));
  const int nblk = history ? 0 : (q_last + high) / kBlock + 1;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const bool has_rows = 16 * kPrefillRT * wave < a.span_rows;  // wavefront-uniform

  const uint8_t* kb = reinterpret_cast<const uint8_t*>(a.key + qstart * a.ks0 + head * a.ks1);
  const uint8_t* vb = reinterpret_cast<const uint8_t*>(a.value + qstart * a.vs0 + head * a.vs1);
  const uint32_t kstride = static_cast<uint32_t>(a.ks0 * 2), vstride = static_cast<uint32_t>(a.vs0 * 2);
  auto copy_block = [&](int b, uint8_t* stage) {
    if constexpr (kChunk)
      chunk_copy_block(a, c, qstart, head, end, b, stage);
    else
      prefill_copy_block(kb, vb, kstride, vstride, qlen, b, stage);
  };
  for (int b = 0; b < kAheadP && b < nblk; ++b)  // block b + kAheadP: iteration b
    copy_block(b, s_kv[b]);

  // Query rows of this wavefront's tile: row16 = row0 + 16 w + n.
  u32x4 qb[kPrefillRT][8];
  int qi_row[kPrefillRT];
#pragma unroll
  for (int rt = 0; rt < kPrefillRT; ++rt) {
    const int row = row0 + 16 * (kPrefillRT * wave + rt) + n;
    const int qi = static_cast<int>(fastdiv(static_cast<uint32_t>(row), a.g_div));
    qi_row[rt] = row < row_end ? qi : -1;
#pragma unroll
    for (int m = 0; m < 8; ++m) qb[rt][m] = u32x4{0u, 0u, 0u, 0u};
    if (row < row_end) {
      const int qhead = head * a.g + (row - qi * a.g);
      const uint16_t* qp = a.query + (qstart + qi) * a.qs0 + qhead * a.qs1 + 64 * g;
#pragma unroll
      for (int m = 0; m < 8; ++m) qb[rt][m] = *reinterpret_cast<const u32x4*>(qp + 8 * m);
    }
  }
  // The query rows land here (with the first blocks' copies): no wait for them in the loop,
  // where it would also wait for the blocks in flight.
  OSCAR_WAIT_VM0_SEEN();
  State<kPrefillRT, 16> st;
  state_init(st);
  // Blocks whose every key (raw index) is at or below this wavefront's first query's last
  // key and the request's end, and at or above masked_below, need no mask.
  const int qi_first = static_cast<int>(
      fastdiv(static_cast<uint32_t>(row0 + 16 * kPrefillRT * wave), a.g_div));
  const int full_below = min(qi_first + high, end - 1);  // last key every row of the wave sees
  int key_lim[kPrefillRT];  // last raw index row rt sees (-1: a row past the span's end)
#pragma unroll
  for (int rt = 0; rt < kPrefillRT; ++rt) key_lim[rt] = qi_row[rt] < 0 ? -1 : qi_row[rt] + high;
  // Per-lane LDS offsets of the K operands within a stage: rows 16 tt + n, chunk 8 g + m.
  uint32_t koff[2][8];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int t = 16 * tt + n;
      koff[tt][m] = t * kRowBytes + 16 * chunk_pos(t, 8 * g + m);
    }
  // Pairing (wavefronts w < 8): lane l of wavefront w takes token pair q = l % 16 (tokens t0, t0 + 1 with
  // t0 = tau(q / 4, 2 (q % 4))) and 8-dim chunk c = 8 (l / 16) + w of the block's V rows; dim
  // 8 c + j goes to row r = 16 ((8 c + j) % 16) + (8 c + j) / 16 = 128 (c % 2) + 16 j + c / 2.
  // (The two 16-lane halves of a write then fall on disjoint banks: their rows are 4 apart.)
  const int pq = lane & 15, pc = 8 * (lane >> 4) + wave;
  const int pt0 = tau(pq >> 2, 2 * (pq & 3));
  const uint32_t pair_src0 = kBlockBytes + pt0 * kRowBytes + 16 * chunk_pos(pt0, pc);
  const uint32_t pair_src1 = kBlockBytes + (pt0 + 1) * kRowBytes + 16 * chunk_pos(pt0 + 1, pc);
  // (Rows 16 j apart share the column swizzle, so the rows 16 j + r of one lane are a fixed
  // stride apart.)
  const uint32_t pair_dst = pair_pos(128 * (pc & 1) + (pc >> 1), pq);
  // P*V operand of lane (n, g), dim tile j: row 16 j + n, dwords 4 g .. 4 g + 3.
  const uint32_t pv_off = pair_pos(n, 4 * g);
  auto pair_block = [&](const uint8_t* stage, uint8_t* pairs) {
    const u32x4 x0 = *reinterpret_cast<const u32x4*>(stage + pair_src0);
    const u32x4 x1 = *reinterpret_cast<const u32x4*>(stage + pair_src1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      *reinterpret_cast<uint32_t*>(pairs + pair_dst + 16 * j * kPairRowBytes) =
          __builtin_amdgcn_perm(x1[j >> 1], x0[j >> 1], sel);
    }
  };
  auto pv_block = [&](const uint8_t* pairs, const u32x4 (&ap)[kPrefillRT]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const u32x4 bv = *reinterpret_cast<const u32x4*>(pairs + pv_off + 16 * j * kPairRowBytes);
#pragma unroll
      for (int rt = 0; rt < kPrefillRT; ++rt) st.o[rt][j] = mfma16x16x32(ap[rt], bv, st.o[rt][j]);
    }
  };
  // P of the block before the first: zero, with zeroed pairs, so that every iteration runs
  // the previous block's P*V (adding exact zeros the first time) without a branch, and the
  // scores and P*V MFMAs of an iteration interleave.
  u32x4 ap_prev[kPrefillRT];
#pragma unroll
  for (int rt = 0; rt < kPrefillRT; ++rt) ap_prev[rt] = u32x4{0u, 0u, 0u, 0u};
  for (int i = threadIdx.x; i < 2 * kPairBytes / 16; i += kThreadsP)
    reinterpret_cast<u32x4*>(&s_pair[0][0])[i] = u32x4{0u, 0u, 0u, 0u};

  for (int b = 0; b < nblk; ++b) {
    const uint8_t* stage = s_kv[b % kStagesP];
    // Wait for block b (the blocks issued after it stay in flight) and the barrier that makes
    // every wavefront's copies of it, and the pairs of block b - 1, visible; it is the only
    // barrier of a block. After it, block b + 3 goes to the stage of block b - 1: every
    // wavefront finished with that block (scores, pairing) before reaching the barrier.
    static_assert(kAheadP + 1 <= kStagesP && kAheadP == 3, "the stage refilled is one block old");
    const int after = min(nblk - 1 - b, kAheadP - 1);
    if (after >= 2)
      OSCAR_WAIT_VM(2 * kDmaPerWave);
    else if (after == 1)
      OSCAR_WAIT_VM(kDmaPerWave);
    else
      OSCAR_WAIT_VM(0);
    barrier_lds();  // block b landed, pairs of block b - 1 written
    if (b + kAheadP < nblk) copy_block(b + kAheadP, s_kv[(b + kAheadP) % kStagesP]);
    // P*V of block b - 1 (the accumulators take it before block b's lazy max may rescale
    // them, the order of the one-block-at-a-time stream) interleaved with block b's scores
    // S^T = K Q^T (A = K rows 16 tt + n, chunk 8 g + m): two P*V tiles per score k-step.
    const uint8_t* pairs = s_pair[(b + 1) & 1];  // block b - 1's
    if (has_rows) {
    f32x4 sc[kPrefillRT][2];
#pragma unroll
    for (int rt = 0; rt < kPrefillRT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const u32x4 kd = *reinterpret_cast<const u32x4*>(stage + koff[tt][m]);
#pragma unroll
        for (int rt = 0; rt < kPrefillRT; ++rt) sc[rt][tt] = mfma16x16x32(kd, qb[rt][m], sc[rt][tt]);
        const int j = 2 * m + tt;
        const u32x4 bv = *reinterpret_cast<const u32x4*>(pairs + pv_off + 16 * j * kPairRowBytes);
#pragma unroll
        for (int rt = 0; rt < kPrefillRT; ++rt)
          st.o[rt][j] = mfma16x16x32(ap_prev[rt], bv, st.o[rt][j]);
      }
    }
    float s2[kPrefillRT][8];
    if (kBlock * b >= masked_below && kBlock * b + kBlock - 1 <= full_below) {
      block_scores_full(sc, a.scale_log2, s2);
    } else {
      bool ok[kPrefillRT][8];
#pragma unroll
      for (int rt = 0; rt < kPrefillRT; ++rt)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = kBlock * b + tau(g, e);
          ok[rt][e] = key < end && key <= key_lim[rt] && key >= masked_below;
        }
      block_scores(sc, ok, a.scale_log2, s2);
    }
    update_max(st, s2, g);
    block_p(st, s2, ap_prev);
    }
    // Pairs of block b (into the buffer block b - 2 used, read before the barrier above).
    if (wave < kCopyWavesP) pair_block(stage, s_pair[b & 1]);
  }
  if (nblk > 0) {
    barrier_lds();  // the last block's pairs
    if (has_rows) pv_block(s_pair[(nblk - 1) & 1], ap_prev);
  }
  if (!has_rows) return;

  // Normalize and store: lane (n, g) holds rows 4 g + v of each tile, dims 16 n + j.
#pragma unroll
  for (int rt = 0; rt < kPrefillRT; ++rt) {
    const float den_n = row_sum(st.psum[rt]);
    const int tile_row = row0 + 16 * (kPrefillRT * wave + rt);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = tile_row + 4 * g + v;
      const float den = fmaxf(__shfl(den_n, 4 * g + v, kWave), 1.0e-30f);
      if (row >= row_end) continue;
      const int qi = static_cast<int>(fastdiv(static_cast<uint32_t>(row), a.g_div));
      const int qhead = head * a.g + (row - qi * a.g);
      if constexpr (kChunk) {
        float* dst = a.partials + ((qstart + qi) * a.hq + qhead) * kHeadDim + 16 * n;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 x = history ? make_float4(NAN, NAN, NAN, NAN)
                                   : make_float4(st.o[rt][4 * k][v] / den,
                                                 st.o[rt][4 * k + 1][v] / den,
                                                 st.o[rt][4 * k + 2][v] / den,
                                                 st.o[rt][4 * k + 3][v] / den);
          *reinterpret_cast<float4*>(dst + 4 * k) = x;
        }
        continue;
      }
      uint32_t w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        w[k] = history ? 0x7fc07fc0u
                       : pack_bf16x2(st.o[rt][2 * k][v] / den, st.o[rt][2 * k + 1][v] / den);
      uint16_t* dst = a.out + ((qstart + qi) * a.hq + qhead) * kHeadDim + 16 * n;
      *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(dst + 8) = u32x4{w[4], w[5], w[6], w[7]};
    }
    float* lse_out = kChunk ? a.plse : a.lse;
    if (g == 0 && lse_out) {
      const int row = tile_row + n;
      if (row < row_end) {
        const int qi = static_cast<int>(fastdiv(static_cast<uint32_t>(row), a.g_div));
        const int qhead = head * a.g + (row - qi * a.g);
        lse_out[(qstart + qi) * a.hq + qhead] = history ? NAN : row_lse(st.m[rt], den_n);
      }
    }
  }
}

// Rows of tokens at or past counts[1]: zero output, LSE -inf (the reference zeroes
// output[num_actual_tokens:]).
__global__ __launch_bounds__(kThreads) void prefill_clear_kernel(const PrefillArgs a) {
  // The rows of tokens [counts[1], n) only (all of them for a negative count, none past n).
  const int64_t active = min(max(static_cast<int64_t>(a.counts[1]), int64_t{0}), a.n);
  const int64_t total = a.n * a.hq;
  for (int64_t row = active * a.hq + static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
       row < total; row += static_cast<int64_t>(gridDim.x) * 4) {
    const int lane = threadIdx.x & 63;
    *reinterpret_cast<uint2*>(a.out + row * kHeadDim + 4 * lane) = make_uint2(0u, 0u);
    if (a.lse && lane == 0) a.lse[row] = -INFINITY;
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Rows per workgroup of a launch over `rows` rows per (request, KV head): kSpanRows, unless
// the launch would then have fewer workgroups than the chip's 256 CUs (one long request);
// then 96 or 48 rows: more workgroups over the same blocks, each copying every block of its
// rows. A row's arithmetic does not depend on the rows beside it, so neither do its bits.
int span_rows_for(int64_t rows, int64_t reqs, int64_t heads) {
  constexpr int64_t kChipCUs = 256;
  for (const int r : {kSpanRows, kSpanRows / 2})
    if (reqs * heads * ((rows + r - 1) / r) >= kChipCUs) return r;
  return kSpanRows / 4;
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_prefill_attention(
    const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1,
    const void* value, int64_t v_s0, int64_t v_s1, const int32_t* qstarts,
    const int32_t* seq_lens, const int32_t* counts, int64_t n, int64_t hq, int64_t max_reqs,
    int32_t max_query_len, float scale, const oscar_layout* layout, void* output,
    float* merged_lse, void* stream) {
  using namespace oscar;
  Layout L;
  const int st = make_layout(layout, &L);
  if (st != OSCAR_OK) return st;
  const int64_t h = L.kv_heads;
  if (n < 0 || hq <= 0 || hq % h || max_reqs < 1 || max_reqs > 65535 || max_query_len < 0 ||
      n * hq > 0x7fffffffll)
    return OSCAR_E_SHAPE;
  if (!(scale > 0.f) || !(scale < INFINITY)) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!query || !key || !value || !qstarts || !seq_lens || !counts || !output) return OSCAR_E_NULL;
  if (q_s0 % 8 || q_s1 % 8 || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 || !aligned16(query) ||
      !aligned16(key) || !aligned16(value) || !aligned16(output))
    return OSCAR_E_ALIGN;
  const int64_t g = hq / h;
  PrefillArgs a{};
  a.query = static_cast<const uint16_t*>(query);
  a.qs0 = q_s0;
  a.qs1 = q_s1;
  a.key = static_cast<const uint16_t*>(key);
  a.ks0 = k_s0;
  a.ks1 = k_s1;
  a.value = static_cast<const uint16_t*>(value);
  a.vs0 = v_s0;
  a.vs1 = v_s1;
  a.qstarts = qstarts;
  a.seq_lens = seq_lens;
  a.counts = counts;
  a.n = n;
  a.g = static_cast<int32_t>(g);
  a.hq = static_cast<int32_t>(hq);
  a.kv_heads = static_cast<int32_t>(h);
  a.g_div = make_fastdiv(static_cast<uint32_t>(g));
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(output);
  a.lse = merged_lse;
  // Spans per request: its rows (query tokens x g) in span_rows-row groups; a request has at
  // most max_query_len (when given) or n query tokens. Rows past the spans of a request that
  // breaks the given bound are written as NaN.
  const int64_t qmax = max_query_len > 0 && max_query_len < n ? max_query_len : n;
  a.span_rows = span_rows_for(qmax * g, max_reqs, h);
  const int64_t spans = (qmax * g + a.span_rows - 1) / a.span_rows;
  if (spans > 65535) return OSCAR_E_SHAPE;  // grid y
  hipStream_t s = as_stream(stream);
  // Requests vary fastest: the workgroups of the longest spans of every request dispatch
  // first (a longest-first order of the whole batch), and consecutive workgroups, which the
  // dispatcher spreads over the XCDs, keep each XCD on few requests (their K/V stay in its L2).
  hipLaunchKernelGGL(prefill_flash_kernel<false>,
                     dim3(static_cast<unsigned>(max_reqs), static_cast<unsigned>(spans),
                          static_cast<unsigned>(h)),
                     dim3(kThreadsP), 0, s, a);
  const int64_t clear = (n * hq + 3) / 4;
  hipLaunchKernelGGL(prefill_clear_kernel,
                     dim3(static_cast<unsigned>(clear < 1024 ? clear : 1024)), dim3(kThreads), 0,
                     s, a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_chunk_raw_attention(
    const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1,
    const void* value, int64_t v_s0, int64_t v_s1, const void* window, int64_t window_elems,
    const int32_t* qstarts, const int32_t* seq_lens, const int32_t* block_tables,
    int64_t table_stride, int64_t table_columns, const int32_t* counts, int64_t n, int64_t hq,
    int64_t max_reqs, int32_t max_query_len, float scale, const oscar_layout* layout,
    float* raw_partials, float* raw_lse, void* stream) {
  using namespace oscar;
  PrefillArgs a{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  const int64_t h = a.L.kv_heads;
  if (n < 0 || hq <= 0 || hq % h || max_reqs < 1 || max_reqs > 65535 || max_query_len < 0 ||
      table_columns < 0 || window_elems < 0 || n * hq > 0x7fffffffll)
    return OSCAR_E_SHAPE;
  if (!(scale > 0.f) || !(scale < INFINITY)) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!query || !key || !value || !window || !qstarts || !seq_lens || !block_tables || !counts ||
      !raw_partials || !raw_lse)
    return OSCAR_E_NULL;
  if (q_s0 % 8 || q_s1 % 8 || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 || !aligned16(query) ||
      !aligned16(key) || !aligned16(value) || !aligned16(window) || !aligned16(raw_partials) ||
      a.L.page_bytes % 16)
    return OSCAR_E_ALIGN;
  const int64_t g = hq / h;
  a.query = static_cast<const uint16_t*>(query);
  a.qs0 = q_s0;
  a.qs1 = q_s1;
  a.key = static_cast<const uint16_t*>(key);
  a.ks0 = k_s0;
  a.ks1 = k_s1;
  a.value = static_cast<const uint16_t*>(value);
  a.vs0 = v_s0;
  a.vs1 = v_s1;
  a.qstarts = qstarts;
  a.seq_lens = seq_lens;
  a.counts = counts;
  a.n = n;
  a.g = static_cast<int32_t>(g);
  a.hq = static_cast<int32_t>(hq);
  a.kv_heads = static_cast<int32_t>(h);
  a.g_div = make_fastdiv(static_cast<uint32_t>(g));
  a.scale_log2 = scale * kLog2e;
  a.window = static_cast<const uint16_t*>(window);
  a.window_elems = window_elems;
  a.table = block_tables;
  a.table_stride = table_stride;
  a.table_columns = table_columns;
  a.partials = raw_partials;
  a.plse = raw_lse;
  const int64_t qmax = max_query_len > 0 && max_query_len < n ? max_query_len : n;
  a.span_rows = span_rows_for(qmax * g, max_reqs, h);
  const int64_t spans = (qmax * g + a.span_rows - 1) / a.span_rows;
  if (spans > 65535) return OSCAR_E_SHAPE;  // grid y
  hipLaunchKernelGGL(prefill_flash_kernel<true>,
                     dim3(static_cast<unsigned>(max_reqs), static_cast<unsigned>(spans),
                          static_cast<unsigned>(h)),
                     dim3(kThreadsP), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}
