// Fused launches of one FULL-attention layer step. The layer step of the reference
// (oscar_ascend/backend.py:171-226) is nine launches; on MI355X most of them are a few
// microseconds of latency each, so this file folds them into two, around the history kernel:
//
//   pre-attention  = BF16 branch partials (kernels.py:439-482, raw=True, one split)
//                  + q rotation (backend.py:195)
//                  + K/V rotation and INT2 store (backend.py:171-173, kernels.py:175-202);
//   post-attention = split merge (kernels.py:506-511) + inverse V rotation (backend.py:210)
//                  + path merge with the merged LSE (kernels.py:530-541)
//                  + window store (kernels.py:598-620).
//
// Each workgroup of a fused launch plays one role, chosen from blockIdx.x; all roles of a
// launch are independent of each other. The roles run the same device code as the single
// entry points (raw.h, rotate.h, quant.h, merge.h, window.h), so both paths produce the same
// bits. Ordering facts the fusion relies on:
//   * the history branch never reads a current token's slot (it stops at recent_begin <=
//     prefix), so the INT2 store of the step may run beside it;
//   * the window store follows both branches (it is in the post-attention launch), as
//     backend.py:225-226 requires.
#include "finish.h"
#include "post.h"
#include "quant.h"
#include "layer.h"
#include "raw.h"

namespace oscar {
namespace {

struct PreArgs {
  AttnArgs attn;          // BF16 branch: unrotated query, key, value, window, metadata
  const uint16_t* rk_t;   // R_k^T, contiguous: rk_t[c][k] = R_k[k][c]
  const uint16_t* rv_t;   // R_v^T, contiguous
  uint16_t* qrot;         // [n, hq, 256]
  int64_t q_rows;         // n * hq
  int64_t kv_rows;        // n * H
  uint8_t* history;
  int64_t history_bytes;
  const int64_t* slots;
  int32_t mode;
  float k_ratio, v_ratio, k_factor, v_factor;
  FastDiv h_div, hq_div;    // division by H and by hq
  int32_t raw_wgs, kv_wgs;  // role boundaries in blockIdx.x
};

// Rotation of rows [16 tile, +16) by R (given as R^T rows) into a [16][256] bf16 LDS tile
// (kv) or into `out` (q). Wavefront w computes columns 64w .. 64w + 63.
__device__ __forceinline__ void rotate_rows16(const uint16_t* x, int64_t xs0, int64_t xs1,
                                              FastDiv h_div, int64_t h, int64_t rows,
                                              int64_t tile, const uint16_t* rt, uint16_t* lds_tile,
                                              uint16_t* out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = tile * 16 + n;
  const uint16_t* xp = nullptr;
  if (row < rows) {
    const uint32_t token = fastdiv(static_cast<uint32_t>(row), h_div);
    xp = x + static_cast<int64_t>(token) * xs0 + (row - static_cast<int64_t>(token) * h) * xs1;
  }
  // Every operand (the A rows and the four column tiles of R) is requested before the first
  // MFMA: one round of memory latency.
  RotateOperands op;
  u32x4 rb[4][8];
  rotate_load_a<true>(op, xp, 1, g);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    rotate_load_b<true>(op, rt + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[ct][m] = op.b[m];
  }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * wave + 16 * ct + n;
    const f32x4 acc = rotate_mfma(op.a, rb[ct]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      const uint16_t bits = static_cast<uint16_t>(float_to_bf16(acc[v]));
      if (lds_tile) {
        lds_tile[r * kHeadDim + col] = bits;
      } else if (tile * 16 + r < rows) {
        out[(tile * 16 + r) * kHeadDim + col] = bits;
      }
    }
  }
}

template <int RT>
__global__ __launch_bounds__(kThreads) void pre_attention_kernel(const PreArgs p) {
  constexpr int kRawLds = finish_lds_bytes<RT>();
  constexpr int kTileLds = 16 * kHeadDim * 2;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRawLds > kTileLds ? kRawLds : kTileLds];
  const int bid = blockIdx.x;
  const AttnArgs& a = p.attn;
  if (bid < p.raw_wgs) {
    // BF16 branch: workgroup (task, kv head), one split.
    const int h = a.L.kv_heads;
    const int task = bid / h, head = bid - task * h;
    raw_block<RT>(a, task, head, 0, smem);
    return;
  }
  const FastDiv h_div = p.h_div;
  if (bid < p.raw_wgs + p.kv_wgs) {
    // K or V rows: four workgroups share a 16-row rotation tile (each computes it) and each
    // clips/quantizes/packs four of its rows, one per wavefront, into their slots. The
    // row's token count and slot are requested before the rotation.
    const int r = bid - p.raw_wgs;
    const int is_v = r & 1;
    const int64_t quad = r >> 1, tile = quad >> 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rr = 4 * static_cast<int>(quad & 3) + wave;
    const int64_t row = tile * 16 + rr;
    const bool in = row < p.kv_rows;
    const uint32_t token = fastdiv(static_cast<uint32_t>(in ? row : 0), h_div);
    const int head = static_cast<int>((in ? row : 0) - static_cast<int64_t>(token) * a.L.kv_heads);
    const bool live = in && static_cast<int64_t>(token) < a.counts[1];
    const int64_t slot = live ? p.slots[token] : -1;  // in flight beside the rotation loads
    uint16_t* tile_lds = reinterpret_cast<uint16_t*>(smem);
    rotate_rows16(is_v ? a.value : a.key, is_v ? a.vs0 : a.ks0, is_v ? a.vs1 : a.ks1, h_div,
                  a.L.kv_heads, p.kv_rows, tile, is_v ? p.rv_t : p.rk_t, tile_lds, nullptr);
    __syncthreads();
    // Same skips as store_int2 (kernels.py:168-169 and the buffer bound).
    if (!live || slot < 0) return;
    const int64_t page = slot / a.L.bp;
    const int64_t within = slot - page * a.L.bp;
    const int64_t base = page * a.L.page_bytes + (within * a.L.kv_heads + head) * a.L.slot_bytes;
    if (base + 2 * a.L.vector_bytes > p.history_bytes) return;
    const uint2 raw = *reinterpret_cast<const uint2*>(tile_lds + rr * kHeadDim + lane * 4);
    const float x[4] = {bf16_to_float(raw.x & 0xffffu), bf16_to_float(raw.x >> 16),
                        bf16_to_float(raw.y & 0xffffu), bf16_to_float(raw.y >> 16)};
    quantize_store(x, p.mode, is_v ? p.v_ratio : p.k_ratio, is_v ? p.v_factor : p.k_factor,
                   p.history + base + is_v * a.L.vector_bytes);
    return;
  }
  // q tile: rotated rows straight to qrot.
  const int64_t tile = bid - p.raw_wgs - p.kv_wgs;
  rotate_rows16(a.query, a.qs0, a.qs1, p.hq_div, a.hq, p.q_rows, tile, p.rk_t, nullptr, p.qrot);
}

// Workgroups [0, merge_wgs): R (token, query head) rows each (R = 4: one wavefront per row for
// the split merge; R = 1 above 16 splits: the four wavefronts merge the row together). The
// remaining workgroups store the window of one request each; both branches have read the
// window before this launch, and the merges do not touch it.
template <int R, int kMode>
__global__ __launch_bounds__(kThreads) void post_attention_kernel(const PostArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_h[R][kHeadDim];  // merged history rows
  __shared__ float s_l[R];
  __shared__ GroupMergeLds group_lds;
  if (static_cast<int>(blockIdx.x) < p.merge_wgs) {
    post_rows<R, kMode>(p, static_cast<int64_t>(blockIdx.x) * R, p.rows, s_h, s_l, &group_lds);
    return;
  }
  const int req = static_cast<int>(blockIdx.x) - p.merge_wgs;
  for (int head = 0; head < p.win.L.kv_heads; ++head) store_window_request(p.win, req, head);
}

}  // namespace
}  // namespace oscar

namespace {
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

extern "C" int oscar_pre_attention(
    const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1,
    const void* value, int64_t v_s0, int64_t v_s1, const void* window, int64_t window_elems,
    const int32_t* qstarts, const int32_t* seq_lens, const int32_t* block_tables,
    int64_t table_stride, int64_t table_columns, const int32_t* counts, const int32_t* tasks,
    const int32_t* task_count, int64_t n, int64_t hq, int64_t programs, int32_t block_n,
    int32_t query_tile, int32_t max_query_len, float scale, const void* rk_t, const void* rv_t,
    void* history, int64_t history_bytes, const int64_t* slots, const oscar_clip* clip,
    const oscar_layout* layout, float* raw_partials, float* raw_lse, void* qrot, void* stream) {
  using namespace oscar;
  PreArgs p{};
  AttnArgs& a = p.attn;
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  const int64_t h = a.L.kv_heads;
  if (n < 0 || hq <= 0 || hq % h || programs < 1 || programs > (1ll << 20) || block_n < 1 ||
      query_tile < 1 || table_columns < 0 || history_bytes < 0 || n * hq > 0x7fffffffll)
    return OSCAR_E_SHAPE;
  if (!clip) return OSCAR_E_NULL;
  if (clip->mode < OSCAR_CLIP_PERCENTILE || clip->mode > OSCAR_CLIP_SEARCH) return OSCAR_E_SHAPE;
  const int64_t g = hq / h;
  const int64_t qrows = (max_query_len > 0 && max_query_len < query_tile ? max_query_len
                                                                         : query_tile) * g;
  if (qrows > 32) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!query || !key || !value || !window || !qstarts || !seq_lens || !block_tables || !counts ||
      !tasks || !task_count || !rk_t || !rv_t || !history || !slots || !raw_partials ||
      !raw_lse || !qrot)
    return OSCAR_E_NULL;
  if (q_s0 % 8 || q_s1 % 8 || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 || !aligned16(query) ||
      !aligned16(key) || !aligned16(value) || !aligned16(window) || !aligned16(rk_t) ||
      !aligned16(rv_t) || !aligned16(raw_partials) || !aligned16(qrot) ||
      reinterpret_cast<uintptr_t>(history) % 4)
    return OSCAR_E_ALIGN;
  a.query = static_cast<const uint16_t*>(query);
  a.qs0 = q_s0;
  a.qs1 = q_s1;
  a.key = static_cast<const uint16_t*>(key);
  a.ks0 = k_s0;
  a.ks1 = k_s1;
  a.value = static_cast<const uint16_t*>(value);
  a.vs0 = v_s0;
  a.vs1 = v_s1;
  a.window = static_cast<const uint16_t*>(window);
  a.window_elems = window_elems;
  a.qstarts = qstarts;
  a.seq_lens = seq_lens;
  a.table = block_tables;
  a.table_stride = table_stride;
  a.table_columns = table_columns;
  a.counts = counts;
  a.tasks = tasks;
  a.task_count = task_count;
  a.partials = raw_partials;
  a.lse = raw_lse;
  a.n = n;
  a.g = static_cast<int32_t>(g);
  a.g_div = make_fastdiv(static_cast<uint32_t>(g));
  a.hq = static_cast<int32_t>(hq);
  a.qt = query_tile;
  a.splits = 1;
  a.block_n = block_n;
  a.scale_log2 = scale * kLog2e;
  p.rk_t = static_cast<const uint16_t*>(rk_t);
  p.rv_t = static_cast<const uint16_t*>(rv_t);
  p.qrot = static_cast<uint16_t*>(qrot);
  p.q_rows = n * hq;
  p.kv_rows = n * h;
  p.history = static_cast<uint8_t*>(history);
  p.history_bytes = history_bytes;
  p.slots = slots;
  p.mode = clip->mode;
  p.k_ratio = clip->k_ratio;
  p.v_ratio = clip->v_ratio;
  p.k_factor = clip->k_factor;
  p.v_factor = clip->v_factor;
  p.h_div = make_fastdiv(static_cast<uint32_t>(h));
  p.hq_div = make_fastdiv(static_cast<uint32_t>(hq));
  p.raw_wgs = static_cast<int32_t>(programs * h);
  p.kv_wgs = static_cast<int32_t>(2 * 4 * ((p.kv_rows + 15) / 16));
  const int64_t q_wgs = (p.q_rows + 15) / 16;
  const dim3 grid(static_cast<unsigned>(p.raw_wgs + p.kv_wgs + q_wgs));
  hipStream_t s = as_stream(stream);
  if (qrows <= 16)
    hipLaunchKernelGGL(pre_attention_kernel<1>, grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(pre_attention_kernel<2>, grid, dim3(kThreads), 0, s, p);
  return static_cast<int>(hipGetLastError());
}

namespace oscar {
namespace {

// The checks and fields of one post-attention launch (everything but the merge grid).
int make_post_args(const float* history_partials, const float* history_lse, int32_t splits,
                   const float* raw_partials, const float* raw_lse, const int32_t* counts,
                   const void* rv, int64_t n, int64_t hq, void* output, float* merged_lse,
                   const void* key, int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0,
                   int64_t v_s1, void* window, int64_t window_elems, const int32_t* qstarts,
                   const int32_t* seq_lens, const int32_t* block_tables, int64_t table_stride,
                   int64_t max_reqs, const oscar_layout* layout, PostArgs* out) {
  PostArgs& p = *out;
  p = PostArgs{};
  const int st = make_layout(layout, &p.win.L);
  if (st != OSCAR_OK) return st;
  if (n < 0 || hq <= 0 || hq % p.win.L.kv_heads || splits < 1 || max_reqs < 0 ||
      window_elems < 0 || n * hq > 0x7fffffffll)
    return OSCAR_E_SHAPE;
  if (n == 0) return OSCAR_OK;
  if (!history_partials || !history_lse || !raw_partials || !raw_lse || !counts || !rv ||
      !output || !key || !value || !window || !qstarts || !seq_lens || !block_tables)
    return OSCAR_E_NULL;
  if (!aligned16(history_partials) || !aligned16(rv) || reinterpret_cast<uintptr_t>(output) % 2)
    return OSCAR_E_ALIGN;
  p.hp = history_partials;
  p.hl = history_lse;
  p.splits = splits;
  p.rp = raw_partials;
  p.rl = raw_lse;
  p.counts = counts;
  p.rv = static_cast<const uint16_t*>(rv);
  p.rows = n * hq;
  p.hq = static_cast<int32_t>(hq);
  p.out = static_cast<uint16_t*>(output);
  p.merged_lse = merged_lse;
  WindowArgs& w = p.win;
  w.k = static_cast<const uint16_t*>(key);
  w.ks0 = k_s0;
  w.ks1 = k_s1;
  w.ks2 = 1;
  w.v = static_cast<const uint16_t*>(value);
  w.vs0 = v_s0;
  w.vs1 = v_s1;
  w.vs2 = 1;
  w.n = n;
  w.window = static_cast<uint16_t*>(window);
  w.window_elems = window_elems;
  w.qstarts = qstarts;
  w.seq_lens = seq_lens;
  w.table = block_tables;
  w.table_stride = table_stride;
  w.counts = counts;
  p.win_requests = n < max_reqs ? n : max_reqs;
  return OSCAR_OK;
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_post_attention(
    const float* history_partials, const float* history_lse, int32_t splits,
    const float* raw_partials, const float* raw_lse, const int32_t* counts, const void* rv,
    int64_t n, int64_t hq, void* output, float* merged_lse, const void* key, int64_t k_s0,
    int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1, void* window,
    int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t max_reqs,
    const oscar_layout* layout, void* stream) {
  using namespace oscar;
  PostArgs p;
  const int st = make_post_args(history_partials, history_lse, splits, raw_partials, raw_lse,
                                counts, rv, n, hq, output, merged_lse, key, k_s0, k_s1, value,
                                v_s0, v_s1, window, window_elems, qstarts, seq_lens, block_tables,
                                table_stride, max_reqs, layout, &p);
  if (st != OSCAR_OK || n == 0) return st;
  const int mode = merge_mode(p.rows, splits);
  const int64_t merge_wgs = mode == kMergeScanGroup ? p.rows : (p.rows + 3) / 4;
  if (merge_wgs + p.win_requests > 0x7fffffffll) return OSCAR_E_SHAPE;
  p.merge_wgs = static_cast<int32_t>(merge_wgs);
  const dim3 grid(static_cast<unsigned>(merge_wgs + p.win_requests));
  hipStream_t s = as_stream(stream);
  if (mode == kMergeOneRound)
    hipLaunchKernelGGL((post_attention_kernel<4, kMergeOneRound>), grid, dim3(kThreads), 0, s, p);
  else if (mode == kMergeScanWave)
    hipLaunchKernelGGL((post_attention_kernel<4, kMergeScanWave>), grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((post_attention_kernel<1, kMergeScanGroup>), grid, dim3(kThreads), 0, s, p);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_history_post(
    const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* history,
    int64_t history_bytes, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, int64_t n, int64_t hq,
    int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile, int32_t max_query_len,
    float scale, int32_t split_tokens, const oscar_layout* layout, float* partials, float* lse,
    int32_t* counters, int64_t counter_slots, const float* raw_partials, const float* raw_lse,
    const void* rv, void* output, float* merged_lse, const void* key, int64_t k_s0, int64_t k_s1,
    const void* value, int64_t v_s0, int64_t v_s1, void* window, int64_t window_elems,
    int64_t max_reqs, void* stream) {
  using namespace oscar;
  AttnArgs a;
  int64_t qrows = 0;
  int st = make_attn_args(query, q_s0, q_s1, q_s2, nullptr, 0, 0, 1, nullptr, 0, 0, 1, history,
                          history_bytes, nullptr, 0, qstarts, seq_lens, block_tables, table_stride,
                          table_columns, counts, tasks, task_count, n, hq, programs, splits,
                          block_n, query_tile, max_query_len, scale, 0, split_tokens, layout,
                          partials, lse, &a, &qrows);
  if (st != OSCAR_OK) return st;
  // One-round split merge by the completing workgroup, paired-token history kernel.
  if (qrows > 8 || splits > kWaveMergeSplits || splits + 1 > 65535) return OSCAR_E_UNSUPPORTED;
  FinishArgs f{};
  st = make_post_args(partials, lse, splits, raw_partials, raw_lse, counts, rv, n, hq, output,
                      merged_lse, key, k_s0, k_s1, value, v_s0, v_s1, window, window_elems,
                      qstarts, seq_lens, block_tables, table_stride, max_reqs, layout, &f.p);
  if (st != OSCAR_OK || n == 0) return st;
  if (!counters) return OSCAR_E_NULL;
  if (reinterpret_cast<uintptr_t>(counters) % 4) return OSCAR_E_ALIGN;
  if (counter_slots < programs * a.L.kv_heads) return OSCAR_E_SHAPE;
  // The completing workgroup reads the split rows through 32-bit buffer offsets.
  if (n * hq * splits * kHeadDim * 4 >= (1ll << 32)) return OSCAR_E_UNSUPPORTED;
  f.counters = counters;
  f.programs = static_cast<int32_t>(programs);
  return static_cast<int>(launch_history_finish(a, f, as_stream(stream)));
}

extern "C" int oscar_layer_step(
    const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1,
    const void* value, int64_t v_s0, int64_t v_s1, void* history, int64_t history_bytes,
    void* window, int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, const int64_t* slots,
    int64_t n, int64_t hq, int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile,
    int32_t max_query_len, float scale, int32_t split_tokens, const void* rk_t, const void* rv_t,
    const void* rv, const oscar_clip* clip, const oscar_layout* layout, float* partials,
    float* lse, float* raw_partials, float* raw_lse, int32_t* counters, int64_t counter_slots,
    void* output, float* merged_lse, int64_t max_reqs, void* stream) {
  using namespace oscar;
  AttnArgs a;
  int64_t qrows = 0;
  int st = make_attn_args(query, q_s0, q_s1, 1, key, k_s0, k_s1, 1, value, v_s0, v_s1, 1, history,
                          history_bytes, window, window_elems, qstarts, seq_lens, block_tables,
                          table_stride, table_columns, counts, tasks, task_count, n, hq, programs,
                          splits, block_n, query_tile, max_query_len, scale, 0, split_tokens, layout,
                          partials, lse, &a, &qrows);
  if (st != OSCAR_OK) return st;
  // One task per request (every request's tokens in one query tile), <= 8 query rows per task,
  // <= 16 splits (the one-round merges of the finisher).
  if (qrows > 8 || splits > kWaveMergeSplits || max_query_len < 1 || max_query_len > query_tile ||
      query_tile > 4)
    return OSCAR_E_UNSUPPORTED;
  if (!clip) return OSCAR_E_NULL;
  if (clip->mode < OSCAR_CLIP_PERCENTILE || clip->mode > OSCAR_CLIP_SEARCH) return OSCAR_E_SHAPE;
  FinishArgs f{};
  st = make_post_args(partials, lse, splits, raw_partials, raw_lse, counts, rv, n, hq, output,
                      merged_lse, key, k_s0, k_s1, value, v_s0, v_s1, window, window_elems,
                      qstarts, seq_lens, block_tables, table_stride, max_reqs, layout, &f.p);
  if (st != OSCAR_OK || n == 0) return st;
  if (!slots || !rk_t || !rv_t || !counters) return OSCAR_E_NULL;
  if (!aligned16(key) || !aligned16(value) || !aligned16(rk_t) || !aligned16(rv_t) ||
      !aligned16(raw_partials) || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 ||
      reinterpret_cast<uintptr_t>(counters) % 4 || reinterpret_cast<uintptr_t>(history) % 4)
    return OSCAR_E_ALIGN;
  if (counter_slots < programs * a.L.kv_heads) return OSCAR_E_SHAPE;
  // The finisher reads the split rows through 32-bit buffer offsets.
  if (n * hq * splits * kHeadDim * 4 >= (1ll << 32) || n * hq * kRawSplits * kHeadDim * 4 >= (1ll << 32))
    return OSCAR_E_UNSUPPORTED;
  f.counters = counters;
  f.programs = static_cast<int32_t>(programs);
  LayerArgs l{};
  l.rk_t = static_cast<const uint16_t*>(rk_t);
  l.rv_t = static_cast<const uint16_t*>(rv_t);
  l.history = static_cast<uint8_t*>(history);
  l.slots = slots;
  l.mode = clip->mode;
  l.k_ratio = clip->k_ratio;
  l.v_ratio = clip->v_ratio;
  l.k_factor = clip->k_factor;
  l.v_factor = clip->v_factor;
  l.raw_part = raw_partials;
  l.raw_lse = raw_lse;
  return static_cast<int>(launch_layer_step(a, f, l, as_stream(stream)));
}
