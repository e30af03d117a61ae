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
#include "pre.h"
#include "layer.h"

namespace oscar {
namespace {

constexpr int kPostQuarterRows = 2;  // rows per column-quarter post-attention workgroup
constexpr int kPostWideRows = 4;     // rows per all-quarter workgroup (many rows)
constexpr int64_t kPostWideFrom = 512;  // rows from which a workgroup walks all four quarters
constexpr int64_t kPostTileFrom = 4096;  // rows from which a workgroup serves 16 rows

template <int RT>
__global__ __launch_bounds__(kThreads) void pre_attention_kernel(const PreArgs p) {
  // K/V rotation tile of the store role, or the BF16 branch's K stages.
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRawSlots * kRawLdsPerSlot];
  static_assert(16 * kHeadDim * 2 <= kRawSlots * kRawLdsPerSlot, "the store tile fits");
  const int bid = blockIdx.x;
  const AttnArgs& a = p.attn;
  if (bid < p.raw_wgs) {
    // BF16 branch: workgroup (task, kv head), one split.
    const int h = a.L.kv_heads;
    const int task = bid / h, head = bid - task * h;
    raw_block_staged<RT>(a, task, head, 0, smem, kRawSlots);
    return;
  }
  if (bid < p.raw_wgs + p.kv_wgs) {
    kv_store_role(p, bid - p.raw_wgs, smem);
    return;
  }
  // q tile: rotated rows straight to qrot.
  const int64_t tile = bid - p.raw_wgs - p.kv_wgs;
  rotate_rows16(a.query, a.qs0, a.qs1, p.hq_div, a.hq, p.q_rows, tile, p.rk_t, nullptr, p.qrot);
}

// More than 16 splits. Workgroups [0, merge_wgs): R (token, query head) rows each (R = 4: a
// scanned split merge per wavefront-row; R = 1: the four wavefronts merge the row together).
// The remaining workgroups store the window of one request each; both branches have read the
// window before this launch, and the merges do not touch it.
// Grid (merge_wgs + requests, kQuarters == 1 ? 4 : 1): workgroup (x, y) serves R rows
// (merge_mode's rule: R = 1 for a workgroup-row merge) for output columns [64 y, 64 y + 64),
// or for all 256 columns when kQuarters is 4 (many rows: one merge per row instead of four,
// and a quarter of the workgroups); the window workgroups are those of y = 0; both branches
// have read the window before this launch, and the merges do not touch it.
// At most 256 registers per wavefront (two workgroups per CU): the scanned merge's two
// rounds of 16 partial rows in flight took the compiler to 260, one workgroup per CU, and
// the c4 launch (448 workgroups) into two rounds on 256 CUs.
template <int R, int kMode, int kQuarters = 1>
__global__ __launch_bounds__(kThreads, 2) void post_attention_kernel(const PostArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_h[R][kHeadDim];  // merged history rows
  __shared__ float s_l[R];
  __shared__ GroupMergeLds group_lds;
  if (static_cast<int>(blockIdx.x) < p.merge_wgs) {
    post_rows_quarter<R, kMode, kQuarters>(p, static_cast<int64_t>(blockIdx.x) * R,
                                           blockIdx.y, s_h, s_l, &group_lds);
    return;
  }
  if (blockIdx.y != 0) return;
  const int req = static_cast<int>(blockIdx.x) - p.merge_wgs;
  for (int head = 0; head < p.win.L.kv_heads; ++head) store_window_request(p.win, req, head);
}

// Many rows (a long chunk: thousands of (token, query head) rows, one split): 16 rows per
// workgroup, a full MFMA tile. Wavefront w merges rows w, w + 4, ... into LDS, then rotates
// the 16 rows back for its 64 output columns and merges them with the BF16 branch
// (post_rows_map: the row arithmetic of the other forms, the same bits). A workgroup reads
// R_v once per 16 rows instead of once per 4, and the launch needs a quarter of the
// workgroups of the 4-row form, whose rounds of latency set its time at these row counts.
// The one-round merge (one split) keeps two workgroups per CU (256 registers, a few spilled);
// the scanned merge of 16 rows with their rotation operands needs more than 256 and runs one
// workgroup per CU (two spilled about a hundred registers).
// kTiles 2 (one split): a workgroup walks two 16-row tiles with one read of R_v (per tile
// the rows take one round of loads, and R_v's 128 KB from L2 set the first tile's wait).
template <int kMode, int kTiles>
__global__ __launch_bounds__(kThreads, kMode == kMergeOneRound ? 2 : 1) void
post_attention_tile_kernel(const PostArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_h[16][kHeadDim];
  __shared__ float s_l[16];
  __shared__ GroupMergeLds group_lds;
  // The window-store workgroups come first: each walks its request's writers in sequence, so
  // started last they would end the launch.
  const int64_t win = p.win_requests;
  if (static_cast<int64_t>(blockIdx.x) >= win) {
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) - win) * 16 * kTiles;
    const int64_t rows = p.rows;
    post_rows_map<16, kMode, 4, kTiles>(
        p, [row0, rows](int r) -> int64_t { return row0 + r < rows ? row0 + r : -1; },
        p.splits, s_h, s_l, &group_lds);
    return;
  }
  const int req = static_cast<int>(blockIdx.x);
  for (int head = 0; head < p.win.L.kv_heads; ++head) store_window_request(p.win, req, head);
}

}  // namespace
}  // namespace oscar

namespace {
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

namespace oscar {
namespace {

// The checks and fields of one pre-attention launch (all roles; grid sizes in raw_wgs and
// kv_wgs, the q tiles follow when qrot is set). raw_partials and raw_lse both NULL: no BF16
// branch role (raw_wgs 0). OSCAR_OK with *p filled and *qrows = query rows per task, or the
// entry point's error code (OSCAR_OK with nothing filled when n == 0).
int make_pre_args(const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0,
                  int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1, const void* window,
                  int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
                  const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
                  const int32_t* counts, const int32_t* tasks, const int32_t* task_count,
                  int64_t n, int64_t hq, int64_t programs, int32_t block_n, int32_t query_tile,
                  int32_t max_query_len, float scale, const void* rk_t, const void* rv_t,
                  void* history, int64_t history_bytes, const int64_t* slots,
                  const oscar_clip* clip, const oscar_layout* layout, float* raw_partials,
                  float* raw_lse, void* qrot, PreArgs* out, int64_t* qrows_out) {
  PreArgs& p = *out;
  p = PreArgs{};
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
  *qrows_out = qrows;
  if (n == 0) return OSCAR_OK;
  const bool raw = raw_partials || raw_lse;
  if (!query || !key || !value || !window || !qstarts || !seq_lens || !block_tables || !counts ||
      !tasks || !task_count || !rk_t || !rv_t || !history || !slots ||
      (raw && (!raw_partials || !raw_lse)))
    return OSCAR_E_NULL;
  if (q_s0 % 8 || q_s1 % 8 || k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 || !aligned16(query) ||
      !aligned16(key) || !aligned16(value) || !aligned16(window) || !aligned16(rk_t) ||
      !aligned16(rv_t) || (raw && !aligned16(raw_partials)) || (qrot && !aligned16(qrot)) ||
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
  p.raw_wgs = raw ? static_cast<int32_t>(programs * h) : 0;
  p.kv_wgs = static_cast<int32_t>(2 * 4 * ((p.kv_rows + 15) / 16));
  return OSCAR_OK;
}

}  // namespace
}  // namespace oscar

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
  PreArgs p;
  int64_t qrows = 0;
  const int st = make_pre_args(query, q_s0, q_s1, key, k_s0, k_s1, value, v_s0, v_s1, window,
                               window_elems, qstarts, seq_lens, block_tables, table_stride,
                               table_columns, counts, tasks, task_count, n, hq, programs, block_n,
                               query_tile, max_query_len, scale, rk_t, rv_t, history,
                               history_bytes, slots, clip, layout, raw_partials, raw_lse, qrot,
                               &p, &qrows);
  if (st != OSCAR_OK || n == 0) return st;
  const int64_t q_wgs = qrot ? (p.q_rows + 15) / 16 : 0;  // NULL qrot: no q rotation role
  if (p.raw_wgs + p.kv_wgs + q_wgs > 0x7fffffffll) return OSCAR_E_SHAPE;
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

// oscar_history_pre, oscar_history_pre_q and oscar_history_pre_queue: `qrot_out` / `qsync` set
// (the second) or NULL; `queue` set (the third: 17-32 query rows per task) or NULL.
int history_pre_common(
    const void* query_rot, int64_t r_s0, int64_t r_s1, int64_t r_s2, const void* query,
    int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
    int64_t v_s0, int64_t v_s1, void* history, int64_t history_bytes, const void* window,
    int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, int64_t n,
    int64_t hq, int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile,
    int32_t max_query_len, float scale, int32_t split_tokens, const void* rk_t,
    const void* rv_t, const int64_t* slots, const oscar_clip* clip, const oscar_layout* layout,
    float* partials, float* lse, float* raw_partials, float* raw_lse, void* qrot_out,
    int32_t* qsync, int32_t* queue, void* stream) {
  if (n > 0 && (!raw_partials || !raw_lse)) return OSCAR_E_NULL;  // slice 0 is the BF16 branch
  PreArgs p;
  int64_t qrows = 0;
  int st = make_pre_args(query, q_s0, q_s1, key, k_s0, k_s1, value, v_s0, v_s1, window,
                         window_elems, qstarts, seq_lens, block_tables, table_stride,
                         table_columns, counts, tasks, task_count, n, hq, programs, block_n,
                         query_tile, max_query_len, scale, rk_t, rv_t, history, history_bytes,
                         slots, clip, layout, raw_partials, raw_lse, qrot_out, &p, &qrows);
  if (st != OSCAR_OK) return st;
  if (queue) {
    // 17-32 rows per task: the work queue with the roles as units of its own; the rotated
    // query is given, the split length token-bounded, the task rows within the queue's lists.
    if (qrows <= 16 || qrows > 32 || qsync || split_tokens == 0 || programs > kQueueTasks4)
      return OSCAR_E_UNSUPPORTED;
    if (!query_rot) return OSCAR_E_NULL;
    if (reinterpret_cast<uintptr_t>(queue) % 4) return OSCAR_E_ALIGN;
    AttnArgs a;
    int64_t hrows = 0;
    st = make_attn_args(query_rot, r_s0, r_s1, r_s2, nullptr, 0, 0, 1, nullptr, 0, 0, 1, history,
                        history_bytes, window, window_elems, qstarts, seq_lens, block_tables,
                        table_stride, table_columns, counts, tasks, task_count, n, hq, programs,
                        splits, block_n, query_tile, max_query_len, scale, 0, split_tokens,
                        layout, partials, lse, &a, &hrows);
    if (st != OSCAR_OK || n == 0) return st;
    return static_cast<int>(launch_history_queue_pre(a, p, queue, static_cast<int32_t>(programs),
                                                     as_stream(stream)));
  }
  if (qrows > 8) return OSCAR_E_UNSUPPORTED;
  // query_rot == nullptr: the history workgroups rotate the query rows themselves.
  const bool q_roles = qsync != nullptr;
  const bool rotate_query = !q_roles && query_rot == nullptr;
  if (q_roles) {
    // q rotation roles write qrot_out ([n, hq, 256] contiguous), the history reads it.
    if (!rk_t || !qrot_out) return OSCAR_E_NULL;
    if (!aligned16(qrot_out) || reinterpret_cast<uintptr_t>(qsync) % 4) return OSCAR_E_ALIGN;
    query_rot = qrot_out;
    r_s0 = hq * kHeadDim;
    r_s1 = kHeadDim;
    r_s2 = 1;
    p.qsync = qsync;
    p.q_wgs = static_cast<int32_t>((p.q_rows + 15) / 16);
  } else if (rotate_query) {
    if (!rk_t) return OSCAR_E_NULL;
    query_rot = query;
    r_s0 = q_s0;
    r_s1 = q_s1;
    r_s2 = 1;
  }
  AttnArgs a;
  int64_t hrows = 0;
  st = make_attn_args(query_rot, r_s0, r_s1, r_s2, nullptr, 0, 0, 1, nullptr, 0, 0, 1, history,
                      history_bytes, window, window_elems, qstarts, seq_lens, block_tables,
                      table_stride, table_columns, counts, tasks, task_count, n, hq, programs,
                      splits, block_n, query_tile, max_query_len, scale, 0, split_tokens, layout,
                      partials, lse, &a, &hrows);
  if (st != OSCAR_OK || n == 0) return st;
  // Role slices in front of the history splits (dispatched first): slice 0 is the BF16
  // branch of (task, kv head); the next ones hold the q rotation tiles (q roles) and then the
  // K/V store quads. Under the device rule the history slices hold unit slots.
  const int64_t per_slice = programs * a.L.kv_heads;
  const int role_slices =
      1 + static_cast<int>((p.kv_wgs + p.q_wgs + per_slice - 1) / per_slice);
  const int64_t hist_slices =
      split_tokens < 0 ? device_unit_slices(programs, a.L.kv_heads, split_tokens) : splits;
  if (hist_slices + role_slices > 65535) return OSCAR_E_SHAPE;
  if (q_roles && per_slice * (hist_slices + role_slices) > 0x7fffffffll) return OSCAR_E_SHAPE;
  if (split_tokens < 0 && programs > kDeviceUnitTasks) return OSCAR_E_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(programs), static_cast<unsigned>(a.L.kv_heads),
                  static_cast<unsigned>(hist_slices + role_slices));
  return static_cast<int>(
      launch_history_pre(a, p, role_slices, grid, rotate_query, as_stream(stream)));
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_history_pre(
    const void* query_rot, int64_t r_s0, int64_t r_s1, int64_t r_s2, const void* query,
    int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
    int64_t v_s0, int64_t v_s1, void* history, int64_t history_bytes, const void* window,
    int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, int64_t n,
    int64_t hq, int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile,
    int32_t max_query_len, float scale, int32_t split_tokens, const void* rk_t,
    const void* rv_t, const int64_t* slots, const oscar_clip* clip, const oscar_layout* layout,
    float* partials, float* lse, float* raw_partials, float* raw_lse, void* stream) {
  return oscar::history_pre_common(
      query_rot, r_s0, r_s1, r_s2, query, q_s0, q_s1, key, k_s0, k_s1, value, v_s0, v_s1,
      history, history_bytes, window, window_elems, qstarts, seq_lens, block_tables,
      table_stride, table_columns, counts, tasks, task_count, n, hq, programs, splits, block_n,
      query_tile, max_query_len, scale, split_tokens, rk_t, rv_t, slots, clip, layout, partials,
      lse, raw_partials, raw_lse, nullptr, nullptr, nullptr, stream);
}

extern "C" int oscar_history_pre_queue(
    const void* query_rot, int64_t r_s0, int64_t r_s1, int64_t r_s2, const void* query,
    int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
    int64_t v_s0, int64_t v_s1, void* history, int64_t history_bytes, const void* window,
    int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, int64_t n,
    int64_t hq, int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile,
    int32_t max_query_len, float scale, int32_t split_tokens, const void* rk_t,
    const void* rv_t, const int64_t* slots, const oscar_clip* clip, const oscar_layout* layout,
    float* partials, float* lse, float* raw_partials, float* raw_lse, int32_t* queue_counters,
    void* stream) {
  if (!queue_counters) return OSCAR_E_NULL;
  return oscar::history_pre_common(
      query_rot, r_s0, r_s1, r_s2, query, q_s0, q_s1, key, k_s0, k_s1, value, v_s0, v_s1,
      history, history_bytes, window, window_elems, qstarts, seq_lens, block_tables,
      table_stride, table_columns, counts, tasks, task_count, n, hq, programs, splits, block_n,
      query_tile, max_query_len, scale, split_tokens, rk_t, rv_t, slots, clip, layout, partials,
      lse, raw_partials, raw_lse, nullptr, nullptr, queue_counters, stream);
}

extern "C" int oscar_history_pre_q(
    void* qrot, int32_t* qsync, const void* query, int64_t q_s0, int64_t q_s1, const void* key,
    int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1, void* history,
    int64_t history_bytes, const void* window, int64_t window_elems, const int32_t* qstarts,
    const int32_t* seq_lens, const int32_t* block_tables, int64_t table_stride,
    int64_t table_columns, const int32_t* counts, const int32_t* tasks,
    const int32_t* task_count, int64_t n, int64_t hq, int64_t programs, int32_t splits,
    int32_t block_n, int32_t query_tile, int32_t max_query_len, float scale,
    int32_t split_tokens, const void* rk_t, const void* rv_t, const int64_t* slots,
    const oscar_clip* clip, const oscar_layout* layout, float* partials, float* lse,
    float* raw_partials, float* raw_lse, void* stream) {
  if (!qsync) return OSCAR_E_NULL;
  return oscar::history_pre_common(
      nullptr, 0, 0, 1, query, q_s0, q_s1, key, k_s0, k_s1, value, v_s0, v_s1, history,
      history_bytes, window, window_elems, qstarts, seq_lens, block_tables, table_stride,
      table_columns, counts, tasks, task_count, n, hq, programs, splits, block_n, query_tile,
      max_query_len, scale, split_tokens, rk_t, rv_t, slots, clip, layout, partials, lse,
      raw_partials, raw_lse, qrot, qsync, nullptr, stream);
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
  hipStream_t s = as_stream(stream);
  if (mode != kMergeScanGroup && p.rows >= kPostTileFrom) {
    const bool two = mode == kMergeOneRound && splits == 1;  // 32 rows per workgroup
    const int64_t span = two ? 32 : 16;
    const int64_t tiles = (p.rows + span - 1) / span;
    if (tiles + p.win_requests > 0x7fffffffll) return OSCAR_E_SHAPE;
    p.merge_wgs = static_cast<int32_t>(tiles);
    const dim3 grid(static_cast<unsigned>(tiles + p.win_requests));
    if (two)
      hipLaunchKernelGGL((post_attention_tile_kernel<kMergeOneRound, 2>), grid, dim3(kThreads), 0,
                         s, p);
    else if (mode == kMergeOneRound)
      hipLaunchKernelGGL((post_attention_tile_kernel<kMergeOneRound, 1>), grid, dim3(kThreads), 0,
                         s, p);
    else
      hipLaunchKernelGGL((post_attention_tile_kernel<kMergeScanWave, 1>), grid, dim3(kThreads), 0,
                         s, p);
    return static_cast<int>(hipGetLastError());
  }
  const bool wide = mode != kMergeScanGroup && p.rows >= kPostWideFrom;
  const int rows_per_wg = mode == kMergeScanGroup ? 1 : wide ? kPostWideRows : kPostQuarterRows;
  const int64_t groups = (p.rows + rows_per_wg - 1) / rows_per_wg;
  if (groups + p.win_requests > 0x7fffffffll) return OSCAR_E_SHAPE;
  p.merge_wgs = static_cast<int32_t>(groups);
  const dim3 grid(static_cast<unsigned>(groups + p.win_requests), wide ? 1 : 4);
  if (wide && mode == kMergeOneRound)
    hipLaunchKernelGGL((post_attention_kernel<kPostWideRows, kMergeOneRound, 4>), grid,
                       dim3(kThreads), 0, s, p);
  else if (wide)
    hipLaunchKernelGGL((post_attention_kernel<kPostWideRows, kMergeScanWave, 4>), grid,
                       dim3(kThreads), 0, s, p);
  else if (mode == kMergeOneRound)
    hipLaunchKernelGGL((post_attention_kernel<kPostQuarterRows, kMergeOneRound>), grid,
                       dim3(kThreads), 0, s, p);
  else if (mode == kMergeScanWave)
    hipLaunchKernelGGL((post_attention_kernel<kPostQuarterRows, kMergeScanWave>), grid,
                       dim3(kThreads), 0, s, p);
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
  // One-round split merge by the completing workgroup, paired-token history kernel, a split
  // rule fixed at launch (the completing workgroup counts a grid of (task, split) slots).
  if (qrows > 8 || splits > kWaveMergeSplits || splits + 1 > 65535 || split_tokens < 0)
    return OSCAR_E_UNSUPPORTED;
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
      query_tile > 4 || split_tokens < 0)
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
