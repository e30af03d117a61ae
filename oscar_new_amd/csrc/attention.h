// Task, split and query-row bookkeeping shared by the two attention branches (INT2 history
// in history.hip, BF16 sink/ring/current window in attention.hip).
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel`, `attention_partials`).
// One workgroup per (task, kv head, split); a task is (request, first query row) from the
// compact task table; partial outputs are per-split normalized with a natural-log LSE.
#pragma once

#include "common.h"

namespace oscar {

constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kSlot = 160, kVector = 68;

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
  int32_t split_tokens;  // history branch: 0 = kernels.py:368-370 rule, else token-bounded
  FastDiv g_div;  // division by g (query heads per kv head)
  float scale_log2;
  // BF16 branch written as the layer output (initial prefill, no history): bf16 rows
  // [n][hq][256] and, when non-null, their LSE [n][hq].
  uint16_t* direct_out;
  float* direct_lse;
};

struct Task {
  int req, qoff, qstart, qlen, prefix, sink_len, recent_begin;
};

// kernels.py:316-333: the task row, the request's query span and its history bounds.
// The task row is loaded together with the task count (rows below `programs` are always
// allocated), so the dependent loads form two levels instead of three.
__device__ __forceinline__ bool read_task(const AttnArgs& a, Task& t, int task) {
  const int count = a.task_count[0];
  const int req = a.tasks[2 * task];
  const int qoff = a.tasks[2 * task + 1];
  if (task >= count) return false;
  t.req = req;
  t.qoff = qoff;
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

// Splits a request's history uses. The reference rule (split_tokens 0) gives every request
// all `splits`; the token-bounded rule gives a request of `length` history tokens
// min(splits, max(1, ceil(length / split_tokens))) of them, so that a ragged batch splits
// its long requests finely and its short ones not at all. The ranges inside that count
// follow split_range either way.
__device__ __forceinline__ int history_splits(const AttnArgs& a, int length) {
  if (a.split_tokens <= 0) return a.splits;
  return min(a.splits, max(1, cdiv(max(length, 0), a.split_tokens)));
}

// Absolute positions [p_lo, p_hi) of history split `split` of a task with `length` history
// tokens (positions sink_len .. sink_len + length). The reference rule (split_tokens 0):
// split_range's history-relative ranges (kernels.py:368-370) moved up by sink_len. The
// token-bounded rule (split_tokens > 0, no reference counterpart) moves every inner boundary
// down to the 64-token chunk grid of absolute positions: with a 4-token sink the reference
// boundaries sit 4 tokens past a chunk boundary, so each split would touch 33 chunks of 64
// (the chunk on each boundary read by both of its splits, one of the four wavefronts
// streaming 9 chunks while the others stream 8); aligned, a full split is exactly 32.
__device__ __forceinline__ void history_positions(const AttnArgs& a, const Task& t, int length,
                                                  int nsplit, int split, int& p_lo, int& p_hi) {
  int begin, end;
  split_range(length, a.block_n, nsplit, split, begin, end);
  if (a.split_tokens <= 0) {
    p_lo = max(t.sink_len + begin, 0);
    p_hi = t.sink_len + end;
    return;
  }
  const int lo = t.sink_len, hi = t.sink_len + max(length, 0);
  auto cut = [&](int h) {
    if (h <= 0) return lo;
    if (h >= length) return hi;
    return max(lo, (lo + h) & ~63);
  };
  p_lo = cut(begin);
  p_hi = cut(end);
}

struct RowInfo {
  bool valid;
  int qi, qhead;
  int64_t token;
};

// Query row `row` of a task: query index qi = qoff + row / G, head = head * G + row % G.
__device__ __forceinline__ RowInfo row_info(const AttnArgs& a, const Task& t, int head, int row) {
  RowInfo r;
  const int qrow = static_cast<int>(fastdiv(static_cast<uint32_t>(row), a.g_div));
  r.qi = t.qoff + qrow;
  r.token = static_cast<int64_t>(t.qstart) + r.qi;
  r.valid = row < a.qt * a.g && r.qi < t.qlen && r.token >= 0 && r.token < a.n;
  r.qhead = head * a.g + (row - qrow * a.g);
  return r;
}

// A split slot beyond the request's history_splits: only its LSE is written (-inf), which
// the split merges skip without reading the partial row.
__device__ __forceinline__ void write_unused_split(const AttnArgs& a, const Task& t, int head,
                                                   int split) {
  for (int row = threadIdx.x; row < a.qt * a.g; row += kThreads) {
    const RowInfo ri = row_info(a, t, head, row);
    if (ri.valid) a.lse[(ri.token * a.hq + ri.qhead) * a.splits + split] = -INFINITY;
  }
}

// INT2 history branch (history.hip); rows = query rows per task (<= 32).
// `queue`: two zeroed int32 counters for the work-queue form of the 17-32-row kernel
// (token-bounded splits), or nullptr for the grid form.
hipError_t launch_history(const AttnArgs& a, dim3 grid, int rows, hipStream_t stream,
                          int32_t* queue = nullptr);

// The checks and fields of one attention_partials launch (attention.hip): OSCAR_OK with *out
// filled and *qrows = query rows per task, or the entry point's error code. Nothing is
// launched when n == 0 (OSCAR_OK before the pointer checks).
int make_attn_args(const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* key,
                   int64_t k_s0, int64_t k_s1, int64_t k_s2, const void* value, int64_t v_s0,
                   int64_t v_s1, int64_t v_s2, const void* history, int64_t history_bytes,
                   const void* window, int64_t window_elems, const int32_t* qstarts,
                   const int32_t* seq_lens, const int32_t* block_tables, int64_t table_stride,
                   int64_t table_columns, const int32_t* counts, const int32_t* tasks,
                   const int32_t* task_count, int64_t n, int64_t hq, int64_t programs,
                   int32_t splits, int32_t block_n, int32_t query_tile, int32_t max_query_len,
                   float scale, int32_t raw, int32_t split_tokens, const oscar_layout* layout,
                   float* partials, float* lse, AttnArgs* out, int64_t* qrows);

}  // namespace oscar
