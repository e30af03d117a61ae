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
  // History branch split rule: 0 = kernels.py:368-370; > 0 = token-bounded splits of at most
  // about split_tokens tokens; < 0 = the device rule (token-bounded splits whose length the
  // kernel derives from the step's lengths, for a budget of -split_tokens workgroups).
  int32_t split_tokens;
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
// follow split_range either way. `split_tokens` is the launch's value, or under the device
// rule the length device_split_tokens derived.
__device__ __forceinline__ int history_splits(const AttnArgs& a, int length, int split_tokens) {
  if (split_tokens <= 0) return a.splits;
  return min(a.splits, max(1, cdiv(max(length, 0), split_tokens)));
}

// ---------------------------------------------------------------- device split rule
//
// No reference counterpart. The reference sizes splits from host request counts alone
// (config.py:84-89) so that one captured graph serves every context length. A split length
// computed on the host from the step's lengths would be frozen into a captured graph at the
// dummy batch's lengths; under the device rule (split_tokens = -B) every workgroup derives it
// from the lengths in device memory, for a budget of B workgroups:
//   T = max(1024, 64 * ceil(ceil(H * total / room) / 64)),
// total = the tasks' history tokens, H kv heads. A task of L history tokens takes
// min(splits, max(1, ceil(L / T))) splits. For a grid of B unit slots (the paired kernel,
// `fit_grid`) room = max(1, B - H * tasks), so that all tasks together take at most
// total / T + tasks <= room / H + tasks units per kv head: B / H when the budget exceeds one
// unit per task, tasks + 1 otherwise. The grid and work-queue forms of the other kernels
// have a slot per (task, split) or take units as they come: room = B, about B units.
constexpr int kDeviceMinSplit = 1024;

__device__ __forceinline__ int device_split_tokens(int64_t total, int tasks, int heads,
                                                   int budget, bool fit_grid) {
  const int64_t reserve = fit_grid ? static_cast<int64_t>(heads) * tasks : 0;
  const int64_t room = max(static_cast<int64_t>(1), static_cast<int64_t>(budget) - reserve);
  const int64_t per = (static_cast<int64_t>(heads) * total + room - 1) / room;
  const int64_t t = (per + 63) / 64 * 64;
  return static_cast<int>(min(max(t, static_cast<int64_t>(kDeviceMinSplit)),
                              static_cast<int64_t>(1) << 30));
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// History tokens of a task (0 for an inactive row).
__device__ __forceinline__ int task_history(const AttnArgs& a, int task) {
  Task t;
  return read_task(a, t, task) ? max(t.recent_begin - t.sink_len, 0) : 0;
}

// The split length of the launch: split_tokens itself, or under the device rule T from the
// lengths of the task rows below `programs`, summed by the NT threads of the workgroup (all
// of them call it; every thread returns the same value).
template <int NT>
__device__ __forceinline__ int launch_split_tokens(const AttnArgs& a, int programs) {
  if (a.split_tokens >= 0) return a.split_tokens;
  __shared__ int64_t s_wave_total[NT / kWave];
  int64_t s = 0;
  for (int i = threadIdx.x; i < programs; i += NT) s += task_history(a, i);
  s = wave_sum_i64(s);
  if ((threadIdx.x & (kWave - 1)) == 0) s_wave_total[threadIdx.x / kWave] = s;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) total += s_wave_total[w];
  const int count = min(a.task_count[0], programs);
  __syncthreads();  // s_wave_total is read before a later call reuses it
  return device_split_tokens(total, max(count, 0), a.L.kv_heads, -a.split_tokens, false);
}

// A unit of the device rule: the (task, split) that workgroup slot `u` computes. Units run
// task-major (task i holds units [base_i, base_i + nsplit_i), base the exclusive scan of
// nsplit over the task rows), so one captured grid of at least
// max(B / H, programs + 1) slots per kv head covers any lengths; the slots past the last
// unit compute nothing.
struct DeviceUnit {
  Task t;
  int task, split, nsplit, split_tokens;
};

// Every thread of the NT-thread workgroup calls it. `scratch`: LDS for programs + 16 ints,
// free until the call returns. False for a slot past the last unit.
template <int NT>
__device__ bool device_unit(const AttnArgs& a, int programs, int u, int* scratch,
                            DeviceUnit& out) {
  constexpr int kWaves = NT / kWave;
  int* nsplit = scratch;  // per task row: history length, then split count
  __shared__ int64_t s_total[kWaves];
  __shared__ int s_carry[kWaves + 1];
  __shared__ int s_found[9];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  int64_t s = 0;
  // The row of this thread's last task stays in registers: with at most NT task rows, the
  // thread that finds the unit's task has its row already (no second round of loads).
  Task mine{};
  int mine_task = -1;
  for (int i = threadIdx.x; i < programs; i += NT) {
    Task t;
    const bool live = read_task(a, t, i);
    const int len = live ? max(t.recent_begin - t.sink_len, 0) : 0;
    nsplit[i] = len;
    s += len;
    mine = t;
    mine_task = live ? i : -1;
  }
  s = wave_sum_i64(s);
  if (lane == 0) s_total[wave] = s;
  if (threadIdx.x == 0) s_found[0] = -1;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total += s_total[w];
  const int count = max(min(a.task_count[0], programs), 0);
  const int st = device_split_tokens(total, count, a.L.kv_heads, -a.split_tokens, true);
  // Exclusive scan of the split counts, NT task rows at a time (inactive rows: 0 units).
  int carry = 0;
  for (int c0 = 0; c0 < programs; c0 += NT) {
    const int i = c0 + static_cast<int>(threadIdx.x);
    const int ns = i < count ? history_splits(a, nsplit[i], st) : 0;
    int incl = ns;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int y = __shfl_up(incl, d, kWave);
      incl += lane >= d ? y : 0;
    }
    if (lane == kWave - 1) s_carry[wave] = incl;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += s_carry[w];
    int chunk = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) chunk += s_carry[w];
    const int base = before + incl - ns;
    if (ns > 0 && u >= base && u < base + ns) {
      s_found[0] = i;
      s_found[1] = u - base;
      s_found[2] = ns;
      if (i == mine_task) {
        s_found[3] = mine.req;
        s_found[4] = mine.qoff;
        s_found[5] = mine.qstart;
        s_found[6] = mine.qlen;
        s_found[7] = mine.prefix;
        s_found[8] = mine.sink_len;
      } else {
        s_found[3] = -1;  // the row is read again below
      }
    }
    carry += chunk;
    __syncthreads();  // s_carry is read before the next chunk writes it
  }
  const int task = s_found[0];
  if (task >= 0 && s_found[3] < 0 && static_cast<int>(threadIdx.x) == 0) {
    Task t;
    read_task(a, t, task);  // the owner's row, again (the loads hit the L2)
    s_found[3] = t.req;
    s_found[4] = t.qoff;
    s_found[5] = t.qstart;
    s_found[6] = t.qlen;
    s_found[7] = t.prefix;
    s_found[8] = t.sink_len;
  }
  __syncthreads();
  if (task < 0) return false;
  out.task = task;
  out.split = s_found[1];
  out.nsplit = s_found[2];
  out.split_tokens = st;
  out.t.req = s_found[3];
  out.t.qoff = s_found[4];
  out.t.qstart = s_found[5];
  out.t.qlen = s_found[6];
  out.t.prefix = s_found[7];
  out.t.sink_len = s_found[8];
  out.t.recent_begin = max(out.t.sink_len, out.t.prefix - a.L.recent);
  return true;
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
                                                  int nsplit, int split, int split_tokens,
                                                  int& p_lo, int& p_hi) {
  int begin, end;
  split_range(length, a.block_n, nsplit, split, begin, end);
  if (split_tokens <= 0) {
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

// Grid z slices of unit slots for the paired kernel under the device rule (split_tokens < 0,
// budget -split_tokens): max(ceil(B / H), programs + 1) slots per kv head, programs per slice.
// Task rows the unit resolver lists (its scratch is the history kernel's ring, 72 KiB).
constexpr int64_t kDeviceUnitTasks = 16384;
inline int64_t device_unit_slices(int64_t programs, int64_t heads, int32_t split_tokens) {
  const int64_t budget = -static_cast<int64_t>(split_tokens);
  int64_t slots = (budget + heads - 1) / heads;
  if (slots < programs + 1) slots = programs + 1;
  return (slots + programs - 1) / programs;
}

// Split slots [from, to) a request does not use: LSE -inf for every live row of the task,
// (slot, row) pairs spread over the NT threads of the workgroup.
template <int NT>
__device__ __forceinline__ void write_unused_splits(const AttnArgs& a, const Task& t, int head,
                                                    int from, int to) {
  const int rows = a.qt * a.g, slots = to - from;
  for (int i = threadIdx.x; i < rows * max(slots, 0); i += NT) {
    const int row = i % rows, split = from + i / rows;
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
