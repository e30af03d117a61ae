// Split-KV paged decode attention: the BF16 branch (sink, recent ring and current tokens)
// and the C-ABI entry point of both branches; the INT2 history branch is history.hip.
//
// Reference: oscar_ascend/kernels.py:290-482 (`_attention_kernel` with IS_RAW true: raw
// positions = sink + recent window + causal current tokens, kernels.py:421-470).
//
// The BF16 branch's row arithmetic and workgroup layout are raw.h's.
#include "raw.h"

namespace oscar {
namespace {

template <int RT>
__global__ __launch_bounds__(kThreads) void raw_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRawSlots * kRawLdsPerSlot];
  raw_block_staged<RT>(a, blockIdx.x, blockIdx.y, blockIdx.z, ring, kRawSlots);
}

}  // namespace
}  // namespace oscar

namespace oscar {

int make_attn_args(const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* key,
                   int64_t k_s0, int64_t k_s1, int64_t k_s2, const void* value, int64_t v_s0,
                   int64_t v_s1, int64_t v_s2, const void* history, int64_t history_bytes,
                   const void* window, int64_t window_elems, const int32_t* qstarts,
                   const int32_t* seq_lens, const int32_t* block_tables, int64_t table_stride,
                   int64_t table_columns, const int32_t* counts, const int32_t* tasks,
                   const int32_t* task_count, int64_t n, int64_t hq, int64_t programs,
                   int32_t splits, int32_t block_n, int32_t query_tile, int32_t max_query_len,
                   float scale, int32_t raw, int32_t split_tokens, const oscar_layout* layout,
                   float* partials, float* lse, AttnArgs* out, int64_t* qrows_out) {
  AttnArgs& a = *out;
  a = AttnArgs{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  const int64_t h = a.L.kv_heads;
  if (n < 0 || hq <= 0 || hq % h || programs < 1 || splits < 1 || splits > 65535 ||
      block_n < 1 || query_tile < 1 || table_columns < 0 || programs > (1ll << 31) - 1)
    return OSCAR_E_SHAPE;
  if (raw && split_tokens) return OSCAR_E_UNSUPPORTED;  // the BF16 branch keeps one rule
  const int64_t g = hq / h;
  const int64_t qrows = (max_query_len > 0 && max_query_len < query_tile ? max_query_len
                                                                         : query_tile) * g;
  if (qrows > 32) return OSCAR_E_UNSUPPORTED;
  *qrows_out = qrows;
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
    // The history kernel streams 64-token chunks that never straddle a kernel block, and
    // its masked (unmapped-block) chunks read the first 64 records of the buffer.
    if (a.L.bk < 64) return OSCAR_E_UNSUPPORTED;
    if (history_bytes < 64 * h * 160) return OSCAR_E_SHAPE;
    if (!(scale > 0.f) || !(scale < INFINITY)) return OSCAR_E_UNSUPPORTED;
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
  a.g_div = make_fastdiv(static_cast<uint32_t>(g));
  a.hq = static_cast<int32_t>(hq);
  a.qt = query_tile;
  a.splits = splits;
  a.block_n = block_n;
  a.split_tokens = split_tokens;
  a.scale_log2 = scale * kLog2e;
  return OSCAR_OK;
}

}  // namespace oscar

extern "C" int oscar_attention_partials(
    const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* key, int64_t k_s0,
    int64_t k_s1, int64_t k_s2, const void* value, int64_t v_s0, int64_t v_s1, int64_t v_s2,
    const void* history, int64_t history_bytes, const void* window, int64_t window_elems,
    const int32_t* qstarts, const int32_t* seq_lens, const int32_t* block_tables,
    int64_t table_stride, int64_t table_columns, const int32_t* counts, const int32_t* tasks,
    const int32_t* task_count, int64_t n, int64_t hq, int64_t programs, int32_t splits,
    int32_t block_n, int32_t query_tile, int32_t max_query_len, float scale, int32_t raw,
    int32_t split_tokens, const oscar_layout* layout, float* partials, float* lse,
    int32_t* queue_counters, void* stream) {
  using namespace oscar;
  AttnArgs a;
  int64_t qrows = 0;
  const int st = make_attn_args(query, q_s0, q_s1, q_s2, key, k_s0, k_s1, k_s2, value, v_s0, v_s1,
                                v_s2, history, history_bytes, window, window_elems, qstarts,
                                seq_lens, block_tables, table_stride, table_columns, counts, tasks,
                                task_count, n, hq, programs, splits, block_n, query_tile,
                                max_query_len, scale, raw, split_tokens, layout, partials, lse, &a,
                                &qrows);
  if (st != OSCAR_OK || n == 0) return st;
  // The paired kernel (<= 8 rows) under the device rule: z slices of unit slots.
  const int64_t z = !raw && qrows <= 8 && split_tokens < 0
                        ? device_unit_slices(programs, a.L.kv_heads, split_tokens)
                        : splits;
  if (z > 65535) return OSCAR_E_SHAPE;
  if (!raw && qrows <= 8 && split_tokens < 0 && programs > kDeviceUnitTasks)
    return OSCAR_E_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(programs), static_cast<unsigned>(a.L.kv_heads),
                  static_cast<unsigned>(z));
  hipStream_t s = as_stream(stream);
  if (!raw)
    return static_cast<int>(launch_history(a, grid, static_cast<int>(qrows), s, queue_counters));
  if (qrows <= 16)
    hipLaunchKernelGGL(raw_kernel<1>, grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(raw_kernel<2>, grid, dim3(kThreads), 0, s, a);
  return static_cast<int>(hipGetLastError());
}

