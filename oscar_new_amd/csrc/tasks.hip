// prepare_tasks: device-built compact task table (request, query offset) per query tile.
//
// Reference: oscar_ascend/kernels.py:222-287 (`_prepare_tasks_kernel`, `prepare_tasks`).
// One workgroup per program (request). Each workgroup recomputes the exclusive prefix sum of
// tile counts of the requests before it, so no inter-workgroup communication is needed and
// the table is identical for any program execution order.
#include "common.h"

namespace oscar {
namespace {

struct TaskArgs {
  const int32_t* qstarts;
  const int32_t* counts;
  int32_t* tasks;
  int32_t* task_count;
  int64_t capacity;
  int32_t limit;  // requests that may contribute: min(next_pow2(max_reqs), max_reqs)
  int32_t query_tile;
  const int32_t* source;
  int64_t source_stride;
  int32_t* table;
  int64_t table_stride;
  int64_t copy_columns;
};

__device__ __forceinline__ int tiles_of(const TaskArgs& a, int r, int active) {
  const int start = min(a.qstarts[r], active);
  const int end = min(a.qstarts[r + 1], active);
  return cdiv(max(end - start, 0), a.query_tile);
}

__global__ __launch_bounds__(kThreads) void prepare_tasks_kernel(const TaskArgs a) {
  __shared__ int s_before[kThreads / kWave], s_all[kThreads / kWave];
  const int req = blockIdx.x;
  const int nr = a.counts[0], active = a.counts[1];
  if (a.source && req < min(nr, a.limit)) {
    for (int64_t c = threadIdx.x; c < a.copy_columns; c += kThreads)
      a.table[req * a.table_stride + c] = a.source[req * a.source_stride + c];
  }
  const int live = min(nr, a.limit);
  int before = 0, all = 0;
  for (int r = threadIdx.x; r < live; r += kThreads) {
    const int t = tiles_of(a, r, active);
    all += t;
    if (r < req) before += t;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    before += __shfl_xor(before, m, kWave);
    all += __shfl_xor(all, m, kWave);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    s_before[wave] = before;
    s_all[wave] = all;
  }
  __syncthreads();
  before = s_before[0] + s_before[1] + s_before[2] + s_before[3];
  all = s_all[0] + s_all[1] + s_all[2] + s_all[3];
  if (req == 0 && threadIdx.x == 0) a.task_count[0] = all;
  const int count = req < live ? tiles_of(a, req, active) : 0;
  for (int j = threadIdx.x; j < count; j += kThreads) {
    const int64_t idx = static_cast<int64_t>(before) + j;
    if (idx < a.capacity) {
      a.tasks[2 * idx] = req;
      a.tasks[2 * idx + 1] = j * a.query_tile;
    }
  }
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_prepare_tasks(const int32_t* qstarts, const int32_t* counts, int32_t* tasks,
                                   int32_t* task_count, int64_t task_capacity, int64_t max_reqs,
                                   int32_t query_tile, int64_t programs,
                                   const int32_t* source_table, int64_t source_stride,
                                   int32_t* table, int64_t table_stride, int64_t copy_columns,
                                   void* stream) {
  using namespace oscar;
  if (max_reqs < 1 || query_tile < 1 || programs < 1 || task_capacity < 0 || copy_columns < 0)
    return OSCAR_E_SHAPE;
  if (!qstarts || !counts || !tasks || !task_count) return OSCAR_E_NULL;
  if (source_table && (!table || copy_columns > table_stride)) return OSCAR_E_SHAPE;
  if (max_reqs > (1ll << 30) || programs > (1ll << 30)) return OSCAR_E_SHAPE;
  int64_t lanes = 1;
  while (lanes < max_reqs) lanes <<= 1;
  TaskArgs a{qstarts, counts, tasks, task_count, task_capacity,
             static_cast<int32_t>(lanes < max_reqs ? lanes : max_reqs), query_tile,
             source_table, source_stride, table, table_stride,
             source_table ? copy_columns : 0};
  hipLaunchKernelGGL(prepare_tasks_kernel, dim3(static_cast<unsigned>(programs)), dim3(kThreads),
                     0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}
