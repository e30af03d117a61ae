// Allocation-free variant of oscar_history_post: the split partials, their LSEs and the
// completion counters live in one fixed device array of this library instead of caller
// buffers. For callers that cannot allocate device memory (code under graph capture, tight
// serving loops, harnesses that forbid hipMalloc). No reference counterpart.
//
// Scratch layout (bytes from the array's start):
//   [0, kCounterBytes)                 int32 completion counters, zero between calls
//   [kCounterBytes, kScratchBytes)     fp32 partials [n, hq, splits, 256], then fp32 LSEs
//                                      [n, hq, splits] (256-byte aligned)
// Each GPU holds its own copy of the array until the process ends. Every call on a GPU
// shares that GPU's array, so calls that overlap on one GPU (two streams at once) race.
#include <mutex>

#include "common.h"

namespace {

constexpr int64_t kScratchBytes = 32ll << 20;  // OSCAR_NOALLOC_SCRATCH_BYTES
constexpr int64_t kCounterBytes = 64ll << 10;  // 16384 counters
constexpr int kMaxDevices = 64;

static_assert(kScratchBytes == OSCAR_NOALLOC_SCRATCH_BYTES, "header and source agree");

__device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` per device (the host-side name is only a stand-in).
void* g_scratch[kMaxDevices];
std::mutex g_mutex;

__global__ void clear_counters_kernel(int32_t* counters, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counters[i] = 0;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

// This device's scratch address; the first call on a device resolves it and clears the
// counters on `stream` (a kernel, so the clear is ordered before the launch that follows).
int scratch_for_current_device(hipStream_t stream, uint8_t** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return static_cast<int>(err);
  if (dev < 0 || dev >= kMaxDevices) return OSCAR_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return static_cast<int>(err);
    if (!ptr) return static_cast<int>(hipErrorInvalidSymbol);
    const int n = static_cast<int>(kCounterBytes / 4);
    hipLaunchKernelGGL(clear_counters_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                       static_cast<int32_t*>(ptr), n);
    err = hipGetLastError();
    if (err != hipSuccess) return static_cast<int>(err);
    g_scratch[dev] = ptr;
  }
  *out = static_cast<uint8_t*>(g_scratch[dev]);
  return OSCAR_OK;
}

}  // namespace

extern "C" int64_t oscar_noalloc_scratch_bytes(int64_t n, int64_t hq, int32_t splits) {
  if (n < 0 || hq < 0 || splits < 0) return -1;
  const int64_t rows = n * hq * splits;
  return kCounterBytes + align256(rows * oscar::kHeadDim * 4) + align256(rows * 4);
}

extern "C" int oscar_history_post_noalloc(
    const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2, const void* history,
    int64_t history_bytes, const int32_t* qstarts, const int32_t* seq_lens,
    const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
    const int32_t* counts, const int32_t* tasks, const int32_t* task_count, int64_t n, int64_t hq,
    int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile, int32_t max_query_len,
    float scale, int32_t split_tokens, const oscar_layout* layout, const float* raw_partials,
    const float* raw_lse, const void* rv, void* output, float* merged_lse, const void* key,
    int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1, void* window,
    int64_t window_elems, int64_t max_reqs, void* stream) {
  if (!layout) return OSCAR_E_NULL;
  if (n < 0 || hq <= 0 || splits <= 0 || programs <= 0) return OSCAR_E_SHAPE;
  // Sizes beyond the fixed array are refused before anything is launched.
  if (oscar_noalloc_scratch_bytes(n, hq, splits) > kScratchBytes) return OSCAR_E_SCRATCH;
  if (programs * static_cast<int64_t>(layout->kv_heads) > kCounterBytes / 4)
    return OSCAR_E_SCRATCH;
  if (n == 0) return OSCAR_OK;
  uint8_t* base = nullptr;
  const int st = scratch_for_current_device(oscar::as_stream(stream), &base);
  if (st != OSCAR_OK) return st;
  const int64_t rows = n * hq * splits;
  int32_t* counters = reinterpret_cast<int32_t*>(base);
  float* partials = reinterpret_cast<float*>(base + kCounterBytes);
  float* lse = reinterpret_cast<float*>(base + kCounterBytes + align256(rows * oscar::kHeadDim * 4));
  return oscar_history_post(query, q_s0, q_s1, q_s2, history, history_bytes, qstarts, seq_lens,
                            block_tables, table_stride, table_columns, counts, tasks, task_count,
                            n, hq, programs, splits, block_n, query_tile, max_query_len, scale,
                            split_tokens, layout, partials, lse, counters, kCounterBytes / 4,
                            raw_partials, raw_lse, rv, output, merged_lse, key, k_s0, k_s1, value,
                            v_s0, v_s1, window, window_elems, max_reqs, stream);
}
