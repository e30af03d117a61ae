// store_windows: write the current BF16 K/V into each request's sink/ring window.
//
// Reference: oscar_ascend/kernels.py:544-620 (`_window_store_kernel`, `store_windows`).
// Window index i < S holds position i. Ring index i >= S holds the LATEST position
// pos < seq with pos = i - S (mod C); only current tokens (prefix <= pos < seq) are
// written, so each ring slot has exactly one writer per step. One workgroup per
// (request, kv head); wavefront w copies window indices w, w+4, ... (1 KiB each).
#include "window.h"

namespace oscar {
namespace {

__global__ __launch_bounds__(kThreads) void store_windows_kernel(const WindowArgs a) {
  store_window_request(a, blockIdx.x, blockIdx.y);
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_store_windows(const void* key, int64_t k_s0, int64_t k_s1, int64_t k_s2,
                                   const void* value, int64_t v_s0, int64_t v_s1, int64_t v_s2,
                                   int64_t n, void* window, int64_t window_elems,
                                   const int32_t* qstarts, const int32_t* seq_lens,
                                   const int32_t* block_tables, int64_t table_stride,
                                   const int32_t* counts, int64_t max_reqs,
                                   const oscar_layout* layout, void* stream) {
  using namespace oscar;
  if (n < 0 || max_reqs < 0 || window_elems < 0) return OSCAR_E_SHAPE;
  WindowArgs a{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  const int64_t programs = n < max_reqs ? n : max_reqs;
  if (programs == 0) return OSCAR_OK;
  if (!key || !value || !window || !qstarts || !seq_lens || !block_tables || !counts)
    return OSCAR_E_NULL;
  a.k = static_cast<const uint16_t*>(key);
  a.ks0 = k_s0;
  a.ks1 = k_s1;
  a.ks2 = k_s2;
  a.v = static_cast<const uint16_t*>(value);
  a.vs0 = v_s0;
  a.vs1 = v_s1;
  a.vs2 = v_s2;
  a.n = n;
  a.window = static_cast<uint16_t*>(window);
  a.window_elems = window_elems;
  a.qstarts = qstarts;
  a.seq_lens = seq_lens;
  a.table = block_tables;
  a.table_stride = table_stride;
  a.counts = counts;
  hipLaunchKernelGGL(store_windows_kernel,
                     dim3(static_cast<unsigned>(programs), static_cast<unsigned>(a.L.kv_heads)),
                     dim3(kThreads), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}
