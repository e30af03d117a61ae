// store_windows: write the current BF16 K/V into each request's sink/ring window.
//
// Reference: oscar_ascend/kernels.py:544-620 (`_window_store_kernel`, `store_windows`).
// Window index i < S holds position i. Ring index i >= S holds the LATEST position
// pos < seq with pos = i - S (mod C); only current tokens (prefix <= pos < seq) are
// written, so each ring slot has exactly one writer per step. One workgroup per
// (request, kv head); wavefront w copies window indices w, w+4, ... (1 KiB each).
#include "common.h"

namespace oscar {
namespace {

struct WindowArgs {
  const uint16_t* k;
  int64_t ks0, ks1, ks2;
  const uint16_t* v;
  int64_t vs0, vs1, vs2;
  int64_t n;
  uint16_t* window;
  int64_t window_elems;
  const int32_t* qstarts;
  const int32_t* seq_lens;
  const int32_t* table;
  int64_t table_stride;
  const int32_t* counts;
  Layout L;
};

__global__ __launch_bounds__(kThreads) void store_windows_kernel(const WindowArgs a) {
  const int req = blockIdx.x, head = blockIdx.y;
  if (req >= a.counts[0]) return;
  const int qstart = a.qstarts[req];
  const int qend = min(a.qstarts[req + 1], a.counts[1]);
  if (qend <= qstart) return;
  const int seq = a.seq_lens[req];
  const int prefix = seq - (qend - qstart);
  const int first = a.table[static_cast<int64_t>(req) * a.table_stride];
  if (first < 0) return;
  const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = a.L.kv_heads, sink = a.L.sink, ring = a.L.ring;
  const int64_t page_elems = a.L.page_bytes / 2;
  for (int index = wave; index < sink + ring; index += kThreads / kWave) {
    int pos;
    if (index < sink) {
      pos = index;
    } else {
      const int back = seq - 1 - (index - sink);  // distance of the newest candidate
      if (back < 0) continue;
      pos = seq - 1 - back % ring;
      if (pos < sink) continue;
    }
    if (pos < prefix || pos >= seq) continue;
    const int64_t current = static_cast<int64_t>(qstart) + pos - prefix;
    if (current < 0 || current >= a.n) continue;
    const int64_t dst = owner * page_elems + (static_cast<int64_t>(index) * 2 * h + head) * kHeadDim;
    if (dst + static_cast<int64_t>(h) * kHeadDim + kHeadDim > a.window_elems) continue;
    const uint16_t* ks = a.k + current * a.ks0 + head * a.ks1;
    const uint16_t* vs = a.v + current * a.vs0 + head * a.vs1;
    uint16_t* kd = a.window + dst;
    uint16_t* vd = a.window + dst + static_cast<int64_t>(h) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane * 4 + i;
      kd[d] = ks[d * a.ks2];
      vd[d] = vs[d * a.vs2];
    }
  }
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
