// Window store of one request: the current BF16 K/V into its sink/ring window, shared by the
// store_windows entry point and the fused post-attention kernel.
//
// Reference: oscar_ascend/kernels.py:544-620 (`_window_store_kernel`, `store_windows`).
// Window index i < S holds position i. Ring index i >= S holds the LATEST position
// pos < seq with pos = i - S (mod C); only current tokens (prefix <= pos < seq) are
// written, so each ring slot has exactly one writer per step.
#pragma once

#include "common.h"

namespace oscar {


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

// One (request, kv head) of kernels.py:569-595, by the four wavefronts of a workgroup.
// Stated per index, the reference rule is: index i < S receives position i, ring index i
// receives the latest position pos < seq with pos = i - S (mod C), and only current tokens
// (prefix <= pos < seq) are written, never a ring write of a position below S. Stated per
// current token, that is the same set of writes: token pos writes index pos if pos < S, else
// index S + pos % C if no later token of the request has the same residue (pos + C >= seq).
// Each index therefore has at most one writer. The writers are the sink tokens
// [prefix, min(S, seq)) and the ring tokens [max(prefix, S, seq - C), seq): at most S + C of
// them however long the chunk, taken kBatch at a time per wavefront (writer j by wavefront
// (j / kBatch) mod 4), each batch's rows all requested before any is stored.
__device__ __forceinline__ void store_window_request(const WindowArgs& a, int req, int head) {
  constexpr int kBatch = 8;
  if (req >= a.counts[0]) return;
  const int qstart = a.qstarts[req];
  const int qend = min(a.qstarts[req + 1], a.counts[1]);
  const int seq = a.seq_lens[req];
  const int first = a.table[static_cast<int64_t>(req) * a.table_stride];
  if (qend <= qstart || first < 0) return;
  const int prefix = seq - (qend - qstart);
  const int64_t owner = fastdiv(static_cast<uint32_t>(first), a.L.bpp_div);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = a.L.kv_heads, sink = a.L.sink, ring = a.L.ring;
  const int64_t page_elems = a.L.page_bytes / 2;
  const int s0 = max(prefix, 0), s1 = max(s0, min(sink, seq));  // sink writers
  const int r0 = max(max(prefix, sink), seq - ring), r1 = max(r0, seq);  // ring writers
  const int nsink = s1 - s0, total = nsink + (r1 - r0);
  const bool vec = a.ks2 == 1 && a.vs2 == 1 && a.ks0 % 4 == 0 && a.ks1 % 4 == 0 &&
                   a.vs0 % 4 == 0 && a.vs1 % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(a.k) % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(a.v) % 8 == 0;
  const bool vst = reinterpret_cast<uintptr_t>(a.window) % 8 == 0;
  for (int base = wave * kBatch; base < total; base += (kThreads / kWave) * kBatch) {
    uint16_t kx[kBatch][4], vx[kBatch][4];
    int64_t dst[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int j = base + b;
      dst[b] = -1;
      if (j >= total) continue;
      const int pos = j < nsink ? s0 + j : r0 + (j - nsink);
      int index = pos;
      if (pos >= sink) {
        const uint32_t lap = fastdiv(static_cast<uint32_t>(pos), a.L.ring_div);
        index = sink + pos - static_cast<int>(lap) * ring;
      }
      const int64_t current = static_cast<int64_t>(qstart) + pos - prefix;
      if (current < 0 || current >= a.n) continue;
      const int64_t d = owner * page_elems + (static_cast<int64_t>(index) * 2 * h + head) * kHeadDim;
      if (d + static_cast<int64_t>(h) * kHeadDim + kHeadDim > a.window_elems) continue;
      dst[b] = d;
      const uint16_t* ks = a.k + current * a.ks0 + head * a.ks1;
      const uint16_t* vs = a.v + current * a.vs0 + head * a.vs1;
      if (vec) {  // contiguous, 8-byte aligned rows: one 8-byte load per lane and row
        const uint2 kw = *reinterpret_cast<const uint2*>(ks + lane * 4);
        const uint2 vw = *reinterpret_cast<const uint2*>(vs + lane * 4);
        kx[b][0] = kw.x & 0xffffu, kx[b][1] = kw.x >> 16, kx[b][2] = kw.y & 0xffffu, kx[b][3] = kw.y >> 16;
        vx[b][0] = vw.x & 0xffffu, vx[b][1] = vw.x >> 16, vx[b][2] = vw.y & 0xffffu, vx[b][3] = vw.y >> 16;
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = lane * 4 + i;
        kx[b][i] = ks[e * a.ks2];
        vx[b][i] = vs[e * a.vs2];
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (dst[b] < 0) continue;
      uint16_t* kd = a.window + dst[b];
      uint16_t* vd = kd + static_cast<int64_t>(h) * kHeadDim;
      if (vst) {  // window rows start 512 bytes apart from an 8-byte aligned base
        *reinterpret_cast<uint2*>(kd + lane * 4) =
            make_uint2(kx[b][0] | (static_cast<uint32_t>(kx[b][1]) << 16),
                       kx[b][2] | (static_cast<uint32_t>(kx[b][3]) << 16));
        *reinterpret_cast<uint2*>(vd + lane * 4) =
            make_uint2(vx[b][0] | (static_cast<uint32_t>(vx[b][1]) << 16),
                       vx[b][2] | (static_cast<uint32_t>(vx[b][3]) << 16));
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kd[lane * 4 + i] = kx[b][i];
        vd[lane * 4 + i] = vx[b][i];
      }
    }
  }
}

}  // namespace oscar
