// Post-attention folded into the history launch: the last split workgroup of a (task, kv
// head) to finish merges that task's rows, rotates them back and merges them with the BF16
// branch; an extra slice of the grid stores the windows and clears padded rows. It runs the
// row arithmetic of post_attention (post.h), so the two-launch step produces the bits of the
// three-launch one.
//
// Reference: oscar_ascend/backend.py:209-226 (`merge_splits`, `rotate(hrot, Rv.T)`,
// `merge_paths`, `store_windows` after both branches; kernels.py:485-620).
//
// Completion protocol (one counter per (task, kv head), zero between launches): every split
// workgroup writes its partial rows and LSEs with device-coherent stores (store_coherent),
// waits until they are done, and then one lane adds 1 to the counter (device-scope atomic).
// The workgroup that brings it to the task's split count resets it to zero (no other
// workgroup of the launch touches it afterwards, and the next launch on the stream starts
// after this one ends) and reads the other splits' rows with device-coherent loads. No
// workgroup waits for another, and no whole-L2 write-back or invalidate is needed. Calls that
// overlap on one device with the same counters race.
#pragma once

#include "attention.h"
#include "dma.h"
#include "post.h"

namespace oscar {

struct FinishArgs {
  PostArgs p;           // p.hp / p.hl are the launch's partials / LSEs, p.splits its splits
  int32_t* counters;    // [programs][kv heads]
  int32_t programs;     // grid x of the launch
};

// Called by every thread of a split workgroup once its partial rows are written (with
// store_coherent): true in the workgroup that completes the (task, head); the other splits'
// rows are then readable with load_coherent.
__device__ __forceinline__ bool finish_arrive(int32_t* counter, int nsplit, int* s_flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores are done
  __syncthreads();
  if (threadIdx.x == 0) {
    const int done = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = done == nsplit - 1 ? 1 : 0;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_flag) != 0;
}

// LDS of the finisher, inside the history kernel's ring (free once its token loop is done):
// R_v column tiles 2 and 3 of each wavefront ([wave][tile][k-step][lane] x 16 bytes, by DMA),
// the merged rows (8 x 256 bf16), the output rows (8 x 256 bf16) and the merged rows' LSEs.
constexpr int kFinishRvBytes = 4 * 2 * 8 * 64 * 16;
constexpr int kFinishRowBytes = 8 * kHeadDim * 2;
constexpr int kFinishLdsBytes = kFinishRvBytes + 2 * kFinishRowBytes + 8 * 4;

// The task's query rows r < 8 (row_info order) by the completing workgroup, with the row
// arithmetic of post_attention (split merge in split order, bf16 rounding, inverse V rotation,
// path merge). Every load is issued in one round, because a round trip at the end of the
// launch costs several microseconds: lane l of wavefront w merges row l / 8, dims 64 w +
// 8 (l % 8) .. + 7, over the task's `nsplit` splits (device-coherent reads), while R_v column
// tiles 2 and 3 arrive in LDS by DMA and tiles 0 and 1 and the BF16-branch rows in registers.
// The output rows are staged in LDS and stored 16 bytes per thread.
__device__ __forceinline__ void finish_task8(const FinishArgs& f, const AttnArgs& a, const Task& t,
                                             int head, int nsplit, uint8_t* lds) {
  const PostArgs& p = f.p;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  // Task rows are below the token count by construction (row_info bounds the query span by
  // counts[1]); the count is not reloaded, so that no compiler wait for it also drains the
  // R_v DMA below (the compiler does not count asm loads).
  constexpr int active = 0x7fffffff;
  const int task_rows = a.qt * a.g;
  auto row_of = [&](int r) -> int64_t {
    if (r >= task_rows) return -1;
    const RowInfo ri = row_info(a, t, head, r);
    return ri.valid ? ri.token * a.hq + ri.qhead : -1;
  };
  auto* s_h = reinterpret_cast<uint16_t(*)[kHeadDim]>(lds + kFinishRvBytes);
  auto* s_out = reinterpret_cast<uint16_t(*)[kHeadDim]>(lds + kFinishRvBytes + kFinishRowBytes);
  float* s_l = reinterpret_cast<float*>(lds + kFinishRvBytes + 2 * kFinishRowBytes);
  // R_v tiles 2, 3 of this wavefront: lane (n, g) k-step m holds R_v[64 w + 16 ct + n][32 m +
  // 8 g .. + 7], the B operand rotate_load_b would load.
  const uint32_t rv_lds = lds_addr(lds) + wave * 2 * 8 * 64 * 16;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int m = 0; m < 8; ++m)
      dma_dwordx4(p.rv + static_cast<int64_t>(64 * wave + 16 * (c + 2) + n) * kHeadDim + 32 * m +
                      8 * g,
                  rv_lds + (c * 8 + m) * 64 * 16);
  u32x4 rb[2][8];
  {
    RotateOperands op;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      rotate_load_b<true>(op, p.rv + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1,
                          g);
#pragma unroll
      for (int k = 0; k < 8; ++k) rb[ct][k] = op.b[k];
    }
  }
  PathRows pr;
  load_path_rows<8>(p, row_of, active, pr);
  // ---- merge (merge_splits_row arithmetic, 8 dims per lane)
  const int r = lane >> 3, d0 = 64 * wave + 8 * (lane & 7);
  const int64_t row = row_of(r);
  const bool live = row >= 0 && row / p.hq < active;
  const int end = live ? min(nsplit, 16) : 0;  // splits at or past `end` are not used
  // One resource per buffer (the host keeps both below 4 GiB); slot (row, split) is split row
  // row * splits + split. Slots past `end` may hold another launch's values: they are loaded
  // (inside the buffer) but never used.
  const auto part = coherent_rsrc(p.hp, static_cast<uint32_t>(p.rows * p.splits * kHeadDim * 4));
  const auto lses = coherent_rsrc(p.hl, static_cast<uint32_t>(p.rows * p.splits * 4));
  const uint32_t slot0 = static_cast<uint32_t>((row >= 0 ? row : 0) * p.splits);
  // The row's 16 LSEs live two per lane across its 8 lanes (split j and 8 + j in lane j of the
  // group) and are fetched by lane shuffles where the merge needs them, so that only the
  // partial values occupy registers while the loads are in flight.
  const float lse_lo = load_coherent(lses, (slot0 + (lane & 7)) * 4);
  const float lse_hi = load_coherent(lses, (slot0 + 8 + (lane & 7)) * 4);
  float4 v[16][2];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t at = ((slot0 + k) * kHeadDim + d0) * 4;
    v[k][0] = load_coherent4(part, at);
    v[k][1] = load_coherent4(part, at + 16);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the merge starts
  const int group = lane & ~7;
  auto lse_of = [&](int k) {
    const float x = __shfl(k < 8 ? lse_lo : lse_hi, group + (k & 7), kWave);
    return k < end ? x : -INFINITY;
  };
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) mx = fmaxf(mx, lse_of(k));
  const float safe = mx == -INFINITY ? 0.f : mx;
  float den = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float lk = lse_of(k);
    if (lk == -INFINITY) continue;  // zero weight: that split's row is never used
    const float w = expf(lk - safe);
    den += w;
    const float x[8] = {v[k][0].x, v[k][0].y, v[k][0].z, v[k][0].w,
                        v[k][1].x, v[k][1].y, v[k][1].z, v[k][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, x[i], acc[i]);
  }
  SplitMerge m0, m1;  // the lane's two groups of four dims, as merge_splits_out takes them
  m0.den = m1.den = den;
  m0.mx = m1.mx = mx;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m0.acc[i] = acc[i];
    m1.acc[i] = acc[4 + i];
  }
  *reinterpret_cast<uint2*>(&s_h[r][d0]) = merge_splits_out(m0);
  *reinterpret_cast<uint2*>(&s_h[r][d0 + 4]) = merge_splits_out(m1);
  if (wave == 0 && (lane & 7) == 0) s_l[r] = merge_splits_lse(m0);
  OSCAR_WAIT_VM(0);  // the R_v DMA of this wavefront
  __syncthreads();
  // ---- the rotation and path merge of post_attention, output rows through LDS
  const uint8_t* rv_tiles = lds + wave * 2 * 8 * 64 * 16;
  rotate_merge<8>(
      p, pr,
      [&](int ct, u32x4(&b)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          b[k] = ct < 2 ? rb[ct][k]
                        : *reinterpret_cast<const u32x4*>(rv_tiles + ((ct - 2) * 8 + k) * 64 * 16 +
                                                          lane * 16);
      },
      s_h, s_l, [&](int tr, int64_t, int col, uint16_t bits) { s_out[tr][col] = bits; });
  __syncthreads();
  {
    const int orow = threadIdx.x >> 5, c0 = 8 * (threadIdx.x & 31);
    const int64_t out_row = row_of(orow);
    if (out_row >= 0)
      *reinterpret_cast<uint4*>(p.out + out_row * kHeadDim + c0) =
          *reinterpret_cast<const uint4*>(&s_out[orow][c0]);
  }
}

// Workgroup (x, head) of the extra slice: the window store of request x (as the
// post-attention launch does; both branches have read the window before this launch, and the
// history branch never reads it), and, for head 0, rows of tokens x, x + programs, ... at or
// past the token count (zero output, LSE -inf: the path merge of two empty branches).
__device__ __forceinline__ void finish_extra(const FinishArgs& f, int head) {
  const int x = blockIdx.x;
  if (x < f.p.win_requests) store_window_request(f.p.win, x, head);
  if (head != 0) return;
  const int active = f.p.counts[1];
  const int64_t tokens = f.p.rows / f.p.hq;
  for (int64_t tok = x; tok < tokens; tok += f.programs) {
    if (tok < active) continue;
    uint16_t* out = f.p.out + tok * f.p.hq * kHeadDim;
    for (int e = threadIdx.x; e < f.p.hq * kHeadDim; e += kThreads) out[e] = 0;
    if (f.p.merged_lse && threadIdx.x < f.p.hq) f.p.merged_lse[tok * f.p.hq + threadIdx.x] = -INFINITY;
  }
}

// Two-launch step, history side (history.hip): grid (programs, kv heads, splits + 1), query
// rows per task <= 8, splits <= 16 (one-round split merge).
hipError_t launch_history_finish(const AttnArgs& a, const FinishArgs& f, hipStream_t stream);

}  // namespace oscar
