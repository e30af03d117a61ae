// Pre-attention pieces shared by the fused launches: the arguments of the BF16 branch, the q
// rotation and the K/V INT2 store of one step, the 16-row rotation tile, and the K/V store
// role. step.hip runs them as the pre-attention launch; history.hip can run the BF16 branch and
// the store as extra workgroups of the history launch.
#pragma once

#include "quant.h"
#include "raw.h"

namespace oscar {

struct PreArgs {
  AttnArgs attn;          // BF16 branch: unrotated query, key, value, window, metadata
  const uint16_t* rk_t;   // R_k^T, contiguous: rk_t[c][k] = R_k[k][c]
  const uint16_t* rv_t;   // R_v^T, contiguous
  uint16_t* qrot;         // [n, hq, 256]
  int64_t q_rows;         // n * hq
  int64_t kv_rows;        // n * H
  uint8_t* history;
  int64_t history_bytes;
  const int64_t* slots;
  int32_t mode;
  float k_ratio, v_ratio, k_factor, v_factor;
  FastDiv h_div, hq_div;    // division by H and by hq
  int32_t raw_wgs, kv_wgs;  // role boundaries in blockIdx.x
  // History launch with q rotation roles (qsync set): q_wgs 16-row tiles rotated into qrot
  // by role workgroups of the same launch; qsync[0] counts finished tiles, qsync[1] finished
  // workgroups, qsync[2] is set when a history workgroup gave up waiting (see q_rotate_role).
  int32_t* qsync;
  int32_t q_wgs;
};

// Rotation of rows [16 tile, +16) by R (given as R^T rows) into a [16][256] bf16 LDS tile
// (kv) or into `out` (q). Wavefront w computes columns 64w .. 64w + 63.
__device__ __forceinline__ void rotate_rows16(const uint16_t* x, int64_t xs0, int64_t xs1,
                                              FastDiv h_div, int64_t h, int64_t rows,
                                              int64_t tile, const uint16_t* rt, uint16_t* lds_tile,
                                              uint16_t* out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = tile * 16 + n;
  const uint16_t* xp = nullptr;
  if (row < rows) {
    const uint32_t token = fastdiv(static_cast<uint32_t>(row), h_div);
    xp = x + static_cast<int64_t>(token) * xs0 + (row - static_cast<int64_t>(token) * h) * xs1;
  }
  // Every operand (the A rows and the four column tiles of R) is requested before the first
  // MFMA: one round of memory latency.
  RotateOperands op;
  u32x4 rb[4][8];
  rotate_load_a<true>(op, xp, 1, g);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    rotate_load_b<true>(op, rt + static_cast<int64_t>(64 * wave + 16 * ct + n) * kHeadDim, 1, g);
#pragma unroll
    for (int m = 0; m < 8; ++m) rb[ct][m] = op.b[m];
  }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * wave + 16 * ct + n;
    const f32x4 acc = rotate_mfma(op.a, rb[ct]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * g + v;
      const uint16_t bits = static_cast<uint16_t>(float_to_bf16(acc[v]));
      if (lds_tile) {
        lds_tile[r * kHeadDim + col] = bits;
      } else if (tile * 16 + r < rows) {
        out[(tile * 16 + r) * kHeadDim + col] = bits;
      }
    }
  }
}

// K or V rows of quad r (K: r even, V: r odd): four workgroups share a 16-row rotation tile
// (each computes it) and each clips/quantizes/packs four of its rows, one per wavefront, into
// their slots. The row's token count and slot are requested before the rotation. `smem`:
// 16 x 256 bf16 of 16-byte aligned LDS.
__device__ __forceinline__ void kv_store_role(const PreArgs& p, int r, uint8_t* smem) {
  const AttnArgs& a = p.attn;
  const FastDiv h_div = p.h_div;
  const int is_v = r & 1;
  const int64_t quad = r >> 1, tile = quad >> 2;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rr = 4 * static_cast<int>(quad & 3) + wave;
  const int64_t row = tile * 16 + rr;
  const bool in = row < p.kv_rows;
  const uint32_t token = fastdiv(static_cast<uint32_t>(in ? row : 0), h_div);
  const int head = static_cast<int>((in ? row : 0) - static_cast<int64_t>(token) * a.L.kv_heads);
  const bool live = in && static_cast<int64_t>(token) < a.counts[1];
  const int64_t slot = live ? p.slots[token] : -1;  // in flight beside the rotation loads
  uint16_t* tile_lds = reinterpret_cast<uint16_t*>(smem);
  rotate_rows16(is_v ? a.value : a.key, is_v ? a.vs0 : a.ks0, is_v ? a.vs1 : a.ks1, h_div,
                a.L.kv_heads, p.kv_rows, tile, is_v ? p.rv_t : p.rk_t, tile_lds, nullptr);
  __syncthreads();
  // Same skips as store_int2 (kernels.py:168-169 and the buffer bound).
  if (!live || slot < 0) return;
  const int64_t base = slot_offset(a.L, slot, head);
  if (base + 2 * a.L.vector_bytes > p.history_bytes) return;
  const uint2 raw = *reinterpret_cast<const uint2*>(tile_lds + rr * kHeadDim + lane * 4);
  const float x[4] = {bf16_to_float(raw.x & 0xffffu), bf16_to_float(raw.x >> 16),
                      bf16_to_float(raw.y & 0xffffu), bf16_to_float(raw.y >> 16)};
  quantize_store(x, p.mode, is_v ? p.v_ratio : p.k_ratio, is_v ? p.v_factor : p.k_factor,
                 p.history + base + is_v * a.L.vector_bytes);
}

// q rotation role of the history launch (its history workgroups read the rotated rows):
// rotates 16-row tile `tile` into a bf16 LDS tile (the bits of rotate_rows16 and the rotate
// entry point), writes the live rows to qrot with device-coherent stores, waits for them, and
// then adds 1 to qsync[0]. Protocol (qsync zero between launches): a history workgroup waits
// until qsync[0] == q_wgs before it reads qrot with device-coherent loads; every workgroup of
// the launch adds 1 to qsync[1] as it ends (q_sync_leave), and the one that completes the
// grid resets both counters, when no workgroup of the launch reads them any more. The q roles
// sit in the leading z-slices, so they are dispatched before any history workgroup, and a
// waiting workgroup never holds a slot that a q role still needs. `smem`: 8 KiB of LDS.
__device__ __forceinline__ void q_rotate_role(const PreArgs& p, int64_t tile, uint8_t* smem) {
  const AttnArgs& a = p.attn;
  uint16_t* tile_lds = reinterpret_cast<uint16_t*>(smem);
  rotate_rows16(a.query, a.qs0, a.qs1, p.hq_div, a.hq, p.q_rows, tile, p.rk_t, tile_lds,
                nullptr);
  __syncthreads();
  const uint32_t* src = reinterpret_cast<const uint32_t*>(tile_lds);
  uint32_t* dst = reinterpret_cast<uint32_t*>(p.qrot + tile * 16 * kHeadDim);
  const int64_t live_words = (p.q_rows - tile * 16) * (kHeadDim / 2);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int w = static_cast<int>(threadIdx.x) + kThreads * i;  // 16 rows x 128 words
    if (w < live_words) __hip_atomic_store(dst + w, src[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's rows are at the device
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(p.qsync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// End of a workgroup of the launch (thread 0, after every wait of its workgroup): the
// workgroup that completes the grid resets the q counters for the next launch. The wait
// orders this workgroup's tile count (q roles) before its arrival here.
__device__ __forceinline__ void q_sync_leave(int32_t* qsync, int total) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const int done =
      __hip_atomic_fetch_add(qsync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (done == total - 1) {
    __hip_atomic_store(qsync, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(qsync + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Polls of qsync[0] before a history workgroup gives up (about a millisecond; the roles take
// a few microseconds). Giving up sets qsync[2] and the workgroup's rows are then wrong, never
// a hang.
constexpr int kQSyncPolls = 4096;

// The history launch with the pre-attention roles (history.hip): grid (programs, H,
// role_slices + splits); z-slice 0 runs the BF16 branch of (task, kv head) (lean form, one
// split), z-slices 1 .. role_slices - 1 the K/V store quads, the rest the history splits.
// rotate_query: a.query is the unrotated query and each history workgroup rotates its rows.
hipError_t launch_history_pre(const AttnArgs& a, const PreArgs& p, int role_slices, dim3 grid,
                              bool rotate_query, hipStream_t stream);

// Task rows of a four-wavefront history work queue (its task lists fit 80 KB of LDS with the
// unit's ring, two workgroups per CU).
constexpr int kQueueTasks4 = 512;

// The history launch of a step with 17-32 query rows per task (history.hip): the work queue of
// token-bounded history units (at most kQueueTasks4 task rows; `queue`: its two counters,
// zero at rest) with the BF16 branch (p.raw_wgs units of (task, kv head)) and the K/V store
// quads (p.kv_wgs) as units of the queue (the BF16 branch first, the K/V store last).
hipError_t launch_history_queue_pre(const AttnArgs& a, const PreArgs& p, int32_t* queue,
                                    int32_t programs, hipStream_t stream);

}  // namespace oscar
