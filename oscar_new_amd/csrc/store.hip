// store_int2: clip + INT2 quantize + pack rotated K/V rows into 160-byte paged slots;
// rotate_store_int2: the K/V rotation and the same store in one launch; unpack: the
// diagnostic dequant of packed slots.
//
// Reference: oscar_ascend/kernels.py:69-202 (`_clip_vec`, `_store_vec`, `_store_kernel`,
// `store_int2`) and kernels.py:205-219, 623-648 (`_load_vec`, `_unpack_kernel`).
// Numerics follow the reference test oracle (tests/oracle.py:6-21) bit for bit:
//   threshold  = torch.quantile(|x|, ratio): rank = f32(ratio)*255 (fp32),
//                a/b = ascending order statistics floor/ceil(rank), fma(w, b - a, a);
//   zero       = fp16(min x); scale = fp16(max((max - min) / 3, 2^-14));
//   code       = clamp(trunc((x - zero) / scale + 0.5), 0, 3)   (IEEE fp32, no contraction).
// One wavefront quantizes one 256-element vector; lane l owns elements 4l..4l+3, i.e.
// exactly packed byte l.
#include "quant.h"
#include "rotate.h"

#pragma clang fp contract(off)

namespace oscar {
namespace {

struct StoreArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t rows;  // n * H
  uint8_t* history;
  int64_t history_bytes;
  const int64_t* slots;
  const int32_t* counts;
  Layout L;
  int32_t mode;
  float k_ratio, v_ratio, k_factor, v_factor;
  FastDiv h_div;  // division by kv_heads (store_int2_kernel)
};

// Two rows per workgroup; wavefront 2r+0 handles K of row r, 2r+1 handles V.
__global__ __launch_bounds__(kThreads) void store_int2_kernel(const StoreArgs a) {
  // The row, its token, slot and byte offset are wavefront-uniform (scalar registers).
  const int lane = threadIdx.x & 63, wave = uniform(static_cast<int>(threadIdx.x >> 6));
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 2 + (wave >> 1);
  const int is_v = wave & 1;
  if (row >= a.rows) return;
  const uint32_t token = fastdiv(static_cast<uint32_t>(row), a.h_div);  // rows < 2^31
  const int head = static_cast<int>(row - static_cast<int64_t>(token) * a.L.kv_heads);
  // The row's values, the token count and the slot are requested together (every address is
  // in bounds for row < rows); the skips of kernels.py:168-169 and the buffer bound only
  // decide whether the bytes are written, so nothing waits for the slot before the values.
  const uint16_t* src = (is_v ? a.v : a.k) + row * kHeadDim + lane * 4;
  const uint2 raw = *reinterpret_cast<const uint2*>(src);
  const int64_t slot = a.slots[token];
  const bool live = static_cast<int64_t>(token) < a.counts[1] && slot >= 0;
  const int64_t base = live ? slot_offset(a.L, slot, head) : 0;
  const bool write = live && base + 2 * a.L.vector_bytes <= a.history_bytes;
  const float x[4] = {bf16_to_float(raw.x & 0xffffu), bf16_to_float(raw.x >> 16),
                      bf16_to_float(raw.y & 0xffffu), bf16_to_float(raw.y >> 16)};
  quantize_store(x, a.mode, is_v ? a.v_ratio : a.k_ratio, is_v ? a.v_factor : a.k_factor,
                 write ? a.history + base + is_v * a.L.vector_bytes : nullptr);
}

// ---- rotate_store_int2: the K/V rotation and the INT2 store of many tokens in one launch.
// Workgroup (32-row block x: two 16-row tiles, K or V by y) of 16 wavefronts: the block's rows
// are staged once in LDS (16-byte piece p of row r at slot p ^ r), wavefront w computes output
// columns 16 w .. 16 w + 15 of both tiles with the operands, MFMA and k order of rotate_kernel
// (B from the columns of R, i.e. rows of R^T, through L2, read once per 32 rows), the bf16
// block is kept in LDS, and wavefront w then clips, quantizes and stores rows w and w + 16 as
// store_int2_kernel does. The rotated rows never go to HBM.
struct RotateStoreArgs {
  const uint16_t* x[2];  // K, V: row (token, head) at token * s0 + head * s1, contiguous, 16-B aligned
  int64_t s0[2], s1[2];
  const uint16_t* rt[2];  // R_k^T, R_v^T: contiguous [256][256]
  FastDiv h_div;
  StoreArgs st;  // rows, history, slots, counts, layout and clip (st.k / st.v unused)
};

constexpr int kRsWaves = 16;

__device__ __forceinline__ int rs_piece(int row, int piece) { return row * kHeadDim + 8 * (piece ^ row); }

constexpr int kRsTiles = 2;  // 16-row tiles per workgroup

__global__ __launch_bounds__(kRsWaves * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void rotate_store_kernel(const RotateStoreArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kRsTiles * 16 * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t s_rot[kRsTiles * 16 * kHeadDim];
  const StoreArgs& st = a.st;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int is_v = blockIdx.y;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 16 * kRsTiles;
  const int h = st.L.kv_heads;
  int64_t slot[kRsTiles];
  int head[kRsTiles];
  bool live[kRsTiles];
#pragma unroll
  for (int t = 0; t < kRsTiles; ++t) {
    const int64_t row = r0 + 16 * t + wave;
    const bool in = row < st.rows;
    const uint32_t token = fastdiv(static_cast<uint32_t>(in ? row : 0), a.h_div);
    head[t] = static_cast<int>((in ? row : 0) - static_cast<int64_t>(token) * h);
    live[t] = in && static_cast<int64_t>(token) < st.counts[1];
    slot[t] = live[t] ? st.slots[token] : -1;
  }
  for (int idx = tid; idx < kRsTiles * 16 * 32; idx += kRsWaves * kWave) {
    const int rr = idx >> 5, piece = idx & 31;
    const int64_t xrow = r0 + rr;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (xrow < st.rows) {
      const uint32_t xt = fastdiv(static_cast<uint32_t>(xrow), a.h_div);
      const int64_t xh = xrow - static_cast<int64_t>(xt) * h;
      v = *reinterpret_cast<const u32x4*>(a.x[is_v] + static_cast<int64_t>(xt) * a.s0[is_v] +
                                          xh * a.s1[is_v] + 8 * piece);
    }
    *reinterpret_cast<u32x4*>(s_x + rs_piece(rr, piece)) = v;
  }
  RotateOperands op;
  rotate_load_b<true>(op, a.rt[is_v] + static_cast<int64_t>(16 * wave + n) * kHeadDim, 1, g);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kRsTiles; ++t) {
#pragma unroll
    for (int m = 0; m < 8; ++m)
      op.a[m] = *reinterpret_cast<const u32x4*>(s_x + rs_piece(16 * t + n, 4 * m + g));
    const f32x4 acc = rotate_mfma(op);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      s_rot[(16 * t + 4 * g + v) * kHeadDim + 16 * wave + n] =
          static_cast<uint16_t>(float_to_bf16(acc[v]));
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kRsTiles; ++t) {
    // Same skips as store_int2_kernel (kernels.py:168-169 and the buffer bound).
    const int64_t base = live[t] && slot[t] >= 0 ? slot_offset(st.L, slot[t], head[t]) : 0;
    const bool write = live[t] && slot[t] >= 0 && base + 2 * st.L.vector_bytes <= st.history_bytes;
    if (!write) continue;
    const uint2 raw = *reinterpret_cast<const uint2*>(s_rot + (16 * t + wave) * kHeadDim + lane * 4);
    const float x[4] = {bf16_to_float(raw.x & 0xffffu), bf16_to_float(raw.x >> 16),
                        bf16_to_float(raw.y & 0xffffu), bf16_to_float(raw.y >> 16)};
    quantize_store(x, st.mode, is_v ? st.v_ratio : st.k_ratio, is_v ? st.v_factor : st.k_factor,
                   st.history + base + is_v * st.L.vector_bytes);
  }
}

struct UnpackArgs {
  const uint8_t* history;
  int64_t history_bytes;
  const int64_t* slots;
  int64_t n;
  Layout L;
  uint16_t* k;
  uint16_t* v;
};

// One wavefront per (token, head, K|V) vector; lane l decodes packed byte l.
__global__ __launch_bounds__(kThreads) void unpack_kernel(const UnpackArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 2 + (wave >> 1);
  const int is_v = wave & 1;
  const int h = a.L.kv_heads;
  if (item >= a.n * h) return;
  const int64_t token = item / h;
  const int head = static_cast<int>(item - token * h);
  const int64_t slot = a.slots[token];
  uint32_t lo = 0, hi = 0;
  if (slot >= 0) {
    const int64_t base = slot_offset(a.L, slot, head) + is_v * a.L.vector_bytes;
    if (base + a.L.vector_bytes <= a.history_bytes) {
      const uint8_t* p = a.history + base;
      const uint32_t byte = p[lane];
      const uint32_t sz = *reinterpret_cast<const uint32_t*>(p + 64);
      const float scale = half_lo_to_float(sz), zero = half_hi_to_float(sz);
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        val[i] = static_cast<float>((byte >> (2 * i)) & 3u) * scale + zero;
      lo = pack_bf16x2(val[0], val[1]);
      hi = pack_bf16x2(val[2], val[3]);
    }
  }
  uint16_t* out = (is_v ? a.v : a.k) + item * kHeadDim + lane * 4;
  *reinterpret_cast<uint2*>(out) = make_uint2(lo, hi);
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_store_int2(const void* key_rot, const void* value_rot, int64_t n,
                                void* history, int64_t history_bytes, const int64_t* slots,
                                const int32_t* counts, const oscar_layout* layout,
                                const oscar_clip* clip, void* stream) {
  using namespace oscar;
  if (n < 0 || history_bytes < 0) return OSCAR_E_SHAPE;
  StoreArgs a{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  if (!clip) return OSCAR_E_NULL;
  if (clip->mode < OSCAR_CLIP_PERCENTILE || clip->mode > OSCAR_CLIP_SEARCH) return OSCAR_E_SHAPE;
  if (n == 0) return OSCAR_OK;
  if (!key_rot || !value_rot || !history || !slots || !counts) return OSCAR_E_NULL;
  if (reinterpret_cast<uintptr_t>(key_rot) % 8 || reinterpret_cast<uintptr_t>(value_rot) % 8 ||
      reinterpret_cast<uintptr_t>(history) % 4)
    return OSCAR_E_ALIGN;
  a.k = static_cast<const uint16_t*>(key_rot);
  a.v = static_cast<const uint16_t*>(value_rot);
  a.rows = n * a.L.kv_heads;
  if (a.rows > 0x7fffffffll) return OSCAR_E_SHAPE;
  a.h_div = make_fastdiv(static_cast<uint32_t>(a.L.kv_heads));
  a.history = static_cast<uint8_t*>(history);
  a.history_bytes = history_bytes;
  a.slots = slots;
  a.counts = counts;
  a.mode = clip->mode;
  a.k_ratio = clip->k_ratio;
  a.v_ratio = clip->v_ratio;
  a.k_factor = clip->k_factor;
  a.v_factor = clip->v_factor;
  const dim3 grid(static_cast<unsigned>((a.rows + 1) / 2));
  hipLaunchKernelGGL(store_int2_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_rotate_store_int2(const void* key, int64_t k_s0, int64_t k_s1,
                                       const void* value, int64_t v_s0, int64_t v_s1, int64_t n,
                                       const void* rk_t, const void* rv_t, void* history,
                                       int64_t history_bytes, const int64_t* slots,
                                       const int32_t* counts, const oscar_layout* layout,
                                       const oscar_clip* clip, void* stream) {
  using namespace oscar;
  if (n < 0 || history_bytes < 0) return OSCAR_E_SHAPE;
  RotateStoreArgs a{};
  StoreArgs& st = a.st;
  const int status = make_layout(layout, &st.L);
  if (status != OSCAR_OK) return status;
  if (!clip) return OSCAR_E_NULL;
  if (clip->mode < OSCAR_CLIP_PERCENTILE || clip->mode > OSCAR_CLIP_SEARCH) return OSCAR_E_SHAPE;
  if (n == 0) return OSCAR_OK;
  if (!key || !value || !rk_t || !rv_t || !history || !slots || !counts) return OSCAR_E_NULL;
  if (n * st.L.kv_heads > 0x7fffffffll) return OSCAR_E_SHAPE;
  auto aligned16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!aligned16(key) || !aligned16(value) || !aligned16(rk_t) || !aligned16(rv_t) ||
      k_s0 % 8 || k_s1 % 8 || v_s0 % 8 || v_s1 % 8 || reinterpret_cast<uintptr_t>(history) % 4)
    return OSCAR_E_ALIGN;
  a.x[0] = static_cast<const uint16_t*>(key);
  a.x[1] = static_cast<const uint16_t*>(value);
  a.s0[0] = k_s0;
  a.s1[0] = k_s1;
  a.s0[1] = v_s0;
  a.s1[1] = v_s1;
  a.rt[0] = static_cast<const uint16_t*>(rk_t);
  a.rt[1] = static_cast<const uint16_t*>(rv_t);
  a.h_div = make_fastdiv(static_cast<uint32_t>(st.L.kv_heads));
  st.rows = n * st.L.kv_heads;
  st.history = static_cast<uint8_t*>(history);
  st.history_bytes = history_bytes;
  st.slots = slots;
  st.counts = counts;
  st.mode = clip->mode;
  st.k_ratio = clip->k_ratio;
  st.v_ratio = clip->v_ratio;
  st.k_factor = clip->k_factor;
  st.v_factor = clip->v_factor;
  const dim3 grid(static_cast<unsigned>((st.rows + 16 * kRsTiles - 1) / (16 * kRsTiles)), 2);
  hipLaunchKernelGGL(rotate_store_kernel, grid, dim3(kRsWaves * kWave), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_unpack(const void* history, int64_t history_bytes, const int64_t* slots,
                            int64_t n, const oscar_layout* layout, void* key_out,
                            void* value_out, void* stream) {
  using namespace oscar;
  if (n < 0 || n > 4096) return OSCAR_E_SHAPE;
  UnpackArgs a{};
  const int st = make_layout(layout, &a.L);
  if (st != OSCAR_OK) return st;
  if (n == 0) return OSCAR_OK;
  if (!history || !slots || !key_out || !value_out) return OSCAR_E_NULL;
  if (reinterpret_cast<uintptr_t>(key_out) % 8 || reinterpret_cast<uintptr_t>(value_out) % 8 ||
      reinterpret_cast<uintptr_t>(history) % 4)
    return OSCAR_E_ALIGN;
  a.history = static_cast<const uint8_t*>(history);
  a.history_bytes = history_bytes;
  a.slots = slots;
  a.n = n;
  a.k = static_cast<uint16_t*>(key_out);
  a.v = static_cast<uint16_t*>(value_out);
  const dim3 grid(static_cast<unsigned>((n * a.L.kv_heads + 1) / 2));
  hipLaunchKernelGGL(unpack_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}
