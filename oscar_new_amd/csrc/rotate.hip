// rotate: out[t, h, :] = bf16(x[t, h, :] @ R) on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reference: oscar_ascend/kernels.py:14-66 (`_rotate_kernel`, `rotate`).
// The products here are small (a decode step rotates 32-200 rows), so the kernel is
// latency-bound: it maximizes parallelism instead of reuse. One wavefront computes one
// 16-row x 16-column output tile; both MFMA operands are read straight from global memory
// (every row of x and every column of R is re-read by the 16 tiles that need it, from L2),
// all 16 loads of a lane in flight at once. R is read column-wise: when its columns are
// contiguous (a transposed view of a row-major matrix, e.g. R^T for the inverse rotation
// or a cached transpose) each lane reads 16 bytes at a time, otherwise element by element.
#include "rotate.h"

namespace oscar {
namespace {

struct RotateArgs {
  const uint16_t* x;
  int64_t rows;  // n * h
  int64_t h, xs0, xs1, xs2;
  const uint16_t* r;
  int64_t rs0, rs1;
  uint16_t* out;
  FastDiv h_div;
};

constexpr int kWavesPerBlock = 4;  // four column tiles of one 16-row block

// kVecX: x rows contiguous and 16-byte aligned; kColR: R columns contiguous (rs0 == 1).
template <bool kVecX, bool kColR>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void rotate_kernel(const RotateArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + n;  // A row of this lane
  const int col = (blockIdx.y * kWavesPerBlock + wave) * 16 + n;  // B column of this lane
  const bool row_ok = row < a.rows;
  const uint32_t token = row_ok ? fastdiv(static_cast<uint32_t>(row), a.h_div) : 0u;
  const int64_t head = row_ok ? row - static_cast<int64_t>(token) * a.h : 0;
  const uint16_t* xp = a.x + static_cast<int64_t>(token) * a.xs0 + head * a.xs1;

  RotateOperands op;
  rotate_load_a<kVecX>(op, row_ok ? xp : nullptr, a.xs2, g);
  rotate_load_b<kColR>(op, a.r + static_cast<int64_t>(col) * a.rs1, a.rs0, g);
  const f32x4 acc = rotate_mfma(op);

  // C layout: lane (n, g) holds rows 4g + v of the tile, column n.
  const int ocol = (blockIdx.y * kWavesPerBlock + wave) * 16 + n;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t orow = static_cast<int64_t>(blockIdx.x) * 16 + 4 * g + v;
    if (orow < a.rows) a.out[orow * kHeadDim + ocol] = static_cast<uint16_t>(float_to_bf16(acc[v]));
  }
}

template <bool kVecX>
void launch(const RotateArgs& a, bool col_r, dim3 grid, hipStream_t s) {
  if (col_r)
    hipLaunchKernelGGL((rotate_kernel<kVecX, true>), grid, dim3(kWavesPerBlock * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((rotate_kernel<kVecX, false>), grid, dim3(kWavesPerBlock * kWave), 0, s, a);
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_rotate(const void* x, int64_t n, int64_t h, int64_t d, int64_t x_s0,
                            int64_t x_s1, int64_t x_s2, const void* rotation, int64_t r_s0,
                            int64_t r_s1, void* out, void* stream) {
  using namespace oscar;
  if (n < 0 || h <= 0) return OSCAR_E_SHAPE;
  if (d != kHeadDim) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!x || !rotation || !out) return OSCAR_E_NULL;
  if (n * h > 0x7fffffffll) return OSCAR_E_SHAPE;
  RotateArgs a{static_cast<const uint16_t*>(x), n * h, h, x_s0, x_s1, x_s2,
               static_cast<const uint16_t*>(rotation), r_s0, r_s1, static_cast<uint16_t*>(out),
               make_fastdiv(static_cast<uint32_t>(h))};
  const bool vec = x_s2 == 1 && (x_s0 % 8 == 0) && (x_s1 % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  const bool col_r = r_s0 == 1 && (r_s1 % 8 == 0) &&
                     (reinterpret_cast<uintptr_t>(rotation) % 16 == 0);
  const dim3 grid(static_cast<unsigned>((a.rows + 15) / 16), kHeadDim / (16 * kWavesPerBlock));
  hipStream_t s = as_stream(stream);
  if (vec)
    launch<true>(a, col_r, grid, s);
  else
    launch<false>(a, col_r, grid, s);
  return static_cast<int>(hipGetLastError());
}
