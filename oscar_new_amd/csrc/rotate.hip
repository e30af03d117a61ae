// rotate: out[t, h, :] = bf16(x[t, h, :] @ R) on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reference: oscar_ascend/kernels.py:14-66 (`_rotate_kernel`, `rotate`).
// Workgroup tile: 64 rows x 64 output columns; each wavefront owns 16 rows and the four
// 16-column MFMA tiles of the slice. The 256x64 slice of R is staged transposed in LDS
// (k contiguous) so both MFMA operands are 16-byte vector reads.
#include "common.h"

namespace oscar {
namespace {

constexpr int kRowsPerBlock = 64;
constexpr int kColsPerBlock = 64;
constexpr int kLdsPitch = kHeadDim + 8;  // bf16 elements per staged column (padding vs banks)

struct RotateArgs {
  const uint16_t* x;
  int64_t rows;  // n * h
  int64_t h, xs0, xs1, xs2;
  const uint16_t* r;
  int64_t rs0, rs1;
  uint16_t* out;
};

template <bool kVecX>
__global__ __launch_bounds__(kThreads) void rotate_kernel(const RotateArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t rt[kColsPerBlock * kLdsPitch];
  const int c0 = blockIdx.y * kColsPerBlock;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock;

  // Stage R[:, c0:c0+64] as rt[j][k]; read along whichever axis of R is contiguous.
  if (a.rs0 == 1) {
    for (int e = threadIdx.x; e < kColsPerBlock * kHeadDim; e += kThreads) {
      const int j = e >> 8, k = e & 255;
      rt[j * kLdsPitch + k] = a.r[k * a.rs0 + (c0 + j) * a.rs1];
    }
  } else {
    for (int e = threadIdx.x; e < kColsPerBlock * kHeadDim; e += kThreads) {
      const int k = e >> 6, j = e & 63;
      rt[j * kLdsPitch + k] = a.r[k * a.rs0 + (c0 + j) * a.rs1];
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t row = r0 + wave * 16 + col;
  const bool row_ok = row < a.rows;
  const int64_t token = row_ok ? row / a.h : 0;
  const int64_t head = row_ok ? row - token * a.h : 0;
  const uint16_t* xp = a.x + token * a.xs0 + head * a.xs1;

  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int k0 = m * 32 + grp * 8;
    u32x4 av = u32x4{0u, 0u, 0u, 0u};
    if (row_ok) {
      if (kVecX) {
        av = *reinterpret_cast<const u32x4*>(xp + k0);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = xp[(k0 + 2 * e) * a.xs2];
          const uint32_t hi = xp[(k0 + 2 * e + 1) * a.xs2];
          av[e] = lo | (hi << 16);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 bv = *reinterpret_cast<const u32x4*>(&rt[(t * 16 + col) * kLdsPitch + k0]);
      acc[t] = mfma16x16x32(av, bv, acc[t]);
    }
  }

  // C layout: lane holds rows 4*grp + v of the wavefront's 16, column `col` of each tile.
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t orow = r0 + wave * 16 + grp * 4 + v;
      if (orow < a.rows) {
        a.out[orow * kHeadDim + c0 + t * 16 + col] =
            static_cast<uint16_t>(float_to_bf16(acc[t][v]));
      }
    }
  }
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
  RotateArgs a{static_cast<const uint16_t*>(x), n * h, h, x_s0, x_s1, x_s2,
               static_cast<const uint16_t*>(rotation), r_s0, r_s1, static_cast<uint16_t*>(out)};
  const bool vec = x_s2 == 1 && (x_s0 % 8 == 0) && (x_s1 % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  dim3 grid(static_cast<unsigned>((a.rows + kRowsPerBlock - 1) / kRowsPerBlock),
            kHeadDim / kColsPerBlock);
  if (vec)
    hipLaunchKernelGGL(rotate_kernel<true>, grid, dim3(kThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(rotate_kernel<false>, grid, dim3(kThreads), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}
