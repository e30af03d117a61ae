// One 16 x 16 output tile of x @ R on bf16 MFMA (v_mfma_f32_16x16x32_bf16), shared by the
// rotate entry point and the fused pre/post-attention kernels so that every path produces
// the same bits: the same operand layout and the same k order (eight k-steps of 32).
//
// Reference: oscar_ascend/kernels.py:14-48 (`_rotate_kernel`: bf16 operands, fp32
// accumulation, bf16 result).
#pragma once

#include "common.h"

namespace oscar {

// k-step m of lane (n, g): A = x[row n][32m + 8g .. +7], B = R[32m + 8g .. +7][col n].
struct RotateOperands {
  u32x4 a[8], b[8];
};

// A operand from a bf16 row (`row` = the lane's row start; nullptr = zero row). kVecX: the
// row is contiguous and 16-byte aligned; otherwise elements are xs2 apart.
template <bool kVecX>
__device__ __forceinline__ void rotate_load_a(RotateOperands& op, const uint16_t* row, int64_t xs2,
                                              int g) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int k0 = 32 * m + 8 * g;
    op.a[m] = u32x4{0u, 0u, 0u, 0u};
    if (row) {
      if (kVecX) {
        op.a[m] = *reinterpret_cast<const u32x4*>(row + k0);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          op.a[m][e] = static_cast<uint32_t>(row[(k0 + 2 * e) * xs2]) |
                       (static_cast<uint32_t>(row[(k0 + 2 * e + 1) * xs2]) << 16);
      }
    }
  }
}

// B operand from column `col` of R (`col` points at R[0][col]; elements rs0 apart). kColR:
// the column is contiguous (rs0 == 1) and 16-byte aligned.
template <bool kColR>
__device__ __forceinline__ void rotate_load_b(RotateOperands& op, const uint16_t* col, int64_t rs0,
                                              int g) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int k0 = 32 * m + 8 * g;
    const uint16_t* rp = col + static_cast<int64_t>(k0) * rs0;
    if (kColR) {
      op.b[m] = *reinterpret_cast<const u32x4*>(rp);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        op.b[m][e] = static_cast<uint32_t>(rp[(2 * e) * rs0]) |
                     (static_cast<uint32_t>(rp[(2 * e + 1) * rs0]) << 16);
    }
  }
}

// The tile: lane (n, g) receives rows 4g + v (v = 0..3) of column n, fp32.
__device__ __forceinline__ f32x4 rotate_mfma(const u32x4 (&a)[8], const u32x4 (&b)[8]) {
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 8; ++m) acc = mfma16x16x32(a[m], b[m], acc);
  return acc;
}
__device__ __forceinline__ f32x4 rotate_mfma(const RotateOperands& op) {
  return rotate_mfma(op.a, op.b);
}

}  // namespace oscar
