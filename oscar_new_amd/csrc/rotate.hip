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
// From 1024 rows on (a prefill, the store benchmark) rotate_tiled_kernel stages R once per
// workgroup in LDS instead, with the same operands and k order, so both give the same bits.
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

// ---- Large row counts (prefill, the store benchmark): R is staged once per workgroup.
// Workgroup: 4 wavefronts; R^T in LDS as 256 columns x 512 bytes, 16-byte piece p of column
// c at piece slot p ^ (c & 31) (the B reads of 16 lanes, 16 columns at one piece, then cover
// all banks once). The workgroup loops over 16-row blocks blockIdx.x, + gridDim.x, ...;
// wavefront w computes columns 64 w .. 64 w + 63 of a block with the operands, MFMA and k
// order of rotate_kernel (bit-identical results), and the block's output goes through LDS
// so that every lane stores 16 bytes.
constexpr int kTiledRt = kHeadDim * kHeadDim * 2;  // R^T image, 128 KiB
constexpr int64_t kTiledMinRows = 1024;             // below this, rotate_kernel

__device__ __forceinline__ int rt_piece_offset(int col, int piece) {
  return col * (kHeadDim * 2) + 16 * (piece ^ (col & 31));
}

// kVecX: as rotate_kernel. kColR: R columns contiguous (rs0 == 1, 16-byte aligned); otherwise
// R rows are contiguous (rs1 == 1, 16-byte aligned) and are transposed in registers.
template <bool kVecX, bool kColR>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void rotate_tiled_kernel(const RotateArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_rt[kTiledRt];
  __shared__ __attribute__((aligned(16))) uint16_t s_out[16 * kHeadDim];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  // Every load of R is issued before the first LDS write (one memory round trip).
  u32x4 in[32];
  if (kColR) {
    // 8192 pieces: thread tid loads pieces tid, tid + 256, ... (32 per column).
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int item = i * kWavesPerBlock * kWave + tid;
      in[i] = *reinterpret_cast<const u32x4*>(a.r + static_cast<int64_t>(item >> 5) * a.rs1 +
                                              8 * (item & 31));
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int item = i * kWavesPerBlock * kWave + tid;
      *reinterpret_cast<u32x4*>(s_rt + rt_piece_offset(item >> 5, item & 31)) = in[i];
    }
  } else {
    // 1024 blocks of 8 x 8 (k block kb: rows 8 kb.., column block cb: columns 8 cb..), 4 per
    // thread, transposed with v_perm.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int item = i * kWavesPerBlock * kWave + tid;
      const int kb = item >> 5, cb = item & 31;
#pragma unroll
      for (int r = 0; r < 8; ++r)
        in[8 * i + r] = *reinterpret_cast<const u32x4*>(
            a.r + static_cast<int64_t>(8 * kb + r) * a.rs0 + 8 * cb);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int item = i * kWavesPerBlock * kWave + tid;
      const int kb = item >> 5, cb = item & 31;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        u32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          out[e] = __builtin_amdgcn_perm(in[8 * i + 2 * e + 1][j >> 1], in[8 * i + 2 * e][j >> 1],
                                         sel);
        *reinterpret_cast<u32x4*>(s_rt + rt_piece_offset(8 * cb + j, kb)) = out;
      }
    }
  }
  __syncthreads();
  const int64_t nblk = (a.rows + 15) / 16;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t row = blk * 16 + n;
    const bool row_ok = row < a.rows;
    const uint32_t token = row_ok ? fastdiv(static_cast<uint32_t>(row), a.h_div) : 0u;
    const int64_t head = row_ok ? row - static_cast<int64_t>(token) * a.h : 0;
    RotateOperands op;
    rotate_load_a<kVecX>(op, row_ok ? a.x + static_cast<int64_t>(token) * a.xs0 + head * a.xs1
                                    : nullptr,
                         a.xs2, g);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int col = 64 * wave + 16 * ct + n;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        op.b[m] = *reinterpret_cast<const u32x4*>(s_rt + rt_piece_offset(col, 4 * m + g));
      const f32x4 acc = rotate_mfma(op);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        s_out[(4 * g + v) * kHeadDim + col] = static_cast<uint16_t>(float_to_bf16(acc[v]));
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int piece = q * kWavesPerBlock * kWave + tid;  // 512 pieces of 16 bytes
      const int r = piece >> 5, c = 8 * (piece & 31);
      const int64_t orow = blk * 16 + r;
      if (orow < a.rows)
        *reinterpret_cast<u32x4*>(a.out + orow * kHeadDim + c) =
            *reinterpret_cast<const u32x4*>(&s_out[r * kHeadDim + c]);
    }
    __syncthreads();
  }
}

template <bool kVecX>
void launch_tiled(const RotateArgs& a, bool col_r, hipStream_t s) {
  const int64_t nblk = (a.rows + 15) / 16;
  const dim3 grid(static_cast<unsigned>(nblk < 256 ? nblk : 256));
  if (col_r)
    hipLaunchKernelGGL((rotate_tiled_kernel<kVecX, true>), grid, dim3(kWavesPerBlock * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((rotate_tiled_kernel<kVecX, false>), grid, dim3(kWavesPerBlock * kWave), 0, s, a);
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
  const bool row_r = r_s1 == 1 && (r_s0 % 8 == 0) &&
                     (reinterpret_cast<uintptr_t>(rotation) % 16 == 0);
  if (a.rows >= kTiledMinRows && (col_r || row_r) &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    if (vec)
      launch_tiled<true>(a, col_r, s);
    else
      launch_tiled<false>(a, col_r, s);
    return static_cast<int>(hipGetLastError());
  }
  if (vec)
    launch<true>(a, col_r, grid, s);
  else
    launch<false>(a, col_r, grid, s);
  return static_cast<int>(hipGetLastError());
}
