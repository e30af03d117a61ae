// merge_splits / merge_paths: LSE-weighted combination of attention partials.
//
// Reference: oscar_ascend/kernels.py:485-541. One wavefront per (token, query head) row (one
// workgroup per row above 16 splits when rows are few, merge.h merge_mode); lane l owns dims
// 4l..4l+3. Every row is written, padded rows (token >= counts[1]) too,
// because the inverse rotation that follows reads them.
#include "merge.h"

namespace oscar {
namespace {

struct MergeSplitsArgs {
  const float* partials;
  const float* lse;
  const int32_t* counts;
  int64_t rows;
  int32_t hq, splits;
  uint16_t* out;
  float* logsum;
};

// One wavefront per row, four rows per workgroup (kMergeOneRound, kMergeScanWave).
template <int kMode>
__global__ __launch_bounds__(kThreads) void merge_splits_kernel(const MergeSplitsArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const bool valid = row / a.hq < a.counts[1];
  const float* part = a.partials + row * a.splits * kHeadDim;
  const float* ls = a.lse + row * a.splits;
  const SplitMerge r = kMode == kMergeOneRound
                           ? merge_splits_row(part, ls, a.splits, valid, lane)
                           : merge_splits_row_scan(part, ls, a.splits, valid, lane);
  *reinterpret_cast<uint2*>(a.out + row * kHeadDim + lane * 4) = merge_splits_out(r);
  if (lane == 0) a.logsum[row] = merge_splits_lse(r);
}

// One workgroup per row (kMergeScanGroup).
__global__ __launch_bounds__(kThreads) void merge_splits_group_kernel(const MergeSplitsArgs a) {
  __shared__ GroupMergeLds lds;
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x;
  const bool valid = row / a.hq < a.counts[1];
  const SplitMerge r = merge_splits_row_group(a.partials + row * a.splits * kHeadDim,
                                              a.lse + row * a.splits, a.splits, valid, &lds);
  if (threadIdx.x >= kWave) return;
  *reinterpret_cast<uint2*>(a.out + row * kHeadDim + lane * 4) = merge_splits_out(r);
  if (lane == 0) a.logsum[row] = merge_splits_lse(r);
}

struct MergePathsArgs {
  const uint16_t* a;
  const float* la;
  const float* b;
  const float* lb;
  const int32_t* counts;
  int64_t rows;
  int32_t hq;
  uint16_t* out;
  float* lse;
};

__global__ __launch_bounds__(kThreads) void merge_paths_kernel(const MergePathsArgs m) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= m.rows) return;
  const bool valid = row / m.hq < m.counts[1];
  const PathWeights w = path_weights(valid ? m.la[row] : -INFINITY, valid ? m.lb[row] : -INFINITY);
  float av[4] = {0.f, 0.f, 0.f, 0.f}, bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (valid) {
    const uint2 ar = *reinterpret_cast<const uint2*>(m.a + row * kHeadDim + lane * 4);
    av[0] = bf16_to_float(ar.x & 0xffffu);
    av[1] = bf16_to_float(ar.x >> 16);
    av[2] = bf16_to_float(ar.y & 0xffffu);
    av[3] = bf16_to_float(ar.y >> 16);
    const float4 br = *reinterpret_cast<const float4*>(m.b + row * kHeadDim + lane * 4);
    bv[0] = br.x;
    bv[1] = br.y;
    bv[2] = br.z;
    bv[3] = br.w;
  }
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = path_merge(w, av[i], bv[i]);
  *reinterpret_cast<uint2*>(m.out + row * kHeadDim + lane * 4) =
      make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
  if (m.lse && lane == 0) m.lse[row] = path_lse(w);
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_merge_splits(const float* partials, const float* lse, const int32_t* counts,
                                  int64_t n, int64_t hq, int32_t splits, int32_t d, void* out,
                                  float* logsum, void* stream) {
  using namespace oscar;
  if (n < 0 || hq <= 0 || splits <= 0) return OSCAR_E_SHAPE;
  if (d != kHeadDim) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!partials || !lse || !counts || !out || !logsum) return OSCAR_E_NULL;
  if (reinterpret_cast<uintptr_t>(partials) % 16 || reinterpret_cast<uintptr_t>(out) % 8)
    return OSCAR_E_ALIGN;
  MergeSplitsArgs a{partials, lse, counts, n * hq, static_cast<int32_t>(hq), splits,
                    static_cast<uint16_t*>(out), logsum};
  const dim3 four_rows(static_cast<unsigned>((a.rows + 3) / 4));
  switch (merge_mode(a.rows, splits)) {
    case kMergeOneRound:
      hipLaunchKernelGGL(merge_splits_kernel<kMergeOneRound>, four_rows, dim3(kThreads), 0,
                         as_stream(stream), a);
      break;
    case kMergeScanWave:
      hipLaunchKernelGGL(merge_splits_kernel<kMergeScanWave>, four_rows, dim3(kThreads), 0,
                         as_stream(stream), a);
      break;
    default:
      hipLaunchKernelGGL(merge_splits_group_kernel, dim3(static_cast<unsigned>(a.rows)),
                         dim3(kThreads), 0, as_stream(stream), a);
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_merge_paths(const void* history_out, const float* history_lse,
                                 const float* raw_partials, const float* raw_lse,
                                 const int32_t* counts, int64_t n, int64_t hq, int32_t d,
                                 void* output, float* merged_lse, void* stream) {
  using namespace oscar;
  if (n < 0 || hq <= 0) return OSCAR_E_SHAPE;
  if (d != kHeadDim) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!history_out || !history_lse || !raw_partials || !raw_lse || !counts || !output)
    return OSCAR_E_NULL;
  if (reinterpret_cast<uintptr_t>(history_out) % 8 || reinterpret_cast<uintptr_t>(output) % 8 ||
      reinterpret_cast<uintptr_t>(raw_partials) % 16)
    return OSCAR_E_ALIGN;
  MergePathsArgs m{static_cast<const uint16_t*>(history_out), history_lse, raw_partials, raw_lse,
                   counts, n * hq, static_cast<int32_t>(hq), static_cast<uint16_t*>(output),
                   merged_lse};
  hipLaunchKernelGGL(merge_paths_kernel, dim3(static_cast<unsigned>((m.rows + 3) / 4)),
                     dim3(kThreads), 0, as_stream(stream), m);
  return static_cast<int>(hipGetLastError());
}
