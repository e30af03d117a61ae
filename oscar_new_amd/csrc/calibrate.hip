// Calibration math of the K/V rotations on the GPU: streamed Gram (covariance) sums, the
// attention weights of the V covariance, normalization, a batched cyclic Jacobi
// eigensolver, and the rotation R = U H Pbr.
//
// Reference: oscar_ascend/calibration_kernels.py (accumulate_gram 14-70, sst_weights 73-126,
// normalize 129-156, the Jacobi sweeps 159-267, the U H Pbr composition 270-284, the driver
// calibrated_rotations 287-327). Startup-only work, off the decode path.
//
// The eigensolver keeps the upper triangle of one symmetric 256 x 256 matrix in LDS
// (32896 floats = 128.5 KiB of the CU's 160 KiB) and runs every sweep of that matrix in one
// workgroup of 1024 threads: a round computes the 128 disjoint plane rotations of the
// round-robin schedule (pair k of round r is (255, r) for k = 0 and ((r + k) mod 255,
// (r - k) mod 255) otherwise), then updates each 2 x 2 block {p_k, q_k} x {p_l, q_l}
// (k <= l) as J_k^T A J_l in place: the reference's column pass followed by its row pass,
// with the same arithmetic per element. Convergence (max |off-diagonal| / max |diagonal|)
// is checked on the device every second sweep and after the last, so a matrix stops on its
// own with no host round trip. Each round's (cos, sin) pairs are logged; a second kernel
// applies the logged rounds to the rows of U = I (rows are independent under right
// multiplication by the rotations), and a third sorts the eigenpairs ascending and composes
// R row by row (Walsh-Hadamard butterflies, 1/16, bit-reversed columns).
#include "common.h"

namespace oscar {
namespace {

constexpr int kD = 256;
constexpr int kPairs = kD / 2;
constexpr int kRoundsPerSweep = kD - 1;
constexpr int kTri = kD * (kD + 1) / 2;
constexpr int kJacobiThreads = 1024;
constexpr int kMaxSweeps = 64;

// ------------------------------------------------------------------ Gram sums

// C[i][j] += sum_r w_r x_r[i] x_r[j] over rows r = (token, head) of x, fp32 MFMA 16x16x4.
// One workgroup per 32 x 32 tile of C; its four wavefronts take every fourth 4-row k-step
// and their partial tiles are added in wavefront order (deterministic).
struct GramArgs {
  const void* x;
  int64_t rows, heads, s_t, s_h, s_d;
  const float* weights;  // nullptr: unweighted
  float* cov;
  int32_t dim, fp32;
};

__device__ __forceinline__ float gram_load(const GramArgs& a, int64_t r, int col) {
  if (r >= a.rows) return 0.f;
  const int64_t off = (r / a.heads) * a.s_t + (r % a.heads) * a.s_h + col * a.s_d;
  return a.fp32 ? static_cast<const float*>(a.x)[off]
                : bf16_to_float(static_cast<const uint16_t*>(a.x)[off]);
}

__global__ __launch_bounds__(kThreads) void gram_kernel(const GramArgs a) {
  __shared__ float part[4][32][33];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int i0 = blockIdx.x * 32, j0 = blockIdx.y * 32;
  f32x4 acc[2][2] = {};
  for (int64_t k0 = 4 * static_cast<int64_t>(wave); k0 < a.rows; k0 += 16) {
    const int64_t r = k0 + g;
    // A = x^T (row i, k = token row), B = w x (k, col j): lane (n, g) holds A[n][g], B[g][n].
    const float w = (a.weights && r < a.rows) ? a.weights[r] : 1.f;
    float av[2], bv[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      av[t] = gram_load(a, r, i0 + 16 * t + n);
      bv[t] = gram_load(a, r, j0 + 16 * t + n) * w;
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
        acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[ti], bv[tj], acc[ti][tj], 0, 0, 0);
  }
  // D element (row 4g + v, column n) of each 16 x 16 block.
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wave][16 * ti + 4 * g + v][16 * tj + n] = acc[ti][tj][v];
  __syncthreads();
  for (int e = threadIdx.x; e < 32 * 32; e += kThreads) {
    const int i = e >> 5, j = e & 31;
    const float sum = ((part[0][i][j] + part[1][i][j]) + part[2][i][j]) + part[3][i][j];
    float* c = a.cov + static_cast<int64_t>(i0 + i) * a.dim + (j0 + j);
    *c = *c + sum;
  }
}

// ------------------------------------------------------------------ attention weights

// w_t = max(k_t^T C_q k_t, 0) for 8 key rows per workgroup (thread j forms (k_t^T C_q)[j]).
struct SstArgs {
  const void* key;
  int64_t n, s_t, s_d;
  const float* qcov;
  float* weights;
  int32_t fp32;
};

constexpr int kSstRows = 8;

__global__ __launch_bounds__(kThreads) void sst_weights_kernel(const SstArgs a) {
  __shared__ float kv[kSstRows][kD];
  __shared__ float red[kSstRows][4];
  const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kSstRows;
#pragma unroll
  for (int t = 0; t < kSstRows; ++t) {
    float v = 0.f;
    if (t0 + t < a.n) {
      const int64_t off = (t0 + t) * a.s_t + j * a.s_d;
      v = a.fp32 ? static_cast<const float*>(a.key)[off]
                 : bf16_to_float(static_cast<const uint16_t*>(a.key)[off]);
    }
    kv[t][j] = v;
  }
  __syncthreads();
  float acc[kSstRows] = {};
  for (int i = 0; i < kD; ++i) {
    const float c = a.qcov[i * kD + j];
#pragma unroll
    for (int t = 0; t < kSstRows; ++t) acc[t] += kv[t][i] * c;
  }
#pragma unroll
  for (int t = 0; t < kSstRows; ++t) {
    float s = kv[t][j] * acc[t];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (lane == 0) red[t][wave] = s;
  }
  __syncthreads();
  if (j < kSstRows && t0 + j < a.n) {
    const float s = (red[j][0] + red[j][1]) + (red[j][2] + red[j][3]);
    a.weights[t0 + j] = fmaxf(s, 0.f);
  }
}

// *total += sum of n weights (one workgroup, fixed order).
__global__ __launch_bounds__(kThreads) void sum_kernel(const float* w, int64_t n, float* total) {
  __shared__ float red[4];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kThreads) s += w[i];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) *total = *total + ((red[0] + red[1]) + (red[2] + red[3]));
}

// out = x / max(denominator, 1e-30); the denominator is *den (device) or `value`.
__global__ __launch_bounds__(kThreads) void divide_kernel(const float* x, int64_t count,
                                                          const float* den, float value,
                                                          float* out) {
  const float d = fmaxf(den ? *den : value, 1.0e-30f);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    out[i] = x[i] / d;
}

// ------------------------------------------------------------------ Jacobi eigensolver

__device__ __forceinline__ int tri_at(int i, int j) {  // i <= j
  return i * kD - ((i * (i - 1)) >> 1) + (j - i);
}
__device__ __forceinline__ int tri_sym(int i, int j) { return i <= j ? tri_at(i, j) : tri_at(j, i); }

__device__ __forceinline__ void round_pair(int k, int r, int& p, int& q) {
  if (k == 0) {
    p = kD - 1;
    q = r;
  } else {
    p = (r + k) % (kD - 1);
    q = (r - k + kD - 1) % (kD - 1);
  }
}

struct JacobiArgs {
  const float* cov;  // [batch, 256, 256]
  float2* cs_log;    // [batch, max_sweeps * 255, 128]
  float* diag;       // [batch, 256] eigenvalues, unsorted
  int32_t* rounds;   // [batch] rounds logged
  float* info;       // [batch, 2]: sweeps, relative off-diagonal residual
  int32_t max_sweeps;
  float tol;
};

__device__ float block_max(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kJacobiThreads / kWave; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kJacobiThreads) void jacobi_kernel(const JacobiArgs a) {
  __shared__ float tri[kTri];
  __shared__ float cs[2 * kPairs];
  __shared__ float red[kJacobiThreads / kWave];
  const int tid = threadIdx.x, b = blockIdx.x;
  const float* c = a.cov + static_cast<int64_t>(b) * kD * kD;
  for (int f = tid; f < kD * kD; f += kJacobiThreads) {
    const int i = f >> 8, j = f & (kD - 1);
    if (i <= j) tri[tri_at(i, j)] = (c[f] + c[j * kD + i]) * 0.5f;
  }
  __syncthreads();
  float2* log = a.cs_log + static_cast<int64_t>(b) * a.max_sweeps * kRoundsPerSweep * kPairs;
  // Blocks (k, l), k <= l: rows k = grp and 127 - grp hold 129 blocks together, 16 threads
  // per row pair.
  const int grp = tid >> 4, sub = tid & 15;
  float residual = INFINITY;
  int sweep = 0;
  while (sweep < a.max_sweeps) {
    for (int r = 0; r < kRoundsPerSweep; ++r) {
      if (tid < kPairs) {
        int p, q;
        round_pair(tid, r, p, q);
        const float app = tri[tri_at(p, p)], aqq = tri[tri_at(q, q)], apq = tri[tri_sym(p, q)];
        const float delta = (aqq - app) * 0.5f;
        const float sign = delta >= 0.f ? 1.f : -1.f;
        float t = sign * apq / fmaxf(fabsf(delta) + sqrtf(delta * delta + apq * apq), 1e-30f);
        t = fabsf(apq) > 1e-8f * (fabsf(app) + fabsf(aqq)) + 1e-20f ? t : 0.f;
        const float cc = 1.f / sqrtf(1.f + t * t);
        const float ss = t * cc;
        cs[2 * tid] = cc;
        cs[2 * tid + 1] = ss;
        log[static_cast<int64_t>(sweep * kRoundsPerSweep + r) * kPairs + tid] = make_float2(cc, ss);
      }
      __syncthreads();
      for (int m = sub; m < kPairs + 1; m += 16) {
        int k, l;
        if (m < kPairs - grp) {
          k = grp;
          l = grp + m;
        } else {
          k = kPairs - 1 - grp;
          l = k + (m - (kPairs - grp));
        }
        int pk, qk, pl, ql;
        round_pair(k, r, pk, qk);
        round_pair(l, r, pl, ql);
        const float ck = cs[2 * k], sk = cs[2 * k + 1], cl = cs[2 * l], sl = cs[2 * l + 1];
        const int i1 = tri_sym(pk, pl), i2 = tri_sym(pk, ql), i3 = tri_sym(qk, pl),
                  i4 = tri_sym(qk, ql);
        const float xpp = tri[i1], xpq = tri[i2], xqp = tri[i3], xqq = tri[i4];
        // Column pass (A J_l), then row pass (J_k^T B).
        const float bpp = xpp * cl - xpq * sl, bpq = xpp * sl + xpq * cl;
        const float bqp = xqp * cl - xqq * sl, bqq = xqp * sl + xqq * cl;
        const float npp = ck * bpp - sk * bqp, npq = ck * bpq - sk * bqq;
        const float nqp = sk * bpp + ck * bqp, nqq = sk * bpq + ck * bqq;
        if (k == l) {  // i2 == i3: the off-diagonal element, stored once
          tri[i1] = npp;
          tri[i4] = nqq;
          tri[i2] = pk < qk ? npq : nqp;
        } else {
          tri[i1] = npp;
          tri[i2] = npq;
          tri[i3] = nqp;
          tri[i4] = nqq;
        }
      }
      __syncthreads();
    }
    ++sweep;
    if (sweep % 2 == 0 || sweep == a.max_sweeps) {
      float off = 0.f, dg = 0.f;
      bool bad = false;
      if (tid < kD) {
        const float x = tri[tri_at(tid, tid)];
        bad |= !isfinite(x);
        dg = fabsf(x);
      }
      const int i = tid >> 2;
      for (int j = i + 1 + (tid & 3); j < kD; j += 4) {
        const float x = tri[tri_at(i, j)];
        bad |= !isfinite(x);
        off = fmaxf(off, fabsf(x));
      }
      const float worst_off = block_max(bad ? INFINITY : off, red);
      const float worst_diag = block_max(dg, red);
      residual = isfinite(worst_off) ? worst_off / fmaxf(worst_diag, 1.0e-30f) : INFINITY;
      if (!(residual >= a.tol) || !isfinite(residual)) break;
    }
  }
  if (tid < kD) a.diag[b * kD + tid] = tri[tri_at(tid, tid)];
  if (tid == 0) {
    a.rounds[b] = sweep * kRoundsPerSweep;
    a.info[2 * b] = static_cast<float>(sweep);
    a.info[2 * b + 1] = residual;
  }
}

// U = I J_1 J_2 ... J_n from the logged rounds, one wavefront per row of U.
__global__ __launch_bounds__(kThreads) void apply_rounds_kernel(const float2* cs_log,
                                                                const int32_t* rounds,
                                                                int32_t max_sweeps, float* u) {
  __shared__ float rows[4][kD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y, row = blockIdx.x * 4 + wave;
  float* mine = rows[wave];
#pragma unroll
  for (int e = 0; e < 4; ++e) mine[4 * lane + e] = (4 * lane + e == row) ? 1.f : 0.f;
  __builtin_amdgcn_wave_barrier();
  const float2* log = cs_log + static_cast<int64_t>(b) * max_sweeps * kRoundsPerSweep * kPairs;
  const int n = rounds[b];
  float2 next0 = n > 0 ? log[lane] : make_float2(1.f, 0.f);
  float2 next1 = n > 0 ? log[lane + 64] : make_float2(1.f, 0.f);
  for (int rr = 0; rr < n; ++rr) {
    const float2 c0 = next0, c1 = next1;
    if (rr + 1 < n) {
      next0 = log[static_cast<int64_t>(rr + 1) * kPairs + lane];
      next1 = log[static_cast<int64_t>(rr + 1) * kPairs + lane + 64];
    }
    const int r = rr % kRoundsPerSweep;
    int p0, q0, p1, q1;
    round_pair(lane, r, p0, q0);
    round_pair(lane + 64, r, p1, q1);
    const float up0 = mine[p0], uq0 = mine[q0], up1 = mine[p1], uq1 = mine[q1];
    mine[p0] = up0 * c0.x - uq0 * c0.y;
    mine[q0] = up0 * c0.y + uq0 * c0.x;
    mine[p1] = up1 * c1.x - uq1 * c1.y;
    mine[q1] = up1 * c1.y + uq1 * c1.x;
    __builtin_amdgcn_wave_barrier();
  }
  float* out = u + (static_cast<int64_t>(b) * kD + row) * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[4 * lane + e] = mine[4 * lane + e];
}

__device__ __forceinline__ int bit_reverse8(int i) { return static_cast<int>(__brev(i) >> 24); }

// Eigenpairs sorted ascending (ties by index), then R[row][bitrev(255 - i)] = (u_row H)[i] / 16
// for the sorted row u_row; one wavefront per row, element i = 64 e + lane in register e.
__global__ __launch_bounds__(kThreads) void compose_kernel(const float* diag, const float* u,
                                                           float* eigenvalues, float* rotation) {
  __shared__ float ev[kD];
  __shared__ int rank[kD];
  __shared__ float rows[4][kD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.y, row = blockIdx.x * 4 + wave;
  const float v = diag[b * kD + tid];
  ev[tid] = v;
  __syncthreads();
  int cnt = 0;
  for (int o = 0; o < kD; ++o) {
    const float w = ev[o];
    cnt += (w < v) || (w == v && o < tid);
  }
  rank[tid] = cnt;
  if (blockIdx.x == 0) eigenvalues[b * kD + cnt] = v;
  __syncthreads();
  const float* src = u + (static_cast<int64_t>(b) * kD + row) * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) rows[wave][rank[4 * lane + e]] = src[4 * lane + e];
  __builtin_amdgcn_wave_barrier();
  float val[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) val[e] = rows[wave][64 * e + lane];
#pragma unroll
  for (int bit = 1; bit < 64; bit <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float partner = __shfl_xor(val[e], bit);
      val[e] = (lane & bit) == 0 ? val[e] + partner : partner - val[e];
    }
  }
#pragma unroll
  for (int eb = 1; eb < 4; eb <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e & eb) continue;
      const float lo = val[e], hi = val[e | eb];
      val[e] = lo + hi;
      val[e | eb] = lo - hi;
    }
  }
  float* out = rotation + (static_cast<int64_t>(b) * kD + row) * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[bit_reverse8(kD - 1 - (64 * e + lane))] = val[e] / 16.f;
}

}  // namespace
}  // namespace oscar

extern "C" int oscar_accumulate_gram(const void* x, int32_t x_fp32, int64_t n, int64_t heads,
                                     int64_t dim, int64_t s_t, int64_t s_h, int64_t s_d,
                                     const float* weights, float* covariance, void* stream) {
  using namespace oscar;
  if (n < 0 || heads <= 0 || dim <= 0) return OSCAR_E_SHAPE;
  if (dim % 32 || dim > 4096) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!x || !covariance) return OSCAR_E_NULL;
  const GramArgs a{x, n * heads, heads, s_t, s_h, s_d, weights, covariance,
                   static_cast<int32_t>(dim), x_fp32 ? 1 : 0};
  const unsigned tiles = static_cast<unsigned>(dim / 32);
  hipLaunchKernelGGL(gram_kernel, dim3(tiles, tiles), dim3(kThreads), 0, as_stream(stream), a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_sst_weights(const void* key, int32_t key_fp32, int64_t n, int64_t dim,
                                 int64_t s_t, int64_t s_d, const float* q_covariance,
                                 float* weights, float* total_weight, void* stream) {
  using namespace oscar;
  if (n < 0) return OSCAR_E_SHAPE;
  if (dim != kD) return OSCAR_E_UNSUPPORTED;
  if (n == 0) return OSCAR_OK;
  if (!key || !q_covariance || !weights || !total_weight) return OSCAR_E_NULL;
  const SstArgs a{key, n, s_t, s_d, q_covariance, weights, key_fp32 ? 1 : 0};
  hipLaunchKernelGGL(sst_weights_kernel, dim3(static_cast<unsigned>((n + kSstRows - 1) / kSstRows)),
                     dim3(kThreads), 0, as_stream(stream), a);
  hipLaunchKernelGGL(sum_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), weights, n,
                     total_weight);
  return static_cast<int>(hipGetLastError());
}

extern "C" int oscar_normalize(const float* x, int64_t count, const float* denominator,
                               float value, float* out, void* stream) {
  using namespace oscar;
  if (count < 0) return OSCAR_E_SHAPE;
  if (count == 0) return OSCAR_OK;
  if (!x || !out) return OSCAR_E_NULL;
  const int64_t blocks = (count + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(divide_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                     dim3(kThreads), 0, as_stream(stream), x, count, denominator, value, out);
  return static_cast<int>(hipGetLastError());
}

extern "C" int64_t oscar_calibration_workspace_bytes(int32_t batch, int32_t max_sweeps) {
  using namespace oscar;
  if (batch <= 0 || max_sweeps <= 0 || max_sweeps > kMaxSweeps) return -1;
  const int64_t log = static_cast<int64_t>(batch) * max_sweeps * kRoundsPerSweep * kPairs * 8;
  const int64_t u = static_cast<int64_t>(batch) * kD * kD * 4;
  const int64_t diag = static_cast<int64_t>(batch) * kD * 4;
  const int64_t rounds = ((static_cast<int64_t>(batch) * 4 + 255) / 256) * 256;
  return log + u + diag + rounds;
}

extern "C" int oscar_calibrated_rotations(const float* covariances, int32_t batch, int32_t dim,
                                          int32_t max_sweeps, float tolerance, void* workspace,
                                          int64_t workspace_bytes, float* rotations,
                                          float* eigenvalues, float* info, void* stream) {
  using namespace oscar;
  if (batch <= 0 || max_sweeps <= 0 || max_sweeps > kMaxSweeps) return OSCAR_E_SHAPE;
  if (dim != kD) return OSCAR_E_UNSUPPORTED;
  if (!covariances || !workspace || !rotations || !eigenvalues || !info) return OSCAR_E_NULL;
  if (workspace_bytes < oscar_calibration_workspace_bytes(batch, max_sweeps)) return OSCAR_E_SHAPE;
  if (reinterpret_cast<uintptr_t>(workspace) % 16) return OSCAR_E_ALIGN;
  char* ws = static_cast<char*>(workspace);
  float2* log = reinterpret_cast<float2*>(ws);
  ws += static_cast<int64_t>(batch) * max_sweeps * kRoundsPerSweep * kPairs * 8;
  float* u = reinterpret_cast<float*>(ws);
  ws += static_cast<int64_t>(batch) * kD * kD * 4;
  float* diag = reinterpret_cast<float*>(ws);
  ws += static_cast<int64_t>(batch) * kD * 4;
  int32_t* rounds = reinterpret_cast<int32_t*>(ws);
  const JacobiArgs a{covariances, log, diag, rounds, info, max_sweeps, tolerance};
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(jacobi_kernel, dim3(static_cast<unsigned>(batch)), dim3(kJacobiThreads), 0, s,
                     a);
  hipLaunchKernelGGL(apply_rounds_kernel, dim3(kD / 4, static_cast<unsigned>(batch)),
                     dim3(kThreads), 0, s, static_cast<const float2*>(log),
                     static_cast<const int32_t*>(rounds), max_sweeps, u);
  hipLaunchKernelGGL(compose_kernel, dim3(kD / 4, static_cast<unsigned>(batch)), dim3(kThreads), 0,
                     s, static_cast<const float*>(diag), static_cast<const float*>(u), eigenvalues,
                     rotations);
  return static_cast<int>(hipGetLastError());
}
