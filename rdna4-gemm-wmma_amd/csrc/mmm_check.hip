// On-device cross-check kernels (SIMT, no matrix cores).
//
//  * fp32 mode: the reference's GEMM_Naive (mmm.cpp:52-62) -- one fp32 accumulator per output,
//    k ascending, acc += float(a) * float(b).  The product of two fp16 values is exact in fp32,
//    so fused and unfused multiply-add round identically and the result is bit-reproducible
//    on the CPU with the same loop.
//  * fp64 mode: T = sum_k a*b and S = sum_k |a*b| in fp64, k ascending (products exact in
//    fp64).  T is the ground truth and S the scale of the tolerance |C - T| <= rel * S,
//    for every element of a full-size output instead of a sampled sub-grid.
//
// Both take any two-level fold per axis (a plain GEMM is the fold with high extents of 1), so
// they check the tensor contractions at their own layouts as well.  A 64x64 output tile per
// 256-thread block, 4x4 outputs per thread, K staged through LDS 32 deep; the order of the
// additions per output is the plain ascending-k loop whatever the tiling.
#include <type_traits>

#include "mmm_kernels.h"

namespace mmm {
namespace {

constexpr int kNB = 64;  // output tile edge
constexpr int kNK = 32;  // K depth per LDS stage

__device__ __forceinline__ int64_t fold_index(int x, int lo, const int64_t* s) {
  return (int64_t)(x / lo) * s[0] + (int64_t)(x % lo) * s[1];
}

__device__ __forceinline__ float h2f(mmm_half h) { return (float)__builtin_bit_cast(_Float16, h); }

template <bool F64>
__global__ __launch_bounds__(256) void check_fold_kernel(FoldProblem p, double* T, double* S, int tiles_n) {
  using Acc = typename std::conditional<F64, double, float>::type;
  __shared__ mmm_half As[kNK][kNB + 4];  // [k][m]
  __shared__ mmm_half Bs[kNK][kNB + 4];  // [k][n]
  const int t = threadIdx.x;
  const int m0 = (int)(blockIdx.x / tiles_n) * kNB, n0 = (int)(blockIdx.x % tiles_n) * kNB;

  // Staging: A with lanes along k (k-contiguous operands coalesce), B with lanes along n.
  const int a_k = t & 31, a_m = t >> 5;  // rows a_m + 8*i
  const int b_n = t & 63, b_k = t >> 6;  // k rows b_k + 4*i
  int64_t a_row[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + a_m + 8 * i;
    a_row[i] = m < p.M ? fold_index(m, p.m_lo, p.am) : -1;
  }
  const int gn = n0 + b_n;
  const int64_t b_col = gn < p.N ? fold_index(gn, p.n_lo, p.bn) : -1;

  const int tm = (t >> 4) * 4, tn = (t & 15) * 4;
  Acc acc[4][4], sab[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0, sab[i][j] = 0;

  for (int k0 = 0; k0 < p.K; k0 += kNK) {
    {
      const int k = k0 + a_k;
      const int64_t ko = k < p.K ? fold_index(k, p.k_lo, p.ak) : -1;
#pragma unroll
      for (int i = 0; i < 8; ++i) As[a_k][a_m + 8 * i] = (ko >= 0 && a_row[i] >= 0) ? p.A[a_row[i] + ko] : 0;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + b_k + 4 * i;
      Bs[b_k + 4 * i][b_n] = (k < p.K && b_col >= 0) ? p.B[fold_index(k, p.k_lo, p.bk) + b_col] : 0;
    }
    __syncthreads();
    const int kn = min(kNK, p.K - k0);
    for (int kk = 0; kk < kn; ++kk) {
      Acc a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = (Acc)h2f(As[kk][tm + i]), b[i] = (Acc)h2f(Bs[kk][tn + i]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const Acc ab = a[i] * b[j];
          acc[i][j] += ab;
          if constexpr (F64) sab[i][j] += ab < 0 ? -ab : ab;
        }
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + tm + i;
    if (m >= p.M) continue;
    const int64_t row = fold_index(m, p.m_lo, p.cm);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tn + j;
      if (n >= p.N) continue;
      const int64_t o = row + fold_index(n, p.n_lo, p.cn);
      if constexpr (F64) {
        T[o] = acc[i][j];
        if (S) S[o] = sab[i][j];
      } else {
        p.C[o] = acc[i][j];
      }
    }
  }
}

}  // namespace

hipError_t launch_check_fold(const FoldProblem& p, double* T, double* S, hipStream_t stream) {
  const int64_t tiles_m = (p.M + kNB - 1) / kNB, tiles_n = (p.N + kNB - 1) / kNB;
  if (tiles_m * tiles_n > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(tiles_m * tiles_n)), block(256);
  if (T)
    check_fold_kernel<true><<<grid, block, 0, stream>>>(p, T, S, (int)tiles_n);
  else
    check_fold_kernel<false><<<grid, block, 0, stream>>>(p, nullptr, nullptr, (int)tiles_n);
  return hipGetLastError();
}

}  // namespace mmm
