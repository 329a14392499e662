// mmm.hpp -- C++ layer over the C ABI (mmm.h) that keeps the reference's kernel-entry shape.
//
// The reference launches
//     WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J><<<grid, dim3(32, WAVES_I*WAVES_J)>>>(A, B, C)
// (and names the same GEMM WMMA_Templated_Base, WMMA_LDS_Padded, WMMA_LDS_Swizzled and GEMM_Naive,
// all provided below)
// with the sizes in the compile-time globals DIM_I/DIM_J/DIM_K (mmm.cpp:13-15, 1214-1215,
// 1461-1472, 1496), and the tensor variant with the packed G (mmmTensor.cpp:44-45, 345-371).
// Its template parameters fix the block tile: (WAVES_I*WAVE_M*16) x (WAVES_J*WAVE_N*16)
// outputs (mmm.cpp:706-716).  Here the same spelling takes the sizes at run time and keeps
// that meaning -- the block tile -- on the MI355X kernels: a block tile that one of the
// library's gfx950 instantiations provides is used as asked; any other falls back to the
// library's own tile choice (mmm_gemm_f16f32), which is also what WMMA_Auto does.
//
// The reference's launched parameters, <2,2,4,4>, name a 128x128 block (mmm.cpp:1462-1465), so
// this spelling runs the library's 128x128 tile: at 8192^3 on MI355X that tile measured 1031.0
// TFLOP/s against 1372.2 for the 256x256 tile the library picks itself (same box).  Call sites
// that do not need the reference's exact tile should use WMMA_Auto.
#ifndef MMM_HPP
#define MMM_HPP

#include "mmm.h"

#if defined(__FLT16_MANT_DIG__)
#include <type_traits>
#endif

namespace mmm {

// Row-major C[DIM_I][DIM_J] (fp32) = A[DIM_I][DIM_K] * B[DIM_K][DIM_J] (fp16), dense rows.
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J>
inline hipError_t WMMA_Swizzled_Full(const mmm_half* A, const mmm_half* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                     hipStream_t stream = nullptr) {
  constexpr int BLOCK_M = WAVES_I * WAVE_M * 16, BLOCK_N = WAVES_J * WAVE_N * 16;
  static_assert(BLOCK_M > 0 && BLOCK_N > 0, "tile parameters must be positive");
  // gfx950 instantiations (32x32 MFMA tiles per wave, 2x2 waves): block tile -> parameters
  constexpr int wm = BLOCK_M / 64, wn = BLOCK_N / 64;
  constexpr bool have = ((BLOCK_M == 128 || BLOCK_M == 256) && (BLOCK_N == 128 || BLOCK_N == 256)) ||
                        (BLOCK_M == 64 && BLOCK_N == 64) || (BLOCK_M == 192 && BLOCK_N == 192);
  if constexpr (have)
    return mmm_gemm_f16f32_tiled(A, B, C, DIM_I, DIM_J, DIM_K, DIM_K, DIM_J, DIM_J, wm, wn, 2, 2, nullptr, 0, stream);
  else
    return mmm_gemm_f16f32(A, B, C, DIM_I, DIM_J, DIM_K, DIM_K, DIM_J, DIM_J, stream);
}

// The reference's earlier kernels of the same lineage -- WMMA_Templated_Base (mmm.cpp:694-798),
// WMMA_LDS_Padded (mmm.cpp:821-1002) and WMMA_LDS_Swizzled (mmm.cpp:1018-1198) -- take the same
// template parameters and compute the same C as WMMA_Swizzled_Full; they differ from it only in
// how they lay out and read their LDS tiles on RDNA4 (padding, swizzles, hoisted address math).
// The MI355X kernels have their own layout, so these names run WMMA_Swizzled_Full's kernels, with
// the same reading of the parameters.
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J>
inline hipError_t WMMA_Templated_Base(const mmm_half* A, const mmm_half* B, float* C, int DIM_I, int DIM_J,
                                      int DIM_K, hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(A, B, C, DIM_I, DIM_J, DIM_K, stream);
}
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J>
inline hipError_t WMMA_LDS_Padded(const mmm_half* A, const mmm_half* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                  hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(A, B, C, DIM_I, DIM_J, DIM_K, stream);
}
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J>
inline hipError_t WMMA_LDS_Swizzled(const mmm_half* A, const mmm_half* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                    hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(A, B, C, DIM_I, DIM_J, DIM_K, stream);
}

// The reference's GEMM_Naive (mmm.cpp:52-62): one output per thread, its fp32 sum taken in
// ascending k, on the device (mmm_gemm_naive_f16f32, the same order bit for bit).
inline hipError_t GEMM_Naive(const mmm_half* A, const mmm_half* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                             hipStream_t stream = nullptr) {
  return mmm_gemm_naive_f16f32(A, B, C, DIM_I, DIM_J, DIM_K, DIM_K, DIM_J, DIM_J, stream);
}

// Library-chosen kernel (recommended: includes the M <= 64 streaming kernel).  With a workspace
// of mmm_gemm_workspace_f16f32's size, under-filled launches split K (mmm_gemm_f16f32_ws).
inline hipError_t WMMA_Auto(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                            int64_t ldb, int64_t ldc, hipStream_t stream = nullptr, void* workspace = nullptr,
                            size_t workspace_bytes = 0) {
  return mmm_gemm_f16f32_ws(A, B, C, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, stream);
}

// The reference's tensor program (mmmTensor.cpp): Out[m][b][r] = sum_{n,l} G[r][n][m][l] *
// Input[b][n][l], without the host pack of G (mmmTensor.cpp:329-343).
inline hipError_t WMMA_Tensor(const mmm_half* G, const mmm_half* Input, float* Out, int mt, int bt, int rt, int nt,
                              int rt_l, hipStream_t stream = nullptr) {
  mmm_contract_desc d;
  hipError_t e = mmm_contract_desc_reference(&d, mt, bt, rt, nt, rt_l);
  if (e != hipSuccess) return e;
  return mmm_contract5d_f16f32(&d, G, Input, Out, stream);
}

#if defined(__FLT16_MANT_DIG__)
// The reference's own pointer types: its call sites hold the operands as _Float16* (mmm.cpp:1446-1447,
// 1488, 1496; mmmTensor.cpp:44-45, 364, 369), so with a compiler that has _Float16 (hipcc, clang)
// those call sites compile unchanged.  Templates on the pointee, so that a literal nullptr still
// selects the mmm_half forms above without ambiguity.
template <class H>
using if_f16 = typename std::enable_if<std::is_same<typename std::remove_cv<H>::type, _Float16>::value, int>::type;
static_assert(sizeof(_Float16) == sizeof(mmm_half), "_Float16 is the binary16 bit pattern mmm_half holds");

template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J, class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_Swizzled_Full(HA* A, HB* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                     hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>((const mmm_half*)A, (const mmm_half*)B, C, DIM_I,
                                                              DIM_J, DIM_K, stream);
}

template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J, class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_Templated_Base(HA* A, HB* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                      hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>((const mmm_half*)A, (const mmm_half*)B, C, DIM_I,
                                                              DIM_J, DIM_K, stream);
}
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J, class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_LDS_Padded(HA* A, HB* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                  hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>((const mmm_half*)A, (const mmm_half*)B, C, DIM_I,
                                                              DIM_J, DIM_K, stream);
}
template <int WAVE_M, int WAVE_N, int WAVES_I, int WAVES_J, class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_LDS_Swizzled(HA* A, HB* B, float* C, int DIM_I, int DIM_J, int DIM_K,
                                    hipStream_t stream = nullptr) {
  return WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>((const mmm_half*)A, (const mmm_half*)B, C, DIM_I,
                                                              DIM_J, DIM_K, stream);
}

template <class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t GEMM_Naive(HA* A, HB* B, float* C, int DIM_I, int DIM_J, int DIM_K, hipStream_t stream = nullptr) {
  return GEMM_Naive((const mmm_half*)A, (const mmm_half*)B, C, DIM_I, DIM_J, DIM_K, stream);
}

template <class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_Auto(HA* A, HB* B, float* C, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                            hipStream_t stream = nullptr, void* workspace = nullptr, size_t workspace_bytes = 0) {
  return WMMA_Auto((const mmm_half*)A, (const mmm_half*)B, C, M, N, K, lda, ldb, ldc, stream, workspace,
                   workspace_bytes);
}

template <class HA, class HB, if_f16<HA> = 0, if_f16<HB> = 0>
inline hipError_t WMMA_Tensor(HA* G, HB* Input, float* Out, int mt, int bt, int rt, int nt, int rt_l,
                              hipStream_t stream = nullptr) {
  return WMMA_Tensor((const mmm_half*)G, (const mmm_half*)Input, Out, mt, bt, rt, nt, rt_l, stream);
}
#endif

}  // namespace mmm

#endif  // MMM_HPP
