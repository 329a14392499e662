// hipBLASLt witness: the vendor GEMM on the same FP16 -> FP32 row-major problem, used only
// by bench.py and the tests as a comparison point (the reference compares against
// rocblas_gemm_ex the same way, mmm.cpp:1508-1534).  Not part of the product path.
//
// Row-major C[M][N] = A[M][K] * B[K][N] is computed as the column-major product
// C^T[N][M] = B^T[N][K] * A^T[K][M] (the operand swap of mmm.cpp:1519-1521).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdint.h>

namespace {

struct Plan {
  hipblasLtHandle_t handle = nullptr;
};

Plan& plan() {
  static thread_local Plan p;
  return p;
}

}  // namespace

extern "C" {

// Returns 0 on success, a hipblasStatus_t (+1000) or hipError_t otherwise.
int mmm_witness_hipblaslt_gemm(const void* A, const void* B, float* C, int M, int N, int K, int64_t lda,
                               int64_t ldb, int64_t ldc, void* workspace, size_t ws_bytes, hipStream_t stream) {
  Plan& p = plan();
  if (!p.handle && hipblasLtCreate(&p.handle) != HIPBLAS_STATUS_SUCCESS) return 1001;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  int rc = 0;
  hipblasOperation_t op = HIPBLAS_OP_N;
  hipblasLtMatmulHeuristicResult_t heur[1];
  int found = 0;
  const float alpha = 1.0f, beta = 0.0f;
#define WCHK(x)                                     \
  do {                                              \
    hipblasStatus_t s_ = (x);                       \
    if (s_ != HIPBLAS_STATUS_SUCCESS) {             \
      rc = 1000 + (int)s_;                          \
      goto done;                                    \
    }                                               \
  } while (0)
  WCHK(hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  WCHK(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op)));
  WCHK(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op)));
  // column-major: "A" = B^T (N x K, ld ldb), "B" = A^T (K x M, ld lda), "C" = C^T (N x M, ld ldc)
  WCHK(hipblasLtMatrixLayoutCreate(&la, HIP_R_16F, N, K, ldb));
  WCHK(hipblasLtMatrixLayoutCreate(&lb, HIP_R_16F, K, M, lda));
  WCHK(hipblasLtMatrixLayoutCreate(&lc, HIP_R_32F, N, M, ldc));
  WCHK(hipblasLtMatmulPreferenceCreate(&pref));
  {
    uint64_t ws = ws_bytes;
    WCHK(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)));
  }
  WCHK(hipblasLtMatmulAlgoGetHeuristic(p.handle, desc, la, lb, lc, lc, pref, 1, heur, &found));
  if (found < 1) {
    rc = 2000;
    goto done;
  }
  WCHK(hipblasLtMatmul(p.handle, desc, &alpha, B, la, A, lb, &beta, C, lc, C, lc, &heur[0].algo, workspace, ws_bytes,
                       stream));
done:
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (lc) hipblasLtMatrixLayoutDestroy(lc);
  if (lb) hipblasLtMatrixLayoutDestroy(lb);
  if (la) hipblasLtMatrixLayoutDestroy(la);
  if (desc) hipblasLtMatmulDescDestroy(desc);
  return rc;
#undef WCHK
}

}  // extern "C"
