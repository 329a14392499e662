// hipBLASLt witness: the vendor GEMM on the same FP16 -> FP32 row-major problem, used only
// by bench.py and the tests as a comparison point (the reference compares against
// rocblas_gemm_ex the same way, mmm.cpp:1508-1534).  Not part of the product path.
//
// Row-major C[M][N] = A[M][K] * B[K][N] is computed as the column-major product
// C^T[N][M] = B^T[N][K] * A^T[K][M] (the operand swap of mmm.cpp:1519-1521).
//
// A bound plan (mmm_witness_hipblaslt_create) builds the matmul descriptor, the three layouts
// and the preference and asks the algorithm heuristic for up to kMaxAlgos candidates once per
// shape; mmm_witness_hipblaslt_tune times every candidate on the real operands and binds the
// fastest (without it the heuristic's first pick runs).  Each mmm_witness_hipblaslt_run is then
// one hipblasLtMatmul call, so a timed loop measures the vendor kernel and its launch, as the
// library's bound launchers are measured.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdint.h>

#include <algorithm>
#include <new>
#include <vector>

namespace {

constexpr int kMaxAlgos = 16;

hipblasLtHandle_t& shared_handle() {
  static thread_local hipblasLtHandle_t h = nullptr;
  return h;
}

struct WitnessPlan {
  hipblasLtHandle_t handle = nullptr;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasLtMatmulHeuristicResult_t heur[kMaxAlgos]{};
  int n_algos = 0;  // candidates the heuristic returned
  int chosen = 0;   // the candidate each run uses
};

void release(WitnessPlan* w) {
  if (w->pref) hipblasLtMatmulPreferenceDestroy(w->pref);
  if (w->lc) hipblasLtMatrixLayoutDestroy(w->lc);
  if (w->lb) hipblasLtMatrixLayoutDestroy(w->lb);
  if (w->la) hipblasLtMatrixLayoutDestroy(w->la);
  if (w->desc) hipblasLtMatmulDescDestroy(w->desc);
  delete w;
}

}  // namespace

extern "C" {

// Plans the row-major problem once.  Returns 0 and *out on success, a hipblasStatus_t (+1000)
// or 2000 (no algorithm) otherwise.
int mmm_witness_hipblaslt_create(int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, size_t ws_bytes,
                                 void** out) {
  if (!out) return 2001;
  *out = nullptr;
  hipblasLtHandle_t& h = shared_handle();
  if (!h && hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return 1001;
  WitnessPlan* w = new (std::nothrow) WitnessPlan;
  if (!w) return 2002;
  w->handle = h;
  int rc = 0;
  int found = 0;
  hipblasOperation_t op = HIPBLAS_OP_N;
#define WCHK(x)                         \
  do {                                  \
    hipblasStatus_t s_ = (x);           \
    if (s_ != HIPBLAS_STATUS_SUCCESS) { \
      rc = 1000 + (int)s_;              \
      goto fail;                        \
    }                                   \
  } while (0)
  WCHK(hipblasLtMatmulDescCreate(&w->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  WCHK(hipblasLtMatmulDescSetAttribute(w->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op)));
  WCHK(hipblasLtMatmulDescSetAttribute(w->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op)));
  // column-major: "A" = B^T (N x K, ld ldb), "B" = A^T (K x M, ld lda), "C" = C^T (N x M, ld ldc)
  WCHK(hipblasLtMatrixLayoutCreate(&w->la, HIP_R_16F, N, K, ldb));
  WCHK(hipblasLtMatrixLayoutCreate(&w->lb, HIP_R_16F, K, M, lda));
  WCHK(hipblasLtMatrixLayoutCreate(&w->lc, HIP_R_32F, N, M, ldc));
  WCHK(hipblasLtMatmulPreferenceCreate(&w->pref));
  {
    uint64_t ws = ws_bytes;
    WCHK(hipblasLtMatmulPreferenceSetAttribute(w->pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)));
  }
  WCHK(hipblasLtMatmulAlgoGetHeuristic(h, w->desc, w->la, w->lb, w->lc, w->lc, w->pref, kMaxAlgos, w->heur,
                                       &found));
#undef WCHK
  if (found < 1) {
    rc = 2000;
    goto fail;
  }
  w->n_algos = std::min(found, kMaxAlgos);
  w->chosen = 0;
  *out = w;
  return 0;
fail:
  release(w);
  return rc;
}

// One hipblasLtMatmul of a bound plan (C = A * B, alpha 1, beta 0).
int mmm_witness_hipblaslt_run(void* plan, const void* A, const void* B, float* C, void* workspace, size_t ws_bytes,
                              hipStream_t stream) {
  if (!plan) return 2001;
  WitnessPlan* w = (WitnessPlan*)plan;
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s = hipblasLtMatmul(w->handle, w->desc, &alpha, B, w->la, A, w->lb, &beta, C, w->lc, C, w->lc,
                                            &w->heur[w->chosen].algo, workspace, ws_bytes, stream);
  return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + (int)s;
}

// Times every candidate of the plan on these operands -- one untimed matmul, then `reps` matmuls
// between HIP events on `stream`, the median of their durations -- and binds the fastest.  A
// candidate whose workspace exceeds ws_bytes, or whose matmul fails, is skipped.  *best and
// *best_ms (either may be NULL) receive the winner's index in the heuristic's order and its
// median; ms_each (NULL, or n_algos floats) each candidate's median, -1 when skipped.  Synchronises
// the stream.  Returns 0, 2000 if no candidate ran, or a HIP error + 3000.
int mmm_witness_hipblaslt_tune(void* plan, const void* A, const void* B, float* C, void* workspace, size_t ws_bytes,
                               hipStream_t stream, int reps, int* best, float* best_ms, float* ms_each) {
  if (!plan || reps < 1) return 2001;
  WitnessPlan* w = (WitnessPlan*)plan;
  hipEvent_t ev[2 * 64];
  if (reps > 64) reps = 64;
  for (int i = 0; i < 2 * reps; ++i)
    if (hipEventCreate(&ev[i]) != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      return 3000 + (int)hipErrorOutOfMemory;
    }
  int win = -1;
  float win_ms = 0.0f;
  int rc = 0;
  const int keep = w->chosen;
  std::vector<float> t(reps);
  for (int a = 0; a < w->n_algos && rc == 0; ++a) {
    if (ms_each) ms_each[a] = -1.0f;
    if (w->heur[a].workspaceSize > ws_bytes) continue;
    w->chosen = a;
    if (mmm_witness_hipblaslt_run(plan, A, B, C, workspace, ws_bytes, stream) != 0) continue;
    bool ok = true;
    for (int r = 0; r < reps && ok; ++r) {
      ok = hipEventRecord(ev[2 * r], stream) == hipSuccess &&
           mmm_witness_hipblaslt_run(plan, A, B, C, workspace, ws_bytes, stream) == 0 &&
           hipEventRecord(ev[2 * r + 1], stream) == hipSuccess;
    }
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
      rc = 3000 + (int)e;
      break;
    }
    if (!ok) continue;
    for (int r = 0; r < reps && ok; ++r) ok = hipEventElapsedTime(&t[r], ev[2 * r], ev[2 * r + 1]) == hipSuccess;
    if (!ok) continue;
    std::sort(t.begin(), t.end());
    const float med = t[reps / 2];
    if (ms_each) ms_each[a] = med;
    if (win < 0 || med < win_ms) win = a, win_ms = med;
  }
  for (int i = 0; i < 2 * reps; ++i) (void)hipEventDestroy(ev[i]);
  if (rc != 0 || win < 0) {
    w->chosen = keep;
    return rc != 0 ? rc : 2000;
  }
  w->chosen = win;
  if (best) *best = win;
  if (best_ms) *best_ms = win_ms;
  return 0;
}

// The plan's candidate count and the candidate its runs use (index in the heuristic's order).
int mmm_witness_hipblaslt_info(void* plan, int* n_algos, int* chosen) {
  if (!plan) return 2001;
  WitnessPlan* w = (WitnessPlan*)plan;
  if (n_algos) *n_algos = w->n_algos;
  if (chosen) *chosen = w->chosen;
  return 0;
}

void mmm_witness_hipblaslt_destroy(void* plan) {
  if (plan) release((WitnessPlan*)plan);
}

// One-shot form (plan, run, release): for checks, not for timing.
int mmm_witness_hipblaslt_gemm(const void* A, const void* B, float* C, int M, int N, int K, int64_t lda,
                               int64_t ldb, int64_t ldc, void* workspace, size_t ws_bytes, hipStream_t stream) {
  void* plan = nullptr;
  int rc = mmm_witness_hipblaslt_create(M, N, K, lda, ldb, ldc, ws_bytes, &plan);
  if (rc != 0) return rc;
  rc = mmm_witness_hipblaslt_run(plan, A, B, C, workspace, ws_bytes, stream);
  mmm_witness_hipblaslt_destroy(plan);
  return rc;
}

}  // extern "C"
