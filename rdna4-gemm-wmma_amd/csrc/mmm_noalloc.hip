// mmm_gemm_f16f32_noalloc: mmm_gemm_f16f32_ws with the K-split partials in a file-scope device
// array instead of a caller's workspace, for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc).  It calls no allocating routine.
//
// The array is kScratchBytes (64 MiB, the most any planned split uses), and each GPU the library
// runs on holds its own copy until the process ends.  Its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and kept; host code never passes the
// array's own name to a kernel.  Every call on one GPU shares that GPU's array: the split kernels
// overwrite every partial the reduction reads, so nothing needs clearing between calls, but calls
// that overlap on one GPU (different streams, or graph replays concurrent with eager calls) race
// on it.  The kept address is not looked up again: hipDeviceReset frees the device's copy, and
// calls on that device afterwards would hand the kernels a stale address.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "mmm.h"
#include "mmm_kernels.h"

namespace mmm {

constexpr size_t kScratchBytes = kMaxWorkspaceBytes;
static_assert(kScratchBytes >= kMaxWorkspaceBytes, "the scratch array holds every split the planner makes");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// The current device's copy of `scratch` (looked up on the first call on that device).
hipError_t scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

}  // namespace mmm

using namespace mmm;

extern "C" hipError_t mmm_gemm_f16f32_noalloc(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                              int64_t lda, int64_t ldb, int64_t ldc, hipStream_t stream) {
  size_t need = 0;
  hipError_t e = mmm_gemm_workspace_f16f32(A, B, C, M, N, K, lda, ldb, ldc, &need);  // validates the arguments
  if (e != hipSuccess) return e;
  if (need > kScratchBytes) return hipErrorInvalidValue;  // a split beyond the array's size
  if (M == 0 || N == 0) return hipSuccess;
  void* ws = nullptr;
  if ((e = scratch_of_current_device(&ws)) != hipSuccess) return e;
  return mmm_gemm_f16f32_ws(A, B, C, M, N, K, lda, ldb, ldc, ws, kScratchBytes, stream);
}
