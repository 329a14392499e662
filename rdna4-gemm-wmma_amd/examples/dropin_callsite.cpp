// The reference's two call sites, rewritten against the library's C++ spelling (include/mmm.hpp).
//
// The GEMM program follows mmm.cpp:1441-1500: host and device buffers held as _Float16* / float*,
// the inputs copied host -> device, one warm-up launch, nbRun launches between HIP events on the
// null stream, a device synchronise, C copied back.  The only change at the call site is the
// launch itself: WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J><<<grid, block>>>(dA, dB, dC)
// becomes mmm::WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(dA, dB, dC, DIM_I, DIM_J, DIM_K)
// (the sizes move from the compile-time globals of mmm.cpp:13-15 to arguments).  The tensor program
// follows mmmTensor.cpp:345-371 without the host pack of G (mmmTensor.cpp:329-340):
// mmm::WMMA_Tensor(dG, d_Input, d_Output, mt, bt, rt, nt, rt_l).
//
// Inputs and output are raw binary files (fp16 bit patterns in, fp32 out) so that a test can
// generate the operands and check C on its side:
//   dropin_callsite gemm   M N K            A.bin B.bin C.bin [kernel]
//   dropin_callsite tensor mt bt rt nt rt_l G.bin In.bin Out.bin
// The gemm mode's optional last argument names the kernel (default WMMA_Swizzled_Full; also the
// lineage's WMMA_Templated_Base, WMMA_LDS_Padded, WMMA_LDS_Swizzled and GEMM_Naive, mmm.cpp:52-62,
// 694-1215).  Prints one line: the best of the timed launches in ms (the reference's best-of-N,
// mmm.cpp:1376-1385).
#include <cstdio>
#include <cstdlib>
#include <string_view>
#include <vector>

#include <hip/hip_runtime.h>

#include "mmm.hpp"

#define HIP_CHECK(x)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

template <class T>
static void read_file(const char* path, T* dst, size_t n) {
  FILE* f = std::fopen(path, "rb");
  if (!f || std::fread(dst, sizeof(T), n, f) != n) {
    std::fprintf(stderr, "cannot read %zu elements from %s\n", n, path);
    std::exit(1);
  }
  std::fclose(f);
}

static void write_file(const char* path, const float* src, size_t n) {
  FILE* f = std::fopen(path, "wb");
  if (!f || std::fwrite(src, sizeof(float), n, f) != n) {
    std::fprintf(stderr, "cannot write %s\n", path);
    std::exit(1);
  }
  std::fclose(f);
}

// nbRun launches of `launch` between events, after one warm-up; returns the best time in ms.
template <class F>
static float time_best(F&& launch, int nbRun) {
  std::vector<hipEvent_t> start(nbRun), stop(nbRun);
  for (int i = 0; i < nbRun; i++) {
    HIP_CHECK(hipEventCreate(&start[i]));
    HIP_CHECK(hipEventCreate(&stop[i]));
  }
  HIP_CHECK(launch());  // warm-up
  HIP_CHECK(hipDeviceSynchronize());
  for (int i = 0; i < nbRun; i++) {
    HIP_CHECK(hipEventRecord(start[i], 0));
    HIP_CHECK(launch());
    HIP_CHECK(hipEventRecord(stop[i], 0));
  }
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipDeviceSynchronize());
  float best = 1e30f;
  for (int i = 0; i < nbRun; i++) {
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, start[i], stop[i]));
    if (ms > 0.0f && ms < best) best = ms;
    HIP_CHECK(hipEventDestroy(start[i]));
    HIP_CHECK(hipEventDestroy(stop[i]));
  }
  return best;
}

static int run_gemm(int DIM_I, int DIM_J, int DIM_K, const char* a_path, const char* b_path, const char* c_path,
                    std::string_view kernel) {
  _Float16 *hA = nullptr, *hB = nullptr, *dA = nullptr, *dB = nullptr;
  float *hC = nullptr, *dC = nullptr;
  const size_t na = (size_t)DIM_I * DIM_K, nb = (size_t)DIM_K * DIM_J, nc = (size_t)DIM_I * DIM_J;
  HIP_CHECK(hipHostMalloc((void**)&hA, na * sizeof(_Float16)));
  HIP_CHECK(hipHostMalloc((void**)&hB, nb * sizeof(_Float16)));
  HIP_CHECK(hipHostMalloc((void**)&hC, nc * sizeof(float)));
  HIP_CHECK(hipMalloc((void**)&dA, na * sizeof(_Float16)));
  HIP_CHECK(hipMalloc((void**)&dB, nb * sizeof(_Float16)));
  HIP_CHECK(hipMalloc((void**)&dC, nc * sizeof(float)));
  read_file(a_path, hA, na);
  read_file(b_path, hB, nb);
  HIP_CHECK(hipMemcpy(dA, hA, na * sizeof(_Float16), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dB, hB, nb * sizeof(_Float16), hipMemcpyHostToDevice));

  // The reference's launched template parameters (mmm.cpp:1462-1465), on the kernel named on the
  // command line (the reference's main launches one of these names at a time)
  constexpr int WAVE_M = 2, WAVE_N = 2, WAVES_I = 4, WAVES_J = 4;
  auto launch = [&]() -> hipError_t {
    if (kernel == "WMMA_Swizzled_Full")
      return mmm::WMMA_Swizzled_Full<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(dA, dB, dC, DIM_I, DIM_J, DIM_K);
    if (kernel == "WMMA_Templated_Base")
      return mmm::WMMA_Templated_Base<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(dA, dB, dC, DIM_I, DIM_J, DIM_K);
    if (kernel == "WMMA_LDS_Padded")
      return mmm::WMMA_LDS_Padded<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(dA, dB, dC, DIM_I, DIM_J, DIM_K);
    if (kernel == "WMMA_LDS_Swizzled")
      return mmm::WMMA_LDS_Swizzled<WAVE_M, WAVE_N, WAVES_I, WAVES_J>(dA, dB, dC, DIM_I, DIM_J, DIM_K);
    if (kernel == "GEMM_Naive") return mmm::GEMM_Naive(dA, dB, dC, DIM_I, DIM_J, DIM_K);
    return hipErrorInvalidValue;
  };
  const float best = time_best(launch, 50);

  HIP_CHECK(hipMemcpy(hC, dC, nc * sizeof(float), hipMemcpyDeviceToHost));
  write_file(c_path, hC, nc);
  std::printf("gemm %dx%dx%d %.*s best %.6f ms\n", DIM_I, DIM_J, DIM_K, (int)kernel.size(), kernel.data(), best);
  HIP_CHECK(hipHostFree(hA));
  HIP_CHECK(hipHostFree(hB));
  HIP_CHECK(hipHostFree(hC));
  HIP_CHECK(hipFree(dA));
  HIP_CHECK(hipFree(dB));
  HIP_CHECK(hipFree(dC));
  return 0;
}

static int run_tensor(int mt, int bt, int rt, int nt, int rt_l, const char* g_path, const char* in_path,
                      const char* out_path) {
  const size_t ng = (size_t)rt * nt * mt * rt_l, nin = (size_t)bt * nt * rt_l, nout = (size_t)mt * bt * rt;
  std::vector<_Float16> G(ng), Input_tensor(nin);
  std::vector<float> Out(nout);
  read_file(g_path, G.data(), ng);
  read_file(in_path, Input_tensor.data(), nin);
  _Float16 *dG = nullptr, *d_Input = nullptr;
  float* d_Output = nullptr;
  HIP_CHECK(hipMalloc((void**)&dG, ng * sizeof(_Float16)));
  HIP_CHECK(hipMalloc((void**)&d_Input, nin * sizeof(_Float16)));
  HIP_CHECK(hipMalloc((void**)&d_Output, nout * sizeof(float)));
  HIP_CHECK(hipMemcpy(dG, G.data(), ng * sizeof(_Float16), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(d_Input, Input_tensor.data(), nin * sizeof(_Float16), hipMemcpyHostToDevice));

  const _Float16* cG = dG;  // the tensor kernel takes const operands (mmmTensor.cpp:44-45)
  const _Float16* cIn = d_Input;
  const float best = time_best([&] { return mmm::WMMA_Tensor(cG, cIn, d_Output, mt, bt, rt, nt, rt_l); }, 100);

  HIP_CHECK(hipMemcpy(Out.data(), d_Output, nout * sizeof(float), hipMemcpyDeviceToHost));
  write_file(out_path, Out.data(), nout);
  std::printf("tensor mt=%d bt=%d rt=%d nt=%d rt_l=%d best %.6f ms\n", mt, bt, rt, nt, rt_l, best);
  HIP_CHECK(hipFree(dG));
  HIP_CHECK(hipFree(d_Input));
  HIP_CHECK(hipFree(d_Output));
  return 0;
}

int main(int argc, char** argv) {
  if ((argc == 8 || argc == 9) && std::string_view(argv[1]) == "gemm")
    return run_gemm(std::atoi(argv[2]), std::atoi(argv[3]), std::atoi(argv[4]), argv[5], argv[6], argv[7],
                    argc == 9 ? std::string_view(argv[8]) : std::string_view("WMMA_Swizzled_Full"));
  if (argc == 10 && std::string_view(argv[1]) == "tensor")
    return run_tensor(std::atoi(argv[2]), std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]),
                      std::atoi(argv[6]), argv[7], argv[8], argv[9]);
  std::fprintf(stderr,
               "usage: %s gemm M N K A.bin B.bin C.bin [WMMA_Swizzled_Full | WMMA_Templated_Base |\n"
               "            WMMA_LDS_Padded | WMMA_LDS_Swizzled | GEMM_Naive]\n"
               "       %s tensor mt bt rt nt rt_l G.bin In.bin Out.bin\n",
               argv[0], argv[0]);
  return 2;
}
