// Measurement probes: the shader clock, and what the MI355X sustains under its power limit
// with the tile kernel's MFMA stream alone (no operand traffic), with its MFMAs and LDS fragment
// reads on operands already in LDS (lds_mfma_probe_kernel, beside the tile kernels), and with
// pure HBM streaming.
// They give the GEMM's roofline fractions a measured denominator next to the spec peaks.  No
// counterpart in the reference, which reports only ms and GFLOPS (mmm.cpp:1503-1504).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mmm.h"
#include "mmm_dma.h"
#include "mmm_kernels.h"
#include "mmm_tile_map.h"

namespace mmm {

namespace {


// One wave reads the shader-clock counter (s_memtime, one count per shader clock) and the
// constant-rate real-time counter (s_memrealtime, 100 MHz), spins until `ticks` real-time
// ticks have passed, and reads both again: clock = d(memtime) / d(realtime) * 100 MHz.
__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t* out, uint64_t ticks) {
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  uint64_t r1 = r0;
  while (r1 - r0 < ticks) r1 = __builtin_amdgcn_s_memrealtime();
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r1 - r0;
  }
}

// Matrix-core ceiling.  The persistent 256x256 tile kernel's MFMA stream -- 256 workgroups of
// 8 waves (2 x 4), each wave 8 x 4 v_mfma_f32_16x16x32_f16 per 32-deep K-step with the
// operands swapped as there -- over the same tiles and K, with its operands held in registers:
// two K-steps of fragments, read once from the real inputs, alternate over the whole K loop.
// No operand loads, no LDS, no barriers.  store_tiles = 1 writes every tile's accumulators to
// C as the tile kernel does (the sums are not A*B: each wave repeats two K-steps);
// store_tiles = 0 writes one value per lane at the end.  Needs M, N multiples of 256 and K of 64.
constexpr int kCeilFM = 8, kCeilFN = 4;

__global__ __launch_bounds__(512, 1) void mfma_ceiling_kernel(const mmm_half* A, const mmm_half* B, float* C, int M,
                                                              int N, int K, int store_tiles, uint64_t* clk) {
  if (clk != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    clk[0] = __builtin_amdgcn_s_memtime();
    clk[1] = __builtin_amdgcn_s_memrealtime();
  }
  const int tiles_m = M / 256, tiles_n = N / 256, ntiles = tiles_m * tiles_n;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int wm = w / 4, wn = w % 4;
  const _Float16* Ah = (const _Float16*)A;
  const _Float16* Bh = (const _Float16*)B;
  // fragments of K-steps 0 and 1 of the workgroup's first tile (MFMA operand layouts: A row
  // l % 16 with k 8*(l/16) .. +7; B column l % 16 with the same k)
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, 4, &tm, &tn);
  half8 fa[2][kCeilFM], fb[2][kCeilFN];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int k = 32 * s + 8 * (lane >> 4);
#pragma unroll
    for (int mb = 0; mb < kCeilFM; ++mb) {
      const int m = tm * 256 + wm * 128 + 16 * mb + (lane & 15);
      fa[s][mb] = *(const half8*)(Ah + (int64_t)m * K + k);
    }
#pragma unroll
    for (int nb = 0; nb < kCeilFN; ++nb) {
      const int n = tn * 256 + wn * 64 + 16 * nb + (lane & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e) fb[s][nb][e] = Bh[(int64_t)(k + e) * N + n];
    }
  }
  float keep = 0.0f;
  for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
    f32x4 acc[kCeilFM][kCeilFN];
#pragma unroll
    for (int i = 0; i < kCeilFM; ++i)
#pragma unroll
      for (int j = 0; j < kCeilFN; ++j) acc[i][j] = f32x4{};
    for (int kk = 0; kk < K; kk += 64) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < kCeilFM * kCeilFN; ++i)
          acc[i / kCeilFN][i % kCeilFN] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              fb[s][i % kCeilFN], fa[s][i / kCeilFN], acc[i / kCeilFN][i % kCeilFN], 0, 0, 0);
    }
    if (store_tiles) {
      tile_of_block(t, tiles_m, tiles_n, 4, &tm, &tn);
#pragma unroll
      for (int mb = 0; mb < kCeilFM; ++mb) {
        float* crow = C + (int64_t)(tm * 256 + wm * 128 + 16 * mb + (lane & 15)) * N + tn * 256 + wn * 64;
#pragma unroll
        for (int nb = 0; nb < kCeilFN; ++nb) *(f32x4*)(crow + 16 * nb + 4 * (lane >> 4)) = acc[mb][nb];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kCeilFM; ++i)
#pragma unroll
        for (int j = 0; j < kCeilFN; ++j) keep += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
    }
  }
  if (!store_tiles) C[(int64_t)blockIdx.x * 512 + threadIdx.x] = keep;
  if (clk != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    clk[2] = __builtin_amdgcn_s_memtime();
    clk[3] = __builtin_amdgcn_s_memrealtime();
  }
}

// HBM read ceiling, plain loads: lanes stream 16-byte chunks (global_load_dwordx4) over
// `n16` chunks, grid-stride, kReadInFlight non-temporal loads in flight per lane, XOR-folded into
// one dword per thread so the loads stay live.  Launched as kReadBlocks workgroups: of the
// configurations swept on MI355X (1024-16384 workgroups, 4, 8 or 16 loads in flight, cached or
// non-temporal, 1 and 2 GiB), 8192 x 4 non-temporal read fastest over 1 GiB (5.87 TB/s; 2048 x 8,
// this probe's earlier shape, 5.40).
constexpr int kReadInFlight = 4;
constexpr int kReadBlocks = 8192;  // both read probes
__global__ __launch_bounds__(256) void read_ceiling_kernel(const u32x4* src, int64_t n16, uint32_t* out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 x = {0, 0, 0, 0};
  for (; i + (kReadInFlight - 1) * stride < n16; i += kReadInFlight * stride) {
    u32x4 v[kReadInFlight];
#pragma unroll
    for (int j = 0; j < kReadInFlight; ++j) v[j] = __builtin_nontemporal_load(src + i + j * stride);
#pragma unroll
    for (int j = 0; j < kReadInFlight; ++j) x ^= v[j];
  }
  for (; i < n16; i += stride) x ^= src[i];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

// HBM read ceiling, direct to LDS (the tile kernels' staging path): each wave streams 1 KB
// pieces (64 lanes x 16 bytes, buffer_load_dwordx4 ... lds, non-temporal like the register
// probe's loads) into a kLdsSlots-slot LDS ring, grid-stride over the waves, keeping at most
// kLdsSlots loads in flight.  Nothing reads the ring.  Swept on MI355X over 1024-8192 workgroups
// and 8-, 16- and 32-slot rings: 8192 workgroups of 32-slot rings (128 KB, one workgroup per CU)
// read fastest (6.59 TB/s over 1 GiB; 2048 x 8 slots, this probe's earlier shape, 5.45).
constexpr int kLdsSlots = 32;
__global__ __launch_bounds__(256) void read_lds_ceiling_kernel(const void* src, uint32_t bytes, uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) char ring[4 * kLdsSlots * 1024];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const i32x4 rsrc = make_rsrc(src, bytes);
  const uint32_t waves = gridDim.x * 4, wid = blockIdx.x * 4 + w;
  const uint32_t pieces = bytes / 1024;
  const uint32_t ring_base = (uint32_t)(uintptr_t)(ring + w * kLdsSlots * 1024);
  int slot = 0;
  for (uint32_t piece = wid; piece < pieces; piece += waves) {
    const uint32_t voff = piece * 1024 + lane * 16;
    dma_b128_nt(ring_base + slot * 1024, rsrc, voff);
    wait_vmcnt<kLdsSlots - 1>();
    slot = slot + 1 == kLdsSlots ? 0 : slot + 1;
  }
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = *(volatile uint32_t*)ring;
}

}  // namespace

}  // namespace mmm

using namespace mmm;

extern "C" {

hipError_t mmm_probe_clock(uint64_t* out, int64_t ticks, hipStream_t stream) {
  if (!out || ticks < 1 || ticks > 10000000) return hipErrorInvalidValue;  // at most 100 ms of spinning
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, stream, out, (uint64_t)ticks);
  return hipGetLastError();
}

hipError_t mmm_probe_mfma_ceiling(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                  int store_tiles, uint64_t* clock, hipStream_t stream) {
  if (!A || !B || !C || M <= 0 || N <= 0 || K <= 0 || ((uintptr_t)clock & 7)) return hipErrorInvalidValue;
  if (M % 256 || N % 256 || K % 64) return hipErrorInvalidValue;
  if ((int64_t)(M / 256) * (N / 256) > 0x7fffffff || ((uintptr_t)A & 15) || ((uintptr_t)C & 15))
    return hipErrorInvalidValue;
  const int64_t tiles = (int64_t)(M / 256) * (N / 256);
  // store_tiles == 0 writes one float per thread: grid * 512 <= tiles * 512 < M * N floats of C
  const int grid = (int)(tiles < 256 ? tiles : 256);
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(grid), dim3(512), 0, stream, A, B, C, M, N, K, store_tiles ? 1 : 0,
                     clock);
  return hipGetLastError();
}

hipError_t mmm_probe_lds_mfma(const mmm_half* A, const mmm_half* B, float* out, int64_t out_floats, int M, int N,
                              int K, int barrier, uint64_t* clock, hipStream_t stream) {
  if (!A || !B || !out || M <= 0 || N <= 0 || K <= 0 || ((uintptr_t)clock & 7)) return hipErrorInvalidValue;
  if (M % 256 || N % 256 || K % 128 || ((uintptr_t)A & 15) || ((uintptr_t)B & 15)) return hipErrorInvalidValue;
  // the staging reads rows m0 .. m0+255 of A and rows 0 .. 127 of B through 32-bit buffer offsets
  if ((int64_t)255 * K + 128 >= (int64_t)kOobOffset / 2 || (int64_t)127 * N + 256 >= (int64_t)kOobOffset / 2 ||
      (int64_t)(M / 256) * (N / 256) > 0x7fffffff)
    return hipErrorInvalidValue;
  const int64_t tiles = (int64_t)(M / 256) * (N / 256);
  if (out_floats < (tiles < 256 ? tiles : 256) * 512) return hipErrorInvalidValue;
  GemmProblem p{};
  p.A = A, p.B = B, p.C = nullptr;
  p.M = M, p.N = N, p.K = K;
  p.lda = K, p.ldb = N, p.ldc = N;
  p.clk = clock;
  return launch_lds_mfma_probe(p, barrier != 0, out, stream);
}

hipError_t mmm_probe_read(const void* src, int64_t bytes, int direct_to_lds, uint32_t* out, int64_t out_words,
                          hipStream_t stream) {
  if (!src || !out || bytes <= 0 || (bytes & 1023) || ((uintptr_t)src & 15)) return hipErrorInvalidValue;
  const int blocks = kReadBlocks;
  if (direct_to_lds) {
    if (bytes >= 0x7fffffff || out_words < blocks) return hipErrorInvalidValue;
    hipLaunchKernelGGL(read_lds_ceiling_kernel, dim3(blocks), dim3(256), 0, stream, src, (uint32_t)bytes, out);
  } else {
    if (out_words < (int64_t)blocks * 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(read_ceiling_kernel, dim3(blocks), dim3(256), 0, stream, (const u32x4*)src, bytes / 16, out);
  }
  return hipGetLastError();
}

}  // extern "C"
