// C ABI of the MI355X GEMM / contraction library (declarations and reference citations in
// include/mmm.h): argument validation, kernel selection, contraction descriptors, and the
// seeded on-device input generator.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

#include "mmm.h"
#include "mmm_kernels.h"
#include "mmm_tile_map.h"

namespace mmm {

// ---------------------------------------------------------------- seeded input generator
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t stream_key(uint64_t seed, uint32_t tensor_id) {
  uint64_t z = seed * 0x9E3779B97F4A7C15ull + (uint64_t)tensor_id + 1ull;
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// fp64 -> fp16 with a single round-to-nearest-even (integer arithmetic, no fp32 detour).
__device__ __forceinline__ uint16_t f64_to_f16_rne(double d) {
  const uint64_t x = __builtin_bit_cast(uint64_t, d);
  const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
  const uint64_t ax = x & 0x7fffffffffffffffull;
  if (ax >= 0x7ff0000000000000ull) return sign | (ax == 0x7ff0000000000000ull ? 0x7c00u : 0x7e00u);
  if (ax >= 0x40effe0000000000ull) return sign | 0x7c00u;  // >= 65520 rounds to inf
  const int e = (int)(ax >> 52) - 1023;
  if (e >= -14) {
    const uint64_t mant = ax & 0xfffffffffffffull;
    uint64_t h = ((uint64_t)(e + 15) << 10) | (mant >> 42);
    const uint64_t rem = mant & ((1ull << 42) - 1ull);
    if (rem > (1ull << 41) || (rem == (1ull << 41) && (h & 1ull))) h++;
    return sign | (uint16_t)h;
  }
  if (e < -1022) return sign;
  const uint64_t mant = (ax & 0xfffffffffffffull) | (1ull << 52);
  const int shift = 28 - e;
  if (shift > 53) return sign;
  uint64_t h = mant >> shift;
  const uint64_t rem = mant & ((1ull << shift) - 1ull);
  const uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (h & 1ull))) h++;
  return sign | (uint16_t)h;
}

__global__ void fill_uniform_kernel(mmm_half* out, int64_t n, uint64_t key) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t x = splitmix64(key + (uint64_t)i);
    const float v = (float)(uint32_t)(x >> 40) * 1.1920928955078125e-07f - 1.0f;  // exact
    out[i] = __builtin_bit_cast(uint16_t, (_Float16)v);                            // v_cvt_f16_f32, RNE
  }
}

__global__ void fill_normal_kernel(mmm_half* out, int64_t n, uint64_t key, double scale) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t x1 = splitmix64(key + 2ull * (uint64_t)i);
    const uint64_t x2 = splitmix64(key + 2ull * (uint64_t)i + 1ull);
    const double u1 = (double)((x1 >> 11) + 1ull) * 1.1102230246251565e-16;
    const double u2 = (double)(x2 >> 11) * 1.1102230246251565e-16;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    out[i] = f64_to_f16_rne(z * scale);
  }
}

static unsigned fill_blocks(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_fill_uniform(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, hipStream_t stream) {
  hipLaunchKernelGGL(fill_uniform_kernel, dim3(fill_blocks(n)), dim3(256), 0, stream, out, n,
                     stream_key(seed, tensor_id));
  return hipGetLastError();
}

hipError_t launch_fill_normal(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, double scale,
                              hipStream_t stream) {
  hipLaunchKernelGGL(fill_normal_kernel, dim3(fill_blocks(n)), dim3(256), 0, stream, out, n,
                     stream_key(seed, tensor_id), scale);
  return hipGetLastError();
}

// ---------------------------------------------------------------- zero fill (K == 0)
__global__ void zero_kernel(float* C, int M, int N, int64_t ldc) {
  const int64_t total = (int64_t)M * N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
    C[(i / N) * ldc + (i % N)] = 0.0f;
}

__global__ void zero_fold_kernel(FoldProblem p) {
  const int64_t total = (int64_t)p.M * p.N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int m = (int)(i / p.N), n = (int)(i % p.N);
    const int64_t off = (int64_t)(m / p.m_lo) * p.cm[0] + (int64_t)(m % p.m_lo) * p.cm[1] +
                        (int64_t)(n / p.n_lo) * p.cn[0] + (int64_t)(n % p.n_lo) * p.cn[1];
    p.C[off] = 0.0f;
  }
}

hipError_t launch_zero_f32(float* C, int M, int N, int64_t ldc, hipStream_t stream) {
  hipLaunchKernelGGL(zero_kernel, dim3(fill_blocks((int64_t)M * N)), dim3(256), 0, stream, C, M, N, ldc);
  return hipGetLastError();
}

hipError_t launch_zero_fold(const FoldProblem& p, hipStream_t stream) {
  hipLaunchKernelGGL(zero_fold_kernel, dim3(fill_blocks((int64_t)p.M * p.N)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------- tile selection
constexpr double kPartialRoundBoost = 0.3;

// Estimated time of a tile launch, in seconds: rounds of 256 concurrent workgroups (one per
// CU) times the MFMA time of one tile's K range at the tile's relative efficiency -- its MFMA
// rate against the 256x256 tile's.  Measured at 8192^3 with each tile forced, as throughput
// (128x256 0.82, 256x128 0.84, 128x128 0.75, 192x192 0.82, 64x64 0.38) and as the matrix cores'
// busy share under rocprofv3 (SQ_VALU_MFMA_BUSY_CYCLES: 256x256 0.732; 128x256 0.600, 256x128
// 0.598 -> 0.82; 128x128 0.575 -> 0.79; 192x192 0.608 -> 0.83; 64x64 0.291 -> 0.40).  What lowers
// the smaller tiles' rate is operand loads per flop ((BM + BN) / (BM * BN): 1.5x for the narrow
// tiles, 2x for 128x128, 4x for 64x64), which saturate the address unit (TA busy 0.48 for
// 256x256, 0.59-0.65 narrow, 0.83 for 128x128, 0.89 for 64x64); no tile has LDS bank conflicts.
// The narrow tiles are priced at 0.82 and 128x128 at 0.76; 192x192 and 64x64 at 0.86 and 0.30,
// the values that pick the faster tile on the shapes
// measured for them: 192x192 on 3072^3, 3072^2 x 8192, 4357 x 4095 x 4111 and the 4-way K split
// of 1536^2 x 12288 (937 TFLOP/s against 864 for a 7-way split of 256x256 tiles), 256x256 on
// 2304^2 x 8192, 4608^2 x 8192, 6144^3, 6144^2 x 2048 and 3000 x 5000 x 1000; 64x64 on 256^3 to
// 1024^2 x 2048, 128x128 from 1536^3) plus a fixed per-round cost (prologue, epilogue).
// With a K split (gemm_nn_split) the split tiles' round runs K / splits, and the reduction's
// traffic (priced at kSplitCostBps) and launch are added.
// The prices (kEff64, kEff192, kPartialRoundBoost, kSplitCostBps) were fitted, with an offline
// restatement of this function, to every forced-tile time measured on MI355X: the 39 shapes of
// the tile and transformer-layer sweeps, which they pick exactly as before (within 0.13% of the
// fastest tile on average), and 40 shapes of 136 to 256 rows (4096 to 28672 wide, K 4096 to
// 28672), timed with B resident and with B rotating through HBM as a model's weights are.  On
// those the pick went from 3.3% (resident) and 6.2% (rotating) behind the fastest tile on
// average to 0.8% and 0.5%: 64x64 gave way to 128x128 at 136-192 x 4096 x 4096 (rotating B:
// 30.1 -> 23.6 us at 192 rows), 192x192 to 256x128 at 136-192 x 28672 x 8192 (141.0 -> 126.1 us
// at 192 rows), and 256x256 with an 8-way K split to 256x128 at 224-256 x 8192 x 8192 (59.3 ->
// 49.9 us at 256 rows, B resident).
constexpr double kEff64 = 0.30, kEff128 = 0.76, kEffNarrow = 0.82, kEff192 = 0.86;
// Reduction traffic of a K split as tile_cost prices it against other tiles (the split decision
// itself, gemm_nn_split, uses kSplitTrafficBps).
constexpr double kSplitCostBps = 5e12;
// The 128x128 tile in an unsplit launch of one round runs its 3-stage ring (DeepTile128), faster
// per CU than the 2-stage multi-round version the 0.76 was measured on.  Priced at 0.70: that
// still picks it at 512 x 8192 x 8192 (867-919 TFLOP/s against 842-876 for a 4-way K split of 64
// 256x256 tiles) and gives 448-512 x 4096 x 4096 to 256x128 tiles (measured with B rotating
// through HBM 521 against 399 TFLOP/s at 512 rows, B resident +8%), which the earlier 0.80 put on
// 128x128; no other pick of the measured sets changes.
constexpr double kEff128Deep = 0.70;
static double tile_cost(const GemmProblem& p, int tile, int* splits_out) {
  static const double eff_of[kTileCount] = {1.0, kEffNarrow, kEffNarrow, kEff128, kEff64, kEff192};
  const int bm = tile_bm(tile), bn = tile_bn(tile);
  const TileSplit sp = gemm_nn_split(p, tile);
  const double tiles = (double)((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
  const double tile_eff = tile == kTile128x128 && sp.splits <= 1 && tiles <= 256.0 ? kEff128Deep : eff_of[tile];
  const double per_cu_flops = 4.8e12;  // sustained MFMA rate of one CU under load (256x256 at 8192^3)
  // A round with `active` of its 256 slots busy runs each CU faster: the chip is then below its
  // power cap and keeps a higher clock.  Fitted with the prices above (3072^3 ran 878 TFLOP/s
  // on 144 256x256 tiles against 811 on the 128x256 tile the full-load rate preferred; with the
  // refitted tile prices, 0.3 keeps that pick and every other pick of the sweeps).
  auto round = [&](double k, double active) {
    const double boost = 1.0 + kPartialRoundBoost * (1.0 - std::min(active, 256.0) / 256.0);
    return 2.0 * bm * bn * k / (per_cu_flops * tile_eff * boost) + 3e-6;
  };
  // A persistent grid overlaps each tile's epilogue with the next tile's first loads, so its
  // rounds after the first cost 1 us instead of 3 (fitted: it picks the persistent 192x192 grid
  // at 6144^2 x 2048 and 3072 x 6144 x 2048, measured 13% and 16% faster than 256x256 tiles
  // there, and keeps 256x256 at 12288 x 6144 x 2048, 5% faster than 192x192).
  const double later_round_saving = gemm_nn_persistent(p, tile) ? 2e-6 : 0.0;
  auto rounds = [&](double n, double k) {  // n workgroups of K depth k, in rounds of 256
    const double full = std::floor(n / 256.0), rest = n - full * 256.0;
    const double t = full * round(k, 256.0) + (rest > 0.0 ? round(k, rest) : 0.0);
    return t - later_round_saving * std::max(0.0, std::ceil(n / 256.0) - 1.0);
  };
  const double k_full = std::ceil((double)p.K / 64.0) * 64.0;
  double t;
  if (sp.splits > 1) {
    t = rounds(tiles - sp.tiles, k_full) +
        round(std::ceil((double)p.K / sp.splits / 64.0) * 64.0, (double)sp.tiles * sp.splits) +
        (double)sp.tiles * bm * bn * 4.0 * (2.0 * sp.splits + 1) / kSplitCostBps + 3e-6;
  } else {
    t = rounds(tiles, k_full);
  }
  *splits_out = sp.splits;
  return t;
}

// The cheapest tile by tile_cost; a smaller tile must win by 3% (where the estimates are that
// close, the measured times are too, and the larger tile reads less LDS per MAC).
static int pick_tile(const GemmProblem& p) {
  int best = kTile256x256, s = 1;
  double best_cost = 1e300;
  for (int tile : {kTile256x256, kTile256x128, kTile128x256, kTile128x128, kTile64x64, kTile192x192}) {
    if (tile == kTile192x192 && !gemm_nn_direct_to_lds(p, tile)) continue;  // direct-to-LDS only
    const double c = tile_cost(p, tile, &s);
    if (c < best_cost * 0.97) {
      best_cost = c;
      best = tile;
    }
  }
  return best;
}


// What mmm_gemm_f16f32 launches for a validated problem.
struct GemmPlan {
  int kind;       // MMM_KERNEL_*
  int tile;       // TileId of the matrix-core kernel, -1 if none
  int tile_rows;  // rows of C on the matrix-core kernel (the rest on the streaming kernel)
};

static GemmPlan plan_gemm(const GemmProblem& p) {
  if (p.M == 0 || p.N == 0) return {MMM_KERNEL_NONE, -1, 0};
  if (p.K == 0) return {MMM_KERNEL_ZERO, -1, 0};
  // M <= 64: HBM-bound streaming kernel, unless its strips run better as tiles
  if (skinny_ok(p) && !skinny_prefers_tiles(p) && !skinny_tiles_faster(p)) return {MMM_KERNEL_STREAM, -1, 0};
  // A few rows past a whole number of 256-row tiles (4097 = 16*256 + 1) would cost a full
  // extra round of tiles; those rows go to the streaming kernel instead when that saves a round.
  const int rem = p.M % 256;
  if (p.M > 256 && rem > 0 && rem <= kStreamMaxRows) {
    const int Mm = p.M - rem;
    const int64_t tn = (p.N + 255) / 256;
    const int64_t rounds_full = ((int64_t)((p.M + 255) / 256) * tn + 255) / 256;
    const int64_t rounds_main = ((int64_t)(Mm / 256) * tn + 255) / 256;
    GemmProblem pr = p;
    pr.M = rem;
    pr.A = p.A + (int64_t)Mm * p.lda;
    pr.C = p.C + (int64_t)Mm * p.ldc;
    GemmProblem pm = p;
    pm.M = Mm;
    if (rounds_main < rounds_full && skinny_ok(pr) && !skinny_prefers_tiles(pr))
      return {MMM_KERNEL_TILE_STREAM, pick_tile(pm), Mm};
  }
  return {MMM_KERNEL_TILE, pick_tile(p), p.M};
}

static hipError_t check_gemm(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                             int64_t ldb, int64_t ldc) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!C) return hipErrorInvalidValue;
  if (K > 0 && (!A || !B)) return hipErrorInvalidValue;
  if (lda < K || ldb < N || ldc < N) return hipErrorInvalidValue;
  return hipSuccess;
}

static int tile_from_params(int wave_m, int wave_n, int waves_i, int waves_j) {
  if (waves_i != 2 || waves_j != 2) return -1;
  if (wave_m == 4 && wave_n == 4) return kTile256x256;
  if (wave_m == 2 && wave_n == 4) return kTile128x256;
  if (wave_m == 4 && wave_n == 2) return kTile256x128;
  if (wave_m == 2 && wave_n == 2) return kTile128x128;
  if (wave_m == 1 && wave_n == 1) return kTile64x64;
  if (wave_m == 3 && wave_n == 3) return kTile192x192;
  return -1;
}

static bool collapse(int64_t ext_hi, int64_t ext_lo, int64_t s_hi, int64_t s_lo, int64_t* stride) {
  if (ext_hi <= 1) {
    *stride = s_lo;
    return true;
  }
  if (ext_lo <= 1) {
    *stride = s_hi;
    return true;
  }
  if (s_hi == ext_lo * s_lo) {
    *stride = s_lo;
    return true;
  }
  return false;
}

// Descriptor -> FoldProblem with validated extents.  C may be null (the fp64 check writes its
// own outputs at C's offsets); the caller checks it where it is needed.
static hipError_t fold_from_desc(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, float* C,
                                 FoldProblem* out) {
  if (!d) return hipErrorInvalidValue;
  // every extent fits int32 before any product is formed (a product of two caller extents could
  // otherwise overflow int64 and wrap to a small or zero size)
  for (int q = 0; q < 2; ++q)
    if (d->m_ext[q] < 0 || d->n_ext[q] < 0 || d->k_ext[q] < 0 || d->m_ext[q] > 0x7fffffff ||
        d->n_ext[q] > 0x7fffffff || d->k_ext[q] > 0x7fffffff)
      return hipErrorInvalidValue;
  const int64_t M = d->m_ext[0] * d->m_ext[1], N = d->n_ext[0] * d->n_ext[1], K = d->k_ext[0] * d->k_ext[1];
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return hipErrorInvalidValue;
  FoldProblem& p = *out;
  p = FoldProblem{};
  p.A = A, p.B = B, p.C = C;
  p.M = (int)M, p.N = (int)N, p.K = (int)K;
  if (M == 0 || N == 0) return hipSuccess;
  if (K > 0 && (!A || !B)) return hipErrorInvalidValue;
  p.m_lo = (int)(d->m_ext[1] > 0 ? d->m_ext[1] : 1);
  p.n_lo = (int)(d->n_ext[1] > 0 ? d->n_ext[1] : 1);
  p.k_lo = (int)(d->k_ext[1] > 0 ? d->k_ext[1] : 1);
  for (int q = 0; q < 2; ++q) {
    p.am[q] = d->a_m_stride[q], p.ak[q] = d->a_k_stride[q];
    p.bk[q] = d->b_k_stride[q], p.bn[q] = d->b_n_stride[q];
    p.cm[q] = d->c_m_stride[q], p.cn[q] = d->c_n_stride[q];
  }
  return hipSuccess;
}

// A row-major GEMM as a fold whose high sub-indices have extent 1.
static FoldProblem fold_of_gemm(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                                int64_t ldb, int64_t ldc) {
  FoldProblem p{};
  p.A = A, p.B = B, p.C = C;
  p.M = M, p.N = N, p.K = K;
  p.m_lo = M > 0 ? M : 1, p.n_lo = N > 0 ? N : 1, p.k_lo = K > 0 ? K : 1;
  p.am[1] = lda, p.ak[1] = 1;
  p.bk[1] = ldb, p.bn[1] = 1;
  p.cm[1] = ldc, p.cn[1] = 1;
  return p;
}

// Workspace bytes the planned launch's K splits need (0: none).  The tile and streaming
// kernels of a tile+stream plan run one after the other on the stream, so they share it.
static size_t plan_workspace_bytes(const GemmProblem& p, const GemmPlan& pl) {
  size_t need = 0;
  if (pl.kind == MMM_KERNEL_TILE || pl.kind == MMM_KERNEL_TILE_STREAM) {
    GemmProblem pm = p;
    pm.M = pl.tile_rows;
    need = std::max(need, gemm_nn_workspace_bytes(pm, pl.tile));
  }
  if (pl.kind == MMM_KERNEL_STREAM || pl.kind == MMM_KERNEL_TILE_STREAM) {
    GemmProblem pr = p;
    pr.M = p.M - pl.tile_rows;
    pr.A = p.A + (int64_t)pl.tile_rows * p.lda;
    need = std::max(need, skinny_workspace_bytes(pr));
  }
  return need;
}

// A caller's workspace is optional (null: the unsplit kernels run) and 16-byte aligned (the
// reductions read it as float4).
static hipError_t check_workspace(const void* ws) {
  return ((uintptr_t)ws & 15) ? hipErrorInvalidValue : hipSuccess;
}

// A fold that is a plain row-major GEMM (every pair of sub-indices collapses to one stride,
// unit along K for A and along N for B and C): its leading dimensions.
static bool plain_gemm(const mmm_contract_desc* d, int64_t K, int64_t N, int64_t* lda, int64_t* ldb, int64_t* ldc) {
  int64_t ak, bn, cn;
  return collapse(d->m_ext[0], d->m_ext[1], d->a_m_stride[0], d->a_m_stride[1], lda) &&
         collapse(d->k_ext[0], d->k_ext[1], d->a_k_stride[0], d->a_k_stride[1], &ak) && ak == 1 &&
         collapse(d->k_ext[0], d->k_ext[1], d->b_k_stride[0], d->b_k_stride[1], ldb) &&
         collapse(d->n_ext[0], d->n_ext[1], d->b_n_stride[0], d->b_n_stride[1], &bn) && bn == 1 &&
         collapse(d->m_ext[0], d->m_ext[1], d->c_m_stride[0], d->c_m_stride[1], ldc) &&
         collapse(d->n_ext[0], d->n_ext[1], d->c_n_stride[0], d->c_n_stride[1], &cn) && cn == 1 && *lda >= K &&
         *ldb >= N && *ldc >= N;
}

}  // namespace mmm

using namespace mmm;

extern "C" {

hipError_t mmm_gemm_f16f32(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                           int64_t ldb, int64_t ldc, hipStream_t stream) {
  return mmm_gemm_f16f32_ws(A, B, C, M, N, K, lda, ldb, ldc, nullptr, 0, stream);
}

hipError_t mmm_gemm_f16f32_ws(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                              int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return mmm_gemm_f16f32_clocked(A, B, C, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, nullptr, stream);
}

hipError_t mmm_gemm_f16f32_clocked(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                   int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                                   uint64_t* clock, hipStream_t stream) {
  hipError_t e = check_gemm(A, B, C, M, N, K, lda, ldb, ldc);
  if (e != hipSuccess) return e;
  if ((e = check_workspace(workspace)) != hipSuccess) return e;
  if ((uintptr_t)clock & 7) return hipErrorInvalidValue;
  GemmProblem p{A, B, C, M, N, K, lda, ldb, ldc, false, false};
  p.ws = (float*)workspace;
  p.ws_bytes = workspace ? workspace_bytes : 0;
  p.ws_absent = workspace == nullptr;
  p.clk = clock;
  const GemmPlan pl = plan_gemm(p);
  switch (pl.kind) {
    case MMM_KERNEL_NONE:
      return hipSuccess;
    case MMM_KERNEL_ZERO:
      return launch_zero_f32(C, M, N, ldc, stream);
    case MMM_KERNEL_STREAM:
      return launch_gemm_skinny(p, stream);
    case MMM_KERNEL_TILE_STREAM: {
      GemmProblem pm = p, pr = p;
      pm.M = pl.tile_rows;
      pr.M = M - pl.tile_rows;
      pr.clk = nullptr;
      pr.A = A + (int64_t)pl.tile_rows * lda;
      pr.C = C + (int64_t)pl.tile_rows * ldc;
      e = launch_gemm_nn(pm, pl.tile, stream);
      if (e != hipSuccess) return e;
      return launch_gemm_skinny(pr, stream);
    }
    default:
      return launch_gemm_nn(p, pl.tile, stream);
  }
}

hipError_t mmm_gemm_plan_f16f32(const mmm_half* A, const mmm_half* B, const float* C, int M, int N, int K,
                                int64_t lda, int64_t ldb, int64_t ldc, mmm_gemm_plan* plan) {
  if (!plan) return hipErrorInvalidValue;
  // only the addresses' alignment matters here; null stands for a 256-byte-aligned buffer
  const mmm_half* a = A ? A : (const mmm_half*)(uintptr_t)256;
  const mmm_half* b = B ? B : (const mmm_half*)(uintptr_t)256;
  float* c = C ? (float*)C : (float*)(uintptr_t)256;
  hipError_t e = check_gemm(a, b, c, M, N, K, lda, ldb, ldc);
  if (e != hipSuccess) return e;
  const GemmProblem p{a, b, c, M, N, K, lda, ldb, ldc, false, false};
  const GemmPlan pl = plan_gemm(p);
  *plan = mmm_gemm_plan{};
  plan->kernel = pl.kind;
  if (pl.tile >= 0) {
    static const int params[kTileCount][4] = {{4, 4, 2, 2}, {2, 4, 2, 2}, {4, 2, 2, 2},
                                              {2, 2, 2, 2}, {1, 1, 2, 2}, {3, 3, 2, 2}};
    plan->wave_m = params[pl.tile][0], plan->wave_n = params[pl.tile][1];
    plan->waves_i = params[pl.tile][2], plan->waves_j = params[pl.tile][3];
    plan->block_m = tile_bm(pl.tile), plan->block_n = tile_bn(pl.tile);
    plan->tile_rows = pl.tile_rows;
    plan->tile_workgroups = (int64_t)((pl.tile_rows + plan->block_m - 1) / plan->block_m) *
                            ((N + plan->block_n - 1) / plan->block_n);
    GemmProblem pm = p;
    pm.M = pl.tile_rows;
    plan->direct_to_lds = gemm_nn_direct_to_lds(pm, pl.tile) ? 1 : 0;
    const TileSplit sp = gemm_nn_split(pm, pl.tile);
    plan->tile_splits = sp.splits;
    plan->tile_split_tiles = sp.splits > 1 ? sp.tiles : 0;
    plan->tile_persistent = plan->direct_to_lds && gemm_nn_persistent(pm, pl.tile) ? 1 : 0;
  }
  if (pl.kind == MMM_KERNEL_STREAM || pl.kind == MMM_KERNEL_TILE_STREAM) {
    GemmProblem pr = p;
    pr.M = M - pl.tile_rows;
    plan->stream_rows = pr.M;
    plan->stream_workgroups = skinny_workgroups(pr);
    plan->stream_splits = skinny_splits(pr);
    plan->stream_columns = skinny_columns(pr);
  }
  plan->workspace_bytes = (int64_t)plan_workspace_bytes(p, pl);
  return hipSuccess;
}

hipError_t mmm_gemm_workspace_f16f32(const mmm_half* A, const mmm_half* B, const float* C, int M, int N, int K,
                                     int64_t lda, int64_t ldb, int64_t ldc, size_t* bytes) {
  if (!bytes) return hipErrorInvalidValue;
  mmm_gemm_plan plan;
  const hipError_t e = mmm_gemm_plan_f16f32(A, B, C, M, N, K, lda, ldb, ldc, &plan);
  *bytes = e == hipSuccess ? (size_t)plan.workspace_bytes : 0;
  return e;
}

hipError_t mmm_gemm_f16f32_tiled(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                 int64_t lda, int64_t ldb, int64_t ldc, int wave_m, int wave_n, int waves_i,
                                 int waves_j, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int tile = tile_from_params(wave_m, wave_n, waves_i, waves_j);
  if (tile < 0) return hipErrorInvalidValue;
  hipError_t e = check_gemm(A, B, C, M, N, K, lda, ldb, ldc);
  if (e != hipSuccess || M == 0 || N == 0) return e;
  if ((e = check_workspace(workspace)) != hipSuccess) return e;
  if (K == 0) return launch_zero_f32(C, M, N, ldc, stream);
  GemmProblem p{A, B, C, M, N, K, lda, ldb, ldc, false, false};
  p.ws = (float*)workspace;
  p.ws_bytes = workspace ? workspace_bytes : 0;
  p.ws_absent = workspace == nullptr;
  return launch_gemm_nn(p, tile, stream);
}

hipError_t mmm_contract_desc_baseline(mmm_contract_desc* d, int b, int i, int k, int l, int j) {
  if (!d || b < 0 || i < 0 || k < 0 || l < 0 || j < 0) return hipErrorInvalidValue;
  // A[b,i,k,l]: m = (b, i), k = (k, l).  B[k,l,j]: n = (1, j).  C[b,i,j].
  *d = mmm_contract_desc{};
  d->m_ext[0] = b, d->m_ext[1] = i;
  d->k_ext[0] = k, d->k_ext[1] = l;
  d->n_ext[0] = 1, d->n_ext[1] = j;
  d->a_m_stride[0] = (int64_t)i * k * l, d->a_m_stride[1] = (int64_t)k * l;
  d->a_k_stride[0] = l, d->a_k_stride[1] = 1;
  d->b_k_stride[0] = (int64_t)l * j, d->b_k_stride[1] = j;
  d->b_n_stride[0] = j, d->b_n_stride[1] = 1;
  d->c_m_stride[0] = (int64_t)i * j, d->c_m_stride[1] = j;
  d->c_n_stride[0] = j, d->c_n_stride[1] = 1;
  return hipSuccess;
}

hipError_t mmm_contract_desc_reference(mmm_contract_desc* d, int mt, int bt, int rt, int nt, int rt_l) {
  if (!d || mt < 0 || bt < 0 || rt < 0 || nt < 0 || rt_l < 0) return hipErrorInvalidValue;
  // G[r][n][m][l] as A(m', k') with m' = (m, r), k' = (n, l)          (mmmTensor.cpp:329-340)
  // Input[b][n][l] as B(k', b): k' = (n, l) contiguous, n = b          (mmmTensor.cpp:168)
  // Out[m][b][r] as C(m', b)                                           (mmmTensor.cpp:251)
  *d = mmm_contract_desc{};
  d->m_ext[0] = mt, d->m_ext[1] = rt;
  d->k_ext[0] = nt, d->k_ext[1] = rt_l;
  d->n_ext[0] = 1, d->n_ext[1] = bt;
  d->a_m_stride[0] = rt_l, d->a_m_stride[1] = (int64_t)nt * mt * rt_l;
  d->a_k_stride[0] = (int64_t)mt * rt_l, d->a_k_stride[1] = 1;
  d->b_k_stride[0] = rt_l, d->b_k_stride[1] = 1;
  d->b_n_stride[0] = (int64_t)bt * nt * rt_l, d->b_n_stride[1] = (int64_t)nt * rt_l;
  d->c_m_stride[0] = (int64_t)bt * rt, d->c_m_stride[1] = 1;
  d->c_n_stride[0] = (int64_t)bt * rt, d->c_n_stride[1] = rt;
  return hipSuccess;
}

hipError_t mmm_contract5d_f16f32(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, float* C,
                                 hipStream_t stream) {
  return mmm_contract5d_f16f32_ws(d, A, B, C, nullptr, 0, stream);
}

hipError_t mmm_contract5d_f16f32_ws(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, float* C,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  FoldProblem p{};
  hipError_t e = fold_from_desc(d, A, B, C, &p);
  if (e != hipSuccess || p.M == 0 || p.N == 0) return e;
  if (!C) return hipErrorInvalidValue;
  if ((e = check_workspace(workspace)) != hipSuccess) return e;
  // A fold that is a plain row-major GEMM runs on the GEMM kernels (the benchmark's
  // A[b,i,k,l] x B[k,l,j] -> C[b,i,j] is one: M = b*i, K = k*l, N = j).
  int64_t lda, ldb, ldc;
  if (plain_gemm(d, p.K, p.N, &lda, &ldb, &ldc))
    return mmm_gemm_f16f32_ws(A, B, C, p.M, p.N, p.K, lda, ldb, ldc, workspace, workspace_bytes, stream);
  if (p.K == 0) return launch_zero_fold(p, stream);
  return launch_gemm_fold(p, stream);  // the folded kernels split nothing: no workspace
}

hipError_t mmm_contract5d_workspace_f16f32(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B,
                                           const float* C, size_t* bytes) {
  if (!bytes) return hipErrorInvalidValue;
  *bytes = 0;
  FoldProblem p{};
  // only alignment matters here; null stands for a 256-byte-aligned buffer
  const mmm_half* a = A ? A : (const mmm_half*)(uintptr_t)256;
  const mmm_half* b = B ? B : (const mmm_half*)(uintptr_t)256;
  float* c = C ? (float*)C : (float*)(uintptr_t)256;
  hipError_t e = fold_from_desc(d, a, b, c, &p);
  if (e != hipSuccess || p.M == 0 || p.N == 0) return e;
  int64_t lda, ldb, ldc;
  if (!plain_gemm(d, p.K, p.N, &lda, &ldb, &ldc)) return hipSuccess;
  return mmm_gemm_workspace_f16f32(a, b, c, p.M, p.N, p.K, lda, ldb, ldc, bytes);
}

hipError_t mmm_gemm_naive_f16f32(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                                 int64_t ldb, int64_t ldc, hipStream_t stream) {
  hipError_t e = check_gemm(A, B, C, M, N, K, lda, ldb, ldc);
  if (e != hipSuccess || M == 0 || N == 0) return e;
  if (K == 0) return launch_zero_f32(C, M, N, ldc, stream);
  return launch_check_fold(fold_of_gemm(A, B, C, M, N, K, lda, ldb, ldc), nullptr, nullptr, stream);
}

hipError_t mmm_gemm_truth_f64(const mmm_half* A, const mmm_half* B, double* T, double* S, int M, int N, int K,
                              int64_t lda, int64_t ldb, int64_t ldt, hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!T || (K > 0 && (!A || !B)) || lda < K || ldb < N || ldt < N) return hipErrorInvalidValue;
  return launch_check_fold(fold_of_gemm(A, B, nullptr, M, N, K, lda, ldb, ldt), T, S, stream);
}

hipError_t mmm_contract5d_truth_f64(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, double* T,
                                    double* S, hipStream_t stream) {
  FoldProblem p{};
  hipError_t e = fold_from_desc(d, A, B, nullptr, &p);
  if (e != hipSuccess || p.M == 0 || p.N == 0) return e;
  if (!T) return hipErrorInvalidValue;
  return launch_check_fold(p, T, S, stream);
}

hipError_t mmm_fill_uniform_f16(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, hipStream_t stream) {
  if (n < 0 || (n > 0 && !out)) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  return launch_fill_uniform(out, n, seed, tensor_id, stream);
}

hipError_t mmm_fill_normal_f16(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, double scale,
                               hipStream_t stream) {
  if (n < 0 || (n > 0 && !out)) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  return launch_fill_normal(out, n, seed, tensor_id, scale, stream);
}

hipError_t mmm_tile_of_block(int block, int tiles_m, int tiles_n, int* tm, int* tn) {
  if (!tm || !tn || tiles_m <= 0 || tiles_n <= 0) return hipErrorInvalidValue;
  if ((int64_t)tiles_m * tiles_n > 0x7fffffff) return hipErrorInvalidValue;
  if (block < 0 || block >= tiles_m * tiles_n) return hipErrorInvalidValue;
  tile_of_block(block, tiles_m, tiles_n, 4, tm, tn);
  return hipSuccess;
}

const char* mmm_version(void) { return "mmm-gfx950 0.1.0"; }

}  // extern "C"
