// Internal launch interface shared by the kernel sources and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mmm.h"

namespace mmm {

// Plain row-major problem: C[M][N] (ldc) = A[M][K] (lda) * B[K][N] (ldb).
struct GemmProblem {
  const mmm_half* A;
  const mmm_half* B;
  float* C;
  int M, N, K;
  int64_t lda, ldb, ldc;
  bool c_vec4;     // set by the launcher: C 4-byte aligned (16-byte stores of C rows allowed)
  bool tail_regs;  // set by the launcher: the last K tile needs masking (K or N not a multiple
                   // of 8, or rows not 16-byte aligned): patched chunks or a VGPR gather
  int k_splits;    // tile kernel: K ranges computed by separate workgroups (<= 1: none)
  int split_tiles; // k_splits > 1: the last split_tiles tiles in dispatch order are split
  float* partials; // k_splits > 1: [split tile][split][BM][BN] fp32 partial tiles
  float* ws;       // caller's workspace for K splits (16-byte aligned), or null: no split
  size_t ws_bytes; // its size
  uint64_t* clk;   // null, or 4 counters workgroup 0 of a tile kernel writes: shader clock and
                   // real-time counter at its start, then at its end (measurement only)
  bool ws_absent;  // the call has no workspace at all (not set by the plan query, which assumes
                   // one): the tile kernels' K split is unavailable when choosing kernels
};

// Folded problem (the 5-D contraction descriptor, see mmm.h), with int32 extents.
struct FoldProblem {
  const mmm_half* A;
  const mmm_half* B;
  float* C;
  int M, N, K;
  int m_lo, n_lo, k_lo;  // extents of the low sub-index of each axis
  int64_t am[2], ak[2];  // A strides for (m_hi, m_lo), (k_hi, k_lo)
  int64_t bk[2], bn[2];  // B strides for (k_hi, k_lo), (n_hi, n_lo)
  int64_t cm[2], cn[2];  // C strides for (m_hi, m_lo), (n_hi, n_lo)
};

enum TileId { kTile256x256 = 0, kTile128x256 = 1, kTile256x128 = 2, kTile128x128 = 3, kTile64x64 = 4, kTile192x192 = 5 };
constexpr int kTileCount = 6;
// Block tile of each TileId (rows x columns of C).
constexpr int tile_bm(int tile) {
  return tile == kTile256x256 || tile == kTile256x128 ? 256 : tile == kTile64x64 ? 64 : tile == kTile192x192 ? 192 : 128;
}
constexpr int tile_bn(int tile) {
  return tile == kTile256x256 || tile == kTile128x256 ? 256 : tile == kTile64x64 ? 64 : tile == kTile192x192 ? 192 : 128;
}

// Effective rate of a K split's partial-tile traffic (written by the split workgroups, read back
// with C written by the reduction), as the tile planner prices it.  The partials of an
// under-filled round (tens of MB) are read back from the 256 MB Infinity Cache: fitted to the
// measured times of split launches on MI355X (2304^2 x 8192 on 256x256 tiles: 90 us measured).
constexpr double kSplitTrafficBps = 10e12;

hipError_t launch_gemm_nn(const GemmProblem& p, int tile_id, hipStream_t stream);
bool gemm_nn_direct_to_lds(const GemmProblem& p, int tile_id);  // else the register-staged path
// K split of a tile launch: the last `tiles` tiles in dispatch order (the last, partly filled
// round of 256 workgroups, or the whole grid when it is one small round) each run as `splits`
// K ranges; splits == 1: none.
struct TileSplit {
  int splits, tiles;
};
TileSplit gemm_nn_split(const GemmProblem& p, int tile_id);
int gemm_nn_splits(const GemmProblem& p, int tile_id);  // gemm_nn_split(...).splits
bool gemm_nn_persistent(const GemmProblem& p, int tile_id);  // launch as the persistent kernel
// Workspace bytes a tile launch's K split needs (0: no split).  Launches split only when the
// caller's workspace (GemmProblem::ws) holds that much; splits are planned within
// kMaxWorkspaceBytes.
size_t gemm_nn_workspace_bytes(const GemmProblem& p, int tile_id);
constexpr size_t kMaxWorkspaceBytes = (size_t)64 << 20;
hipError_t launch_gemm_fold(const FoldProblem& p, hipStream_t stream);
// The operand-path probe (lds_mfma_probe_kernel): M, N multiples of 256, K of 128, row-major A
// and B 16-byte aligned (lda = K, ldb = N); out holds min(M/256 * N/256, 256) * 512 floats.
hipError_t launch_lds_mfma_probe(const GemmProblem& p, bool barrier, float* out, hipStream_t stream);
// Rows of C up to which the streaming kernels take a GEMM (the kernels handle up to 64).
constexpr int kStreamMaxRows = 64;
static_assert(kStreamMaxRows >= 16 && kStreamMaxRows <= 64, "streaming kernels take 16 to 64 rows");
bool skinny_ok(const GemmProblem& p);  // M <= kStreamMaxRows and operands within 32-bit offsets
hipError_t launch_gemm_skinny(const GemmProblem& p, hipStream_t stream);
int skinny_workgroups(const GemmProblem& p);
int skinny_splits(const GemmProblem& p);  // K ranges reduced across workgroups (0: within one)
int skinny_columns(const GemmProblem& p);  // columns of C per workgroup strip (32, 128, 256)
bool skinny_tiles_faster(const GemmProblem& p);   // 33-64 rows on short, many-strip grids: tiles win
bool skinny_prefers_tiles(const GemmProblem& p);  // several rounds of strips that the tile kernels run faster
size_t skinny_workspace_bytes(const GemmProblem& p);  // workspace its split needs (0: none)
hipError_t launch_fill_uniform(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, hipStream_t stream);
hipError_t launch_fill_normal(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, double scale,
                              hipStream_t stream);
hipError_t launch_zero_f32(float* C, int M, int N, int64_t ldc, hipStream_t stream);
hipError_t launch_zero_fold(const FoldProblem& p, hipStream_t stream);
// Cross-check kernels: fp32 ascending-k accumulation into p.C when T is null, else fp64
// T = sum a*b and (S non-null) S = sum |a*b|, both at p's C offsets.
hipError_t launch_check_fold(const FoldProblem& p, double* T, double* S, hipStream_t stream);

}  // namespace mmm
