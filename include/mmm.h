/*
 * mmm.h -- C ABI of the MI355X (gfx950) FP16->FP32 GEMM and 5-D tensor contraction.
 *
 * Drop-in boundary for the hot path of thrasos-g/RDNA4-GEMM-WMMA.  The reference has no
 * library or FFI layer: its boundary is the kernel entry
 *     template<int WAVE_M,int WAVE_N,int WAVES_I,int WAVES_J>
 *     __global__ void WMMA_Swizzled_Full(_Float16* A, _Float16* B, float* C)   (mmm.cpp:1214-1215)
 * launched as <<<dim3(ceil(DIM_J/BLOCK_N), ceil(DIM_I/BLOCK_M)), dim3(32, WAVES_I*WAVES_J)>>>
 * on the null stream (mmm.cpp:1471-1472, 1488, 1496), with the problem size in the
 * compile-time globals DIM_I/DIM_J/DIM_K (mmm.cpp:13-15).  The entry points below keep that
 * shape -- device pointers, M/N/K and the tile template parameters -- and add what a real
 * boundary needs: run-time sizes and leading dimensions, a stream, and an error code.
 *
 * Conventions (all entry points):
 *  - fp16 tensors are passed as pointers to IEEE binary16 bit patterns (mmm_half).
 *  - Pointers are device pointers owned by the caller.  No entry point synchronises the host,
 *    exits the process or allocates memory at call time.  Loading the library does reserve
 *    memory: a 64 MiB device array (the K-split partials of mmm_gemm_f16f32_noalloc) on every
 *    GPU the process uses the library on, held until the process ends, whether or not that
 *    entry point is ever called.  Launches that would leave most of the chip idle
 *    split K across workgroups and sum the partials in a fixed order; the partials go to a
 *    workspace the caller passes to the _ws entry points (size from mmm_gemm_workspace_f16f32
 *    or mmm_contract5d_workspace_f16f32, at most 64 MiB).  Without one (the entry points
 *    without _ws, a null or too small workspace) the unsplit kernels run; results agree
 *    within rounding (the summation order differs).  Each choice is deterministic.
 *  - C is overwritten (alpha = 1, beta = 0, as mmm.cpp:1512-1513 and the kernel's store at
 *    mmm.cpp:1370); C is never read.
 *  - Errors: hipErrorInvalidValue for null pointers, negative sizes or leading dimensions
 *    smaller than the row length; a launch error is returned as the runtime reports it.
 *    M == 0 or N == 0 is a no-op; K == 0 writes zeros to C.
 *  - Work is enqueued on `stream` (0 = the null stream, as the reference) and is
 *    asynchronous, as the reference's launches are (the caller synchronises, mmm.cpp:1491).
 *  - Thread safety: the only mutable global state is mmm_gemm_f16f32_noalloc's: its 64 MiB
 *    device array (shared by every call of that entry point on one GPU) and a mutex-guarded
 *    table of the array's device address per GPU, filled on the first call on each GPU.  A
 *    workspace serves one call at a time: calls on one stream may share one (they are
 *    ordered); concurrent calls on different streams need their own.
 */
#ifndef MMM_H
#define MMM_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t mmm_half; /* IEEE binary16 bit pattern */

/*
 * C[M][N] (fp32, row-major, ldc) = A[M][K] (fp16, row-major, lda) * B[K][N] (fp16, row-major, ldb).
 * fp32 accumulation.  Leading dimensions are in elements.
 * Replaces: WMMA_Swizzled_Full<2,2,4,4><<<..>>>(dA, dB, dC) with DIM_I = M, DIM_J = N,
 * DIM_K = K (mmm.cpp:1461-1472, 1496) -- the templated lineage mmm.cpp:694-1374.  Unlike
 * the reference's unmasked kernel, any M, N, K and any leading dimensions are accepted
 * (the ragged shapes the tensor variant masks at mmmTensor.cpp:135-178, 246).
 */
hipError_t mmm_gemm_f16f32(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                           int64_t ldb, int64_t ldc, hipStream_t stream);

/*
 * As mmm_gemm_f16f32, with a caller-provided workspace for the K-split partial sums
 * (16-byte aligned; NULL allowed).  When workspace_bytes is at least what
 * mmm_gemm_workspace_f16f32 reports, shapes that would leave most of the chip idle (M <= 64,
 * small grids, an under-filled last round of tiles) split K across workgroups; otherwise they
 * run unsplit.  No reference counterpart: the reference's kernel never splits K and
 * allocates nothing (mmm.cpp:1214-1374).
 */
hipError_t mmm_gemm_f16f32_ws(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                              int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Measurement form of mmm_gemm_f16f32_ws: the same launch, and when it runs a matrix-core tile
 * kernel, thread 0 of its workgroup 0 writes clock[0] = shader-clock counter (s_memtime) and
 * clock[1] = 100 MHz real-time counter (s_memrealtime) at its start and clock[2], clock[3] at its
 * end (device memory, 8-byte aligned; NULL: nothing is written, exactly mmm_gemm_f16f32_ws).
 * The shader clock during the launch is (clock[2] - clock[0]) / (clock[3] - clock[1]) * 100 MHz.
 * Other kernels (M <= 64 streaming, K == 0) leave clock unwritten.  No reference counterpart:
 * it gives a benchmark the clock its own launches ran at, the MI355X clock falling under
 * sustained matrix-core load (power limit).
 */
hipError_t mmm_gemm_f16f32_clocked(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                   int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                                   uint64_t* clock, hipStream_t stream);

/*
 * As mmm_gemm_f16f32_ws, with the K-split partials in a 64 MiB array inside the library (one per
 * GPU, held until the process ends) instead of a caller's workspace: the entry point calls no
 * allocating routine.  No reference counterpart: it is for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The array serves the
 * current device; the first call on a device looks its address up (do that before a capture).
 * Results equal mmm_gemm_f16f32_ws's with a workspace of at least mmm_gemm_workspace_f16f32
 * bytes.  Returns hipErrorInvalidValue where mmm_gemm_f16f32_ws would, and when a planned split
 * needs more than the array holds (not reached by the planner's 64 MiB limit).  Every call on one
 * GPU shares its array: calls that overlap on one GPU (different streams) race on it.  The
 * looked-up address is kept for the life of the process: after hipDeviceReset (which frees the
 * device's copy of the array) this entry point must not be called on that device again.
 */
hipError_t mmm_gemm_f16f32_noalloc(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                   int64_t lda, int64_t ldb, int64_t ldc, hipStream_t stream);

/*
 * Workspace bytes mmm_gemm_f16f32_ws needs for these arguments (0: it would not split).
 * Host only, no GPU call; A, B, C only for their alignment and may be NULL (taken as
 * 256-byte aligned).  No reference counterpart (see mmm_gemm_f16f32_ws).
 */
hipError_t mmm_gemm_workspace_f16f32(const mmm_half* A, const mmm_half* B, const float* C, int M, int N, int K,
                                     int64_t lda, int64_t ldb, int64_t ldc, size_t* bytes);

/*
 * As mmm_gemm_f16f32, with the block tile chosen by the caller through the reference's
 * template parameters (mmm.cpp:694-695, 1462-1465): block tile = (WAVES_I*WAVE_M*32) x
 * (WAVES_J*WAVE_N*32), i.e. the parameters count 32x32 output blocks per wave and waves per
 * workgroup along M and N (the reference counts 16x16 WMMA tiles).  They select the block tile
 * only; each block tile's waves, MFMA shape and K step are the library's own:
 *   (4,4,2,2) 256x256 -- 8 waves (2 x 4) of 128x64, v_mfma_f32_16x16x32_f16, 64-deep K steps;
 *   (2,4,2,2) 128x256, (4,2,2,2) 256x128 -- 8 waves (2 x 4, 4 x 2) of 64x64, v_mfma_f32_16x16x32_f16,
 *             64-deep K steps;
 *   (2,2,2,2) 128x128 -- 8 waves (2 x 4) of 64x32, v_mfma_f32_16x16x32_f16, 64-deep K steps;
 *   (1,1,2,2) 64x64 -- 4 waves, v_mfma_f32_16x16x32_f16, 64-deep K steps;
 *   (3,3,2,2) 192x192 -- 8 waves (2 x 4) of 96x48, v_mfma_f32_16x16x32_f16, 64-deep K steps.
 * Those are the direct-to-LDS kernels.  Problems with odd (1-byte-aligned) fp16 addresses run
 * register-staged versions of 4 waves with v_mfma_f32_32x32x16_f16 (192x192: the 128x128 one).
 * Other parameter sets return hipErrorInvalidValue.  The workspace (NULL allowed) serves the
 * tile's K split as in mmm_gemm_f16f32_ws.
 */
hipError_t mmm_gemm_f16f32_tiled(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                 int64_t lda, int64_t ldb, int64_t ldc, int wave_m, int wave_n, int waves_i,
                                 int waves_j, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Kernels mmm_gemm_f16f32 can launch (mmm_gemm_plan.kernel). */
#define MMM_KERNEL_NONE 0        /* M == 0 or N == 0: nothing */
#define MMM_KERNEL_ZERO 1        /* K == 0: C = 0 */
#define MMM_KERNEL_TILE 2        /* matrix-core tile kernel over all of C */
#define MMM_KERNEL_STREAM 3      /* M <= 64: HBM-streaming kernel */
#define MMM_KERNEL_TILE_STREAM 4 /* tile kernel on the first tile_rows rows, streaming kernel on the rest */

typedef struct mmm_gemm_plan {
    int kernel;                            /* MMM_KERNEL_* */
    int wave_m, wave_n, waves_i, waves_j;  /* tile kernel, as mmm_gemm_f16f32_tiled takes it (0 if none) */
    int block_m, block_n;                  /* its block tile */
    int direct_to_lds;                     /* 1: operands stream HBM -> LDS directly; 0: staged in registers */
    int tile_rows, stream_rows;            /* rows of C on each kernel */
    int64_t tile_workgroups, stream_workgroups;
    int stream_splits;                     /* K ranges of the streaming kernel reduced across
                                              workgroups (0: split among one workgroup's waves) */
    int tile_splits;                       /* K ranges of the tile kernel (1: no split); a split
                                              launch is followed by an ordered reduction kernel */
    int tile_split_tiles;                  /* tiles that run as tile_splits K ranges: the last,
                                              partly filled round of 256 workgroups (all tiles
                                              when the grid is one small round); 0: none */
    int tile_persistent;                   /* 1: 256 workgroups each loop over tiles (whole
                                              interior tiles over several rounds) */
    int64_t workspace_bytes;               /* workspace the splits need (mmm_gemm_f16f32_ws);
                                              the split counts above assume it is given, and so
                                              does the kernel choice for M <= 64: without a
                                              workspace, aligned problems whose 128-column strips
                                              fill rounds of 256 workgroups less than 1/1.8 run
                                              on the streaming kernel, not on tiles */
    int stream_columns;                    /* columns of C per streaming workgroup: 32 (K split
                                              among one workgroup's waves), 128, or 256 (long
                                              K streams); 0: no streaming kernel */
} mmm_gemm_plan;

/*
 * The launch mmm_gemm_f16f32 makes for these arguments, without launching (host only; no GPU
 * call).  A, B, C are used only for their alignment and may be NULL (taken as 256-byte
 * aligned).  No reference counterpart: the reference fixes one tile, <2,2,4,4>, for every
 * size (mmm.cpp:1462-1465); this exposes the size-dependent choice that replaces it.
 */
hipError_t mmm_gemm_plan_f16f32(const mmm_half* A, const mmm_half* B, const float* C, int M, int N, int K,
                                int64_t lda, int64_t ldb, int64_t ldc, mmm_gemm_plan* plan);

/*
 * 5-D tensor contraction descriptor.  Each GEMM axis (m, n, k) is a pair of sub-indices
 * (hi, lo), folded as  m = m_hi * m_ext[1] + m_lo  (same for n and k), and each operand
 * gives an element stride for every sub-index it carries:
 *   A(m, k) = A[m_hi*a_m_stride[0] + m_lo*a_m_stride[1] + k_hi*a_k_stride[0] + k_lo*a_k_stride[1]]
 *   B(k, n) = B[k_hi*b_k_stride[0] + k_lo*b_k_stride[1] + n_hi*b_n_stride[0] + n_lo*b_n_stride[1]]
 *   C(m, n) = C[m_hi*c_m_stride[0] + m_lo*c_m_stride[1] + n_hi*c_n_stride[0] + n_lo*c_n_stride[1]]
 *   C(m, n) = sum_k A(m, k) * B(k, n)   (fp32 accumulate, overwrite)
 * The fold and any index permutation are applied in the kernels' address generation; no
 * operand is repacked or transposed in memory.
 */
typedef struct mmm_contract_desc {
    int64_t m_ext[2], n_ext[2], k_ext[2];
    int64_t a_m_stride[2], a_k_stride[2];
    int64_t b_k_stride[2], b_n_stride[2];
    int64_t c_m_stride[2], c_n_stride[2];
} mmm_contract_desc;

/*
 * Descriptor for C[b,i,j] = sum_{k,l} A[b,i,k,l] * B[k,l,j], all dense in the listed index
 * order: m = (b, i), k = (k, l), n = j.  This is the contraction of the benchmark
 * configuration; the reference has no such preset (its only contraction is the one below).
 */
hipError_t mmm_contract_desc_baseline(mmm_contract_desc* d, int b, int i, int k, int l, int j);

/*
 * Descriptor for the reference's contraction (mmmTensor.cpp:20-28):
 *   Out[m][b][r] = sum_{n,l} G[r][n][m][l] * Input[b][n][l]
 * with G [rt][nt][mt][rt_l], Input [bt][nt][rt_l], Out [mt][bt][rt]:  GEMM m = (m, r),
 * k = (n, l), n = b.  This replaces the reference's host pack of G (mmmTensor.cpp:329-340),
 * its TN read of Input (mmmTensor.cpp:168) and its output remap (mmmTensor.cpp:246-252).
 */
hipError_t mmm_contract_desc_reference(mmm_contract_desc* d, int mt, int bt, int rt, int nt, int rt_l);

/*
 * Runs the contraction described by d.  Replaces the tensor variant
 * WMMA_Swizzled_Full<2,2,4,4><<<..>>>(dA, d_Input, d_Output) (mmmTensor.cpp:44-257, launch
 * mmmTensor.cpp:354-371) together with the host pack it needs (mmmTensor.cpp:329-343).
 */
hipError_t mmm_contract5d_f16f32(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, float* C,
                                 hipStream_t stream);

/*
 * As mmm_contract5d_f16f32, with a caller-provided workspace (as mmm_gemm_f16f32_ws; a fold
 * that is a plain row-major GEMM runs on the GEMM kernels and may split K), and the bytes it
 * needs (host only; pointers only for alignment, may be NULL).  No reference counterpart
 * (the reference's tensor kernel never splits K, mmmTensor.cpp:44-257).
 */
hipError_t mmm_contract5d_f16f32_ws(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, float* C,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream);
hipError_t mmm_contract5d_workspace_f16f32(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B,
                                           const float* C, size_t* bytes);

/*
 * On-device cross-check: the reference's GEMM_Naive (mmm.cpp:52-62) with run-time sizes and
 * leading dimensions.  One fp32 accumulator per output, k ascending, acc += float(a)*float(b);
 * the result is bit-identical to that loop run on a CPU.  SIMT only; slow by design.
 */
hipError_t mmm_gemm_naive_f16f32(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K, int64_t lda,
                                 int64_t ldb, int64_t ldc, hipStream_t stream);

/*
 * fp64 ground truth for validating a full-size output: T[i][j] = sum_k a*b and, when S is not
 * NULL, S[i][j] = sum_k |a*b| (both fp64, k ascending; T and S share the leading dimension
 * ldt).  An fp32 result C is within tolerance when |C - T| <= rel * S.  No reference
 * counterpart: it takes the place of the reference's rocBLAS comparison
 * (mmm.cpp:1387-1407, 1519-1545; mmmTensor.cpp:278-306, 393-420).
 */
hipError_t mmm_gemm_truth_f64(const mmm_half* A, const mmm_half* B, double* T, double* S, int M, int N, int K,
                              int64_t lda, int64_t ldb, int64_t ldt, hipStream_t stream);

/* The same for a contraction: T and S are written at the offsets d gives C. */
hipError_t mmm_contract5d_truth_f64(const mmm_contract_desc* d, const mmm_half* A, const mmm_half* B, double* T,
                                    double* S, hipStream_t stream);

/*
 * Seeded synthetic inputs, generated on the device (the reference fills with unseeded
 * rand()/RAND_MAX on the host, mmm.cpp:1409-1414; these are reproducible instead):
 *   key = splitmix64(seed * 0x9E3779B97F4A7C15 + tensor_id + 1), x_i = splitmix64(key + i)
 *   uniform: (x_i >> 40) * 2^-23 - 1  in [-1, 1), rounded to fp16 (RNE)
 *   normal:  Box-Muller on x_{2i}, x_{2i+1} in fp64, times scale, rounded to fp16 (RNE)
 */
hipError_t mmm_fill_uniform_f16(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, hipStream_t stream);
hipError_t mmm_fill_normal_f16(mmm_half* out, int64_t n, uint64_t seed, uint32_t tensor_id, double scale,
                               hipStream_t stream);

/*
 * Host-side query of the tile scheduler: the output tile (tm, tn) computed by workgroup
 * `block` of a launch with tiles_m x tiles_n tiles.  Lets callers and tests check that every
 * tile is computed exactly once (the reference's remap, mmm.cpp:1219-1236, is not a
 * bijection for every grid).  Returns hipErrorInvalidValue for out-of-range arguments.
 */
hipError_t mmm_tile_of_block(int block, int tiles_m, int tiles_n, int* tm, int* tn);

/*
 * Measurement probes.  No reference counterpart: the reference reports only milliseconds and
 * GFLOPS (mmm.cpp:1503-1504; mmmTensor.cpp:434-436).  They give the kernels' roofline
 * fractions a measured denominator beside the published peaks, since the MI355X clock falls
 * under sustained matrix-core load (power limit).
 *
 * mmm_probe_clock: one wave spins for `ticks` ticks (1 .. 10^7) of the constant 100 MHz
 *   real-time counter and writes out[0] = shader-clock cycles elapsed, out[1] = real-time
 *   ticks elapsed (shader clock = out[0] / out[1] * 100 MHz).
 * mmm_probe_mfma_ceiling: the persistent 256x256 tile kernel's MFMA stream (256 workgroups x
 *   8 waves, 8 x 4 v_mfma_f32_16x16x32_f16 per wave per 32-deep K-step, over every tile and all
 *   of K: 2*M*N*K flops) with the operands held in registers -- no operand loads, LDS or
 *   barriers.  A [M][K] and B [K][N] are contiguous row-major inputs whose first K-steps supply
 *   the fragments; store_tiles != 0 writes each tile's accumulators to C [M][N] as the tile
 *   kernel does, store_tiles == 0 writes one float per thread into C's first 256 * 512 floats.
 *   The values written are not A*B.  M, N multiples of 256, K of 64.  clock (NULL allowed)
 *   receives workgroup 0's start and end counters as mmm_gemm_f16f32_clocked writes them.
 * mmm_probe_lds_mfma: the same kernel's K loop on operands already in LDS.  Each of
 *   min(M/256 * N/256, 256) workgroups stages K tiles 0 and 1 of its first 256x256 tile of A
 *   [M][K] and B [K][N] (contiguous row-major, 16-byte aligned) into the kernel's two LDS ring
 *   slots once, then runs the kernel's fragment reads and MFMAs for every K tile of its share of
 *   the tiles (2*M*N*K flops in all), alternating the two slots, without operand loads or C
 *   stores; barrier != 0 keeps the kernel's one workgroup barrier per K tile.  out (out_floats
 *   floats, at least min(M/256 * N/256, 256) * 512) receives one float per thread: thread t of
 *   workgroup g writes out[g * 512 + t], the
 *   sum of its accumulators; a workgroup's outputs sum to (tiles * K / 128) * (1^T A0)(B0 1),
 *   tiles its number of output tiles, A0 and B0 its first tile's rows of A and columns of B
 *   over K 0 .. 127.  M, N multiples of 256, K of 128.  clock as for mmm_probe_mfma_ceiling.
 * mmm_probe_read: streams `bytes` (a multiple of 1024, 16-byte-aligned src) once over 8192
 *   workgroups: with plain non-temporal 16-byte loads into registers (direct_to_lds == 0; out
 *   receives 8192 * 256 words), or with the tile kernels' direct-to-LDS loads into 32-slot rings
 *   (direct_to_lds != 0, bytes < 2^31; out receives 8192 words).
 */
hipError_t mmm_probe_clock(uint64_t* out, int64_t ticks, hipStream_t stream);
hipError_t mmm_probe_mfma_ceiling(const mmm_half* A, const mmm_half* B, float* C, int M, int N, int K,
                                  int store_tiles, uint64_t* clock, hipStream_t stream);
hipError_t mmm_probe_lds_mfma(const mmm_half* A, const mmm_half* B, float* out, int64_t out_floats, int M, int N,
                              int K, int barrier, uint64_t* clock, hipStream_t stream);
hipError_t mmm_probe_read(const void* src, int64_t bytes, int direct_to_lds, uint32_t* out, int64_t out_words,
                          hipStream_t stream);

/* Library version string. */
const char* mmm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MMM_H */
