// MI355X (gfx950, CDNA4, wave64) FP16->FP32 GEMM kernels.
//
// Computes C[M][N] = A[M][K] * B[K][N] (fp16 in, fp32 accumulate and out, row-major), the
// operation of the reference's templated WMMA lineage (mmm.cpp:694-1374; definition at
// mmm.cpp:52-62).  The design is CDNA4's own, not a translation of the RDNA4 kernel:
//
//  * Math: v_mfma_f32_32x32x16_f16 (one wave, 32x32 outputs, K 16 per instruction).  The
//    MFMA operands are issued swapped (B fragment as src A, A fragment as src B), so the
//    accumulator holds C^T: lane l owns row m = l%32 and, for accumulator v, column
//    n = 8*(v/4) + 4*(l/32) + v%4 -- four consecutive columns per lane, stored as float4.
//  * Block tile BM x BN with K step 64, WGM x WGN waves, each wave (BM/WGM) x (BN/WGN).
//    The default 256x256 tile with 2x2 waves gives every wave 4x4 MFMA tiles (256 fp32
//    accumulators, held in AGPRs), i.e. 32 MACs per LDS byte read -- twice what the
//    MFMA rate needs from LDS.
//  * Operand staging: HBM -> LDS by buffer_load_dwordx4 ... lds (direct to LDS, no VGPR
//    round trip), double-buffered (2 x 64 KB of the 160 KB LDS).  Out-of-range rows and
//    the K tail read as zero through the buffer descriptor's range check.
//  * LDS layouts and swizzles (16-byte chunks, chosen for CDNA4's 64-bank LDS):
//      A stage [BM][64] fp16, row = 8 chunks, chunk c of row m at c ^ fA(m),
//          fA(m) = (m & 7) ^ ((m >> 3) & 3): 16 consecutive rows at one chunk hit 16
//          distinct 16-byte bank groups (ds_read_b128 conflict-free).
//      B stage [64][BN] fp16 (N contiguous, as in HBM), chunk c of row k at c ^ gB(k & 3),
//          gB = {0, 6, 10, 12}: the 4 rows x 4 chunks that 32 lanes of one
//          ds_read_b64_tr_b16 touch land in 16 distinct bank groups.
//    The A fragment is one ds_read_b128 (8 consecutive k of one row).  The B fragment needs
//    8 consecutive k of one column of an N-contiguous tile: two ds_read_b64_tr_b16, which
//    transpose 4x16 blocks across each 16-lane group (lane i receives column i of the 4
//    rows that lanes 4e + i/4 address).
//  * Workgroup -> tile: XCD-aware, L2-grouped bijection (mmm_tile_map.h).
//
// A second instantiation of the same kernel ("generic") stages through VGPRs with
// element-wise masked loads; it serves leading dimensions or pointers that are not
// 16-byte aligned (e.g. the ragged 4097 x 4095 x 4111 configuration) and arbitrary K.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mmm.h"
#include "mmm_dma.h"
#include "mmm_kernels.h"
#include "mmm_tile_map.h"

namespace mmm {

// Fragment offsets a wave keeps per K-step (A) or per B fragment: at most kMaxOff of each.
constexpr int kMaxOff = 8;


// Block tile BM x BN, K step BK (32 or 64), WGM x WGN waves, STAGES-deep LDS ring, OCC
// workgroups per CU targeted by the launch bounds (OCC > 1 caps registers accordingly), MFMA
// shape MF: 32 = v_mfma_f32_32x32x16_f16, 16 = v_mfma_f32_16x16x32_f16 (same MACs per LDS byte;
// a quarter of the accumulator bytes per instruction for half the MACs).
template <int BM_, int BN_, int WGM_, int WGN_, int BK_, int STAGES_, int OCC_ = 1, int MF_ = 32>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_, STAGES = STAGES_, OCC = OCC_;
  static constexpr int MF = MF_;
  static constexpr int NT = 64 * WGM * WGN;
  static constexpr int TM = BM / WGM, TN = BN / WGN;
  static constexpr int FM = TM / MF, FN = TN / MF;
  static constexpr int KK = MF == 32 ? 16 : 32;  // K per MFMA
  static constexpr int KSTEPS = BK / KK;         // MFMA K-steps per stage
  static constexpr int CA = BK / 8;       // 16-byte chunks per A row
  static constexpr int CB = BN / 8;       // 16-byte chunks per B row
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int RA = BM * CA / NT;  // A chunks per thread per stage
  static constexpr int RB = BK * CB / NT;  // B chunks per thread per stage
  static constexpr int LPT = RA + RB;      // direct-to-LDS loads per thread per stage
  // A-row swizzle (chunk c of row m stored at c ^ swz_a(m)).  32x32 fragments, rows of 128 B
  // (BK = 64): 8 consecutive rows take 8 distinct chunk slots and 16 consecutive rows 16
  // distinct 16-byte bank groups of the 256-byte bank window.  Rows of 64 B (BK = 32): four
  // rows share a 256-byte window, so the swizzle uses row bits 1..3.  Both are conflict-free
  // for the 32x32 fragment reads (measured).
  // 16x16 fragments (BK = 64): each ds_read_b128 reads 16 consecutive rows at four logical
  // chunks; row bits 1..3 as the chunk swizzle make it conflict-free (measured with
  // SQ_LDS_BANK_CONFLICT on MI355X: the 32x32 swizzle costs this pattern a 2-way conflict).
  static __device__ __forceinline__ int swz_a(int m) {
    if constexpr (MF == 16) return (m >> 1) & 7;
    else if constexpr (BK == 64) return (m & 7) ^ ((m >> 3) & 3);
    else return ((m >> 1) & 3) ^ ((m >> 3) & 1);
  }
  static constexpr int SWZ_A_ROWS = MF == 16 ? 16 : BK == 64 ? 32 : 16;  // swz_a depends on m % SWZ_A_ROWS
  // A fragment offsets per K-step: 16-row fragments alternate between two swizzle phases when
  // the swizzle spans 32 rows; fragment mb sits (mb / APAR) * AROWS rows past phase mb % APAR.
  static constexpr int APAR = (MF == 16 && SWZ_A_ROWS == 32) ? 2 : 1;
  static constexpr int AROWS = APAR * MF;
  // B-row swizzle (chunk c of row k stored at c ^ swz_bk(k)).  32x32 fragments: {0, 6, 10, 12}
  // by k % 4 (the 4 rows x 4 chunks that 32 lanes of one ds_read_b64_tr_b16 touch land in 16
  // distinct bank groups).  16x16 fragments: those 32 lanes read rows k .. k+3 and k+8 .. k+11
  // (2 chunks each), so rows with bit 3 set also flip chunk bit 1 ({2, 4, 8, 14}).
  static __device__ __forceinline__ int swz_bk(int k) {
    if constexpr (CB == 8 || CB == 24) {
      // Rows of 128 or 384 B (BN = 64, 192): rows k and k+1 start half a 256-byte bank window
      // apart, so {0, 0, 4, 4} by k % 4 puts rows k..k+3 on the four distinct 64-byte quarters
      // of their windows; 16x16 fragments read rows k and k+8 at the same two chunks, so bit 3
      // of k flips chunk bit 1 as for wider rows.  XOR values below 8 keep every chunk inside
      // its group of 8, so a 24-chunk row stays a permutation of itself.
      const int s = (k & 2) << 1;
      if constexpr (MF == 16) return s ^ (((k >> 3) & 1) << 1);
      else return s;
    }
    const int s = (0xCA60 >> (4 * (k & 3))) & 15;
    if constexpr (MF == 16) return s ^ (((k >> 3) & 1) << 1);
    else return s;
  }
  static constexpr int SWZ_B_ROWS = MF == 16 ? 16 : 4;  // swz_bk depends on k % SWZ_B_ROWS
  static_assert(MF == 32 || (MF == 16 && BK == 64), "MFMA shape (16x16 fragments with 64-deep stages)");
  static_assert(BK == 32 || BK == 64, "K step must be 32 or 64");
  static_assert(TM % 32 == 0 && (TN % 32 == 0 || (MF == 16 && TN % 16 == 0)),
                "wave tile must be a multiple of 32x32 (32 x 16 with 16x16 fragments)");
  static_assert(FN <= kMaxOff && KSTEPS * APAR <= kMaxOff, "fragment offsets per wave");
  static_assert(CB == 8 || CB == 24 || CB >= 16, "B swizzle: rows of 8 or 24 chunks or at least 16");
  // B staging: chunk slot s = r*NT + w*64 + lane of a stage's [BK][CB] chunk grid is row s / CB.
  // When CB divides 64, a wave's slots are whole rows and rows advance by NT / CB per r; if that
  // step is also a multiple of the rows the B swizzle depends on, the logical chunk is the same
  // for every r (one base offset plus a uniform step per r).  Otherwise (BN = 192; four waves
  // over 32-chunk rows, 8 rows per round against a 16-row swizzle) each r has its own row and chunk.
  static constexpr bool B_UNIFORM = 64 % CB == 0 && (NT / CB) % SWZ_B_ROWS == 0;
  static_assert((BM * CA) % NT == 0 && (BK * CB) % NT == 0, "chunks must divide evenly over threads");
  static_assert(STAGES >= 2 && OCC * STAGES * STAGE <= 160 * 1024, "LDS rings must fit the 160 KB LDS");
};

// B-row swizzle of the 32x32 layouts (chunk c of row k stored at c ^ swz_b(k)), {0, 6, 10, 12}
// by k % 4.
__device__ __forceinline__ int swz_b(int k) { return (0xCA60 >> (4 * (k & 3))) & 15; }

__device__ __forceinline__ half8 lds_read_a(const char LDS_AS* p) { return *(const half8 LDS_AS*)p; }

__device__ __forceinline__ half8 lds_read_b_tr(const char LDS_AS* p_lo, const char LDS_AS* p_hi) {
  fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)p_lo);
  fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)p_hi);
  half4 l4 = __builtin_bit_cast(half4, lo);
  half4 h4 = __builtin_bit_cast(half4, hi);
  return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Wait until at most n tiles of LPT loads each are still in flight (0 <= n <= NMAX; n is
// wave-uniform, the branch is scalar).
template <int LPT, int NMAX>
__device__ __forceinline__ void wait_tiles(int n) {
  static_assert(NMAX * LPT <= 63, "vmcnt range");
  if constexpr (NMAX == 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= NMAX)
      wait_vmcnt<NMAX * LPT>();
    else
      wait_tiles<LPT, NMAX - 1>(n);
  }
}

// One pass over an LDS stage: KSTEPS K-steps of FM x FN MFMAs.  `after_first_reads` runs
// once the first K-step's fragment reads are issued (the DMA of a later stage goes there,
// so the MFMA pipe is fed before the loads are queued).
// BKM = false: B stage is [BK][BN] (N contiguous), fragments by two transposing reads;
//              b_off[nb] addresses fragment nb, K-steps add whole rows.
// BKM = true : B stage is [BN][BK] (K contiguous, swizzled like A), fragments by one
//              ds_read_b128; b_off[kk] addresses K-step kk, fragments add 32 rows.
// One K-step's MFMA operands for a wave: FM A fragments and FN B fragments.
template <class T>
struct Frags {
  half8 a[T::FM], b[T::FN];
};

// Accumulator of one MF x MF output block (C^T: lane l owns row m = l % MF).
template <class T>
using AccT = typename std::conditional<T::MF == 32, f32x16, f32x4>::type;

// Fragment read unit u of K-step kk: u < FM reads A fragment u; otherwise B fragment u - FM,
// by one ds_read_b128 from a K-major B stage (BKM) or two transposing reads from an
// N-contiguous one.  a_off[kk * APAR + phase]: A fragment offsets; b_off[nb] (N-contiguous
// B) or b_off[kk * APAR + phase] (K-major B, laid out and swizzled like A).
template <class T, bool BKM>
__device__ __forceinline__ void load_frag_unit(const char LDS_AS* a_st, const char LDS_AS* b_st,
                                               const uint32_t (&a_off)[kMaxOff], const uint32_t (&b_off)[kMaxOff], int kk, int u,
                                               Frags<T>& f) {
  if (u < T::FM) {
    f.a[u] = lds_read_a(a_st + a_off[kk * T::APAR + u % T::APAR] + (u / T::APAR) * T::AROWS * T::BK * 2);
  } else {
    const int nb = u - T::FM;
    if constexpr (BKM)
      f.b[nb] = lds_read_a(b_st + b_off[kk * T::APAR + nb % T::APAR] + (nb / T::APAR) * T::AROWS * T::BK * 2);
    else
      f.b[nb] = lds_read_b_tr(b_st + b_off[nb] + (kk * T::KK) * T::BN * 2,
                              b_st + b_off[nb] + (kk * T::KK + 4) * T::BN * 2);
  }
}

// All fragment reads of K-step kk from an LDS stage.
template <class T, bool BKM>
__device__ __forceinline__ void load_frags(const char LDS_AS* a_st, const char LDS_AS* b_st, const uint32_t (&a_off)[kMaxOff],
                                           const uint32_t (&b_off)[kMaxOff], int kk, Frags<T>& f) {
#pragma unroll
  for (int u = 0; u < T::FM + T::FN; ++u) load_frag_unit<T, BKM>(a_st, b_st, a_off, b_off, kk, u, f);
}

// One MFMA of the tile's shape, operands swapped (B fragment as src A): acc holds C^T.
template <class T>
__device__ __forceinline__ void mfma_one(const half8& b, const half8& a, AccT<T>& acc) {
  if constexpr (T::MF == 32)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, acc, 0, 0, 0);
  else
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, acc, 0, 0, 0);
}

// Issue order of a K-step's FM x FN MFMAs: MFMA i updates accumulator (ord_mb(i), ord_nb(i)),
// row by row with the column order reversed on every other row (a snake), so consecutive MFMAs
// share an operand at the turns too.  Each accumulator still sees its K-steps in order, so the
// order does not change any result.  Under sustained load the MI355X runs at its power cap, and
// fewer operand changes between consecutive MFMAs cost less power: at 8192^3 (interleaved runs,
// bit-identical results) the snake ran 1363 TFLOP/s against 1354 for plain row-major or
// column-major order and 1359 for a column snake.
template <class T>
__host__ __device__ constexpr int ord_mb(int i) {
  return i / T::FN;
}
template <class T>
__host__ __device__ constexpr int ord_nb(int i) {
  return ((i / T::FN) & 1) ? T::FN - 1 - i % T::FN : i % T::FN;
}

template <class T>
__device__ __forceinline__ void mfma_frags(const Frags<T>& f, AccT<T> (&acc)[T::FM][T::FN]) {
#pragma unroll
  for (int i = 0; i < T::FM * T::FN; ++i) {
    mfma_one<T>(f.b[ord_nb<T>(i)], f.a[ord_mb<T>(i)], acc[ord_mb<T>(i)][ord_nb<T>(i)]);
  }
}

template <class T, bool BKM, class Hook>
__device__ __forceinline__ void compute_stage(const char LDS_AS* a_st, const char LDS_AS* b_st,
                                              const uint32_t (&a_off)[kMaxOff], const uint32_t (&b_off)[kMaxOff],
                                              AccT<T> (&acc)[T::FM][T::FN], Hook&& after_first_reads) {
  using Frags = mmm::Frags<T>;
  auto load = [&](int kk, Frags& f) { load_frags<T, BKM>(a_st, b_st, a_off, b_off, kk, f); };
  auto mfma = [&](const Frags& f) { mfma_frags<T>(f, acc); };
#pragma unroll
  for (int kk = 0; kk < T::KSTEPS; ++kk) {
    Frags f;
    load(kk, f);
    if (kk == 0) after_first_reads();
    mfma(f);
  }
}

__device__ __forceinline__ void block_sync() { __syncthreads(); }

// ---- C stores as whole 128-byte lines (16x16x32 tiles).  A 16x16 accumulator block gives lane l
// row l % 16 and columns 4*(l/16) .. +3, so one float4 store of a block writes 16 rows x 64
// bytes: half lines.  Blocks nb and nb+1 of a row of blocks cover 32 columns; lanes l and l ^ 8
// (rows r and r + 8) trade their block-(nb+1) values (one DPP move per register), after which
// one store writes rows 0-7 and the next rows 8-15, each row 32 columns: one 128-byte line (the
// 192x192 tile's odd third block of a row stays half lines).  gemm_nn_kernel stores its interior
// tiles this way with every store policy; the persistent kernels with non-temporal stores only.
// Measured on MI355X (interleaved runs,
// same box, exact results), against half lines: 8192^3 +0.6-0.9%, 12288^2 x 4096 +1.4%,
// 16384^2 x 4096 +1.0%, 8192 x 2048 x 2048 +1.4%, 4096^3 +0.8%, 6144^3 +0.4%; with plain
// (L2-allocating) stores the persistent grids lost up to 2% at short K (8192^2 x 2048 -1.6%,
// 16384 x 8192 x 1024 -2.0%).
enum CStore { kStorePlain = 0, kStoreNonTemporal = 1, kStoreWriteThrough = 2 };

// System-scope write-through 16-byte store (sc0 sc1), as inline asm.  The compiler does not see
// a store in inline asm, so it does not add the wait states a VALU write of the store's data
// registers needs after a VMEM store of more than 8 bytes (2 on gfx950); the s_nop supplies them.
// Without it the next VALU write could replace the data before the store read it (seen as
// wrong C values when the epilogue reused the registers at once).
#define WT_STORE_X4 "global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1"

template <int POLICY>
__device__ __forceinline__ void store_c4(float* dst, f32x4 v) {
  if constexpr (POLICY == kStoreNonTemporal)
    __builtin_nontemporal_store(v, (f32x4*)dst);
  else if constexpr (POLICY == kStoreWriteThrough)
    asm volatile(WT_STORE_X4 ::"v"(dst), "v"(v) : "memory");
  else
    *(f32x4*)dst = v;
}

// Lane l's result is lane (l ^ 8)'s x (DPP row_ror:8 within each 16-lane row).  Called
// unconditionally: a cross-lane move inside one arm of a lane-dependent ?: runs with the other
// lanes switched off and reads nothing from them.  Written per element: a loop over a vector's
// elements here compiled to one DPP move reused for all four.
__device__ __forceinline__ float from_lane_xor8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}
__device__ __forceinline__ f32x4 from_lane_xor8(f32x4 v) {
  return f32x4{from_lane_xor8(v.x), from_lane_xor8(v.y), from_lane_xor8(v.z), from_lane_xor8(v.w)};
}

// The lane index read afresh (v_mbcnt in asm, which the compiler cannot hoist out of a loop):
// values derived from it are rebuilt where they are used instead of being kept live.
__device__ __forceinline__ int lane_id_fresh() {
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return lane;
}

template <class T>
constexpr bool c_lines_ok() {
  return T::MF == 16 && T::FN >= 2;
}
// every store of the tile a whole line (an even number of blocks per row)
template <class T>
constexpr bool c_lines_all() {
  return c_lines_ok<T>() && T::FN % 2 == 0;
}
template <class T, int POLICY>
constexpr bool use_c_lines() {
  return c_lines_ok<T>() && POLICY != kStorePlain;
}

// The wave's whole TM x TN accumulator tile to C at `c` (the wave tile's first element; rows
// ldc floats apart), every 32-column pair of blocks as 16 row lines (an odd last block as half
// lines).  The lane's row and column offsets are built here from a fresh lane index: kept from
// before a persistent kernel's tile loop they would stay live across its K loop, which runs at
// the register limit (they spilled).
template <class T, int POLICY>
__device__ __forceinline__ void store_wave_tile_lines(float* c, int64_t ldc, const AccT<T> (&acc)[T::FM][T::FN]) {
  static_assert(c_lines_ok<T>(), "16x16 blocks, at least two per row");
  const int lane = lane_id_fresh();
  const bool lo = (lane & 8) == 0;
  float* r0 = c + (int64_t)(lane & 7) * ldc + 4 * (lane >> 4) + (lo ? 0 : 16);        // rows 0-7
  float* r1 = c + (int64_t)((lane & 7) + 8) * ldc + 4 * (lane >> 4) + (lo ? 16 : 0);  // rows 8-15
#pragma unroll
  for (int mb = 0; mb < T::FM; ++mb) {
#pragma unroll
    for (int nb = 0; nb + 1 < T::FN; nb += 2) {
      // rows 0-7: lanes 0-7 keep block nb, lanes 8-15 take block nb + 1 of lanes 0-7;
      // rows 8-15: lanes 8-15 keep block nb, lanes 0-7 take block nb + 1 of lanes 8-15
      const f32x4 traded = from_lane_xor8(acc[mb][nb + 1]);
      const f32x4 rows_lo = lo ? acc[mb][nb] : traded, rows_hi = lo ? traded : acc[mb][nb];
      store_c4<POLICY>(r0 + (int64_t)16 * mb * ldc + 16 * nb, rows_lo);
      store_c4<POLICY>(r1 + (int64_t)16 * mb * ldc + 16 * nb, rows_hi);
      __builtin_amdgcn_sched_barrier(0);  // one pair at a time: the traded values stay few
    }
    if constexpr (T::FN % 2 != 0)  // the odd last block: lane l's row l % 16, 16 rows x 64 bytes
      store_c4<POLICY>(c + (int64_t)(16 * mb + (lane & 15)) * ldc + 16 * (T::FN - 1) + 4 * (lane >> 4),
                       acc[mb][T::FN - 1]);
  }
}

// Measurement: thread 0 of workgroup 0 writes the shader-clock counter (s_memtime) and the 100 MHz
// real-time counter (s_memrealtime) to clk[at], clk[at + 1] when the caller asked for them.
__device__ __forceinline__ void record_clock(uint64_t* clk, int at) {
  if (clk != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    clk[at] = __builtin_amdgcn_s_memtime();
    clk[at + 1] = __builtin_amdgcn_s_memrealtime();
  }
}

// K-steps 0 .. KSTEPS-2 of the K tile in LDS stage `st`: each step's MFMAs (fragments f[kk & 1])
// run while the next step's fragments are read into f[(kk + 1) & 1]; MFMA i carries fragment
// read i, and scheduling fences keep that order.
template <class T, bool BKM>
__device__ __forceinline__ void ktile_body(const char LDS_AS* st, const uint32_t (&a_off)[kMaxOff],
                                           const uint32_t (&b_off)[kMaxOff], Frags<T> (&f)[2],
                                           AccT<T> (&acc)[T::FM][T::FN]) {
#pragma unroll
  for (int kk = 0; kk + 1 < T::KSTEPS; ++kk) {
#pragma unroll
    for (int i = 0; i < T::FM * T::FN; ++i) {
      mfma_one<T>(f[kk & 1].b[ord_nb<T>(i)], f[kk & 1].a[ord_mb<T>(i)], acc[ord_mb<T>(i)][ord_nb<T>(i)]);
      if (i < T::FM + T::FN) load_frag_unit<T, BKM>(st, st + T::A_BYTES, a_off, b_off, kk + 1, i, f[(kk + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The last K-step of a K tile, after the barrier that publishes the next one in stage `ns`: its
// MFMAs (fragments f[1]) carry the next stage's first fragment reads (into f[0], MFMA i carrying
// read i) and the LPT refill loads dma_one(d, 0 .. LPT-1), spread evenly over the MFMAs after the
// reads when there are enough of them (every load is a 1 KB request to the address unit, and all
// waves refill in the same K-step, so a burst of them fills its queue and stalls each wave's
// MFMAs behind its next load).  Measured on the 256x256 tile (32 MFMAs, 8 loads) at 8192^3: one
// load every MFMA 1258 TFLOP/s, every 2 within 1%, every 3 +1%, every 4 (the even spread) +4.4%.
template <class T, bool BKM, class D, class DmaOne>
__device__ __forceinline__ void ktile_last_step(const char LDS_AS* ns, const uint32_t (&a_off)[kMaxOff],
                                                const uint32_t (&b_off)[kMaxOff], Frags<T> (&f)[2],
                                                AccT<T> (&acc)[T::FM][T::FN], const D& d, DmaOne&& dma_one) {
  constexpr int NM = T::FM * T::FN, NU = T::FM + T::FN;
  constexpr int NL = T::LPT;
  constexpr int DS = NM / NL > 1 ? NM / NL : 1;  // MFMAs between loads
  constexpr int D0 = NM - DS * NL >= NU ? NU : (NM > DS * NL ? NM - DS * NL : 0);
  int issued = 0;
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    const int mb = ord_mb<T>(i), nb = ord_nb<T>(i);
    mfma_one<T>(f[1].b[nb], f[1].a[mb], acc[mb][nb]);
    if (i < NU) load_frag_unit<T, BKM>(ns, ns + T::A_BYTES, a_off, b_off, 0, i, f[0]);
    if (i >= D0 && (i - D0) % DS == 0 && issued < NL) dma_one(d, issued++);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int j = 0; j < NL; ++j)
    if (j >= issued) dma_one(d, j);
}

// Cross-stage K loop over KT K tiles (the direct-to-LDS kernels).  The caller supplies the
// loads: prep(t, slot) builds the per-tile load state of K tile t for ring slot `slot` (and
// advances any running state: tiles are prepared in order), dma_one(d, j) issues load j of
// T::LPT, and issue_tile(t, slot) fills slot `slot` with tile t by whatever means (the last
// tile of an unaligned problem is gathered through VGPRs when tail_regs is set, which leaves
// no loads in flight for it).
//
// pre = 0: the loop issues the first tiles itself.  pre = 1: the caller has issued tiles
// 0 .. S-1 already (KT >= S).  pre = 2: as 1, and NST further vector-memory operations (the
// previous tile's C stores) were issued after them; the first wait lets those stay
// outstanding (vmcnt retires in issue order).
//
// first_wait() runs once tile 0 has landed, before the barrier that publishes it;
// tail_patch(slot) runs once this wave's loads of the last tile (in ring slot `slot`) have
// landed, before the barrier that publishes it: a thread may overwrite the chunks its own
// loads put there.
struct NoHook {
  __device__ __forceinline__ void operator()() const {}
};
struct NoSlotHook {
  __device__ __forceinline__ void operator()(int) const {}
};

template <class T, bool BKM, int NST = 0, class Prep, class DmaOne, class IssueTile, class FirstWait = NoHook,
          class TailPatch = NoSlotHook>
__device__ __forceinline__ void cross_stage(char LDS_AS* lds_base, int KT, bool tail_regs, const uint32_t (&a_off)[kMaxOff],
                                            const uint32_t (&b_off)[kMaxOff], AccT<T> (&acc)[T::FM][T::FN], Prep&& prep,
                                            DmaOne&& dma_one, IssueTile&& issue_tile, int pre = 0,
                                            FirstWait&& first_wait = FirstWait{}, TailPatch&& tail_patch = TailPatch{}) {
  // Ring of S slots, tile u in slot u % S.  Cross-stage pipeline: during the last K-step of
  // tile t, this wave waits for its own loads of tile t+1, then the barrier (a) publishes
  // tile t+1 -- every wave's loads of it have landed -- and (b) retires slot t % S: every
  // wave has completed its reads of tile t, since a barrier waits for outstanding LDS reads
  // and tile t's last fragments were read before it.  After the barrier the wave reads
  // tile t+1's first fragments and refills slot t % S with tile t+S, and only then issues
  // tile t's last MFMAs, which cover the barrier and the first reads' latency.
  constexpr int S = T::STAGES;
  static_assert(T::KSTEPS % 2 == 0, "fragment double buffer alternates per K-step");
  const int first = KT < S ? KT : S;
  if (pre == 0)
    for (int s = 0; s < first; ++s) issue_tile(s, s);
  // tile 0 must land; later tiles may stay in flight (a gathered last tile has no loads)
  if (pre == 2) {
    static_assert((S - 1) * T::LPT + NST <= 63, "vmcnt range");
    wait_vmcnt<(S - 1) * T::LPT + NST>();
  } else {
    wait_tiles<T::LPT, S - 1>(first - 1 - ((tail_regs && first == KT) ? 1 : 0));
  }
  first_wait();
  if (KT == 1) tail_patch(0);
  block_sync();
  Frags<T> f[2];
  load_frags<T, BKM>(lds_base, lds_base + T::A_BYTES, a_off, b_off, 0, f[0]);
  int cur = 0;
  // K-steps 0 .. KSTEPS-2 of the tile in slot `cur` (each step's MFMAs run while the next
  // step's fragments are read).
  auto tile_body = [&] { ktile_body<T, BKM>(lds_base + cur * T::STAGE, a_off, b_off, f, acc); };
  // Last K-step of tile t < KT-1: publish tile t+1, read its first fragments, refill the
  // retired slot (`refill` loads tile t+S into slot `cur`), then the MFMAs.
  auto tile_next = [&](int t, auto&& refill) {
    __builtin_amdgcn_sched_barrier(0);  // the body's MFMAs stay ahead of the waits
    const int issued = t + S < KT ? t + S : KT;  // tiles 0 .. issued-1 are issued
    int ahead = issued - (t + 2);                // of those, after t+1 (may stay in flight)
    if (tail_regs && issued == KT && ahead > 0) --ahead;
    wait_tiles<T::LPT, (S > 2 ? S - 2 : 0)>(ahead);
    const int nslot = cur + 1 == S ? 0 : cur + 1;
    if (t + 1 == KT - 1) tail_patch(nslot);
    block_sync();
    const char LDS_AS* ns = lds_base + nslot * T::STAGE;
    load_frags<T, BKM>(ns, ns + T::A_BYTES, a_off, b_off, 0, f[0]);
    refill();
    mfma_frags<T>(f[1], acc);
    cur = nslot;
  };
  // Steady state: after the barrier the next tile's first fragment reads and the refill's
  // loads are interleaved with the last K-step's MFMAs (ktile_last_step), so neither a burst of
  // LDS reads nor a burst of load issue leaves the matrix pipe idle.
  auto tile_next_interleaved = [&](int t) {
    __builtin_amdgcn_sched_barrier(0);  // the body's MFMAs stay ahead of the waits
    wait_tiles<T::LPT, (S > 2 ? S - 2 : 0)>(S - 2);  // steady state: S-2 tiles after t+1 in flight
    block_sync();
    const int nslot = cur + 1 == S ? 0 : cur + 1;
    ktile_last_step<T, BKM>(lds_base + nslot * T::STAGE, a_off, b_off, f, acc, prep(t + S, cur), dma_one);
    cur = nslot;
  };
  // steady state refills by DMA only; the refill of the last tile (possibly gathered
  // through VGPRs) is peeled so the loop carries no gather registers
  int t = 0;
  for (; t + S < KT - 1; ++t) {
    tile_body();
    tile_next_interleaved(t);
  }
  if (t + S == KT - 1) {
    tile_body();
    tile_next(t, [&] { issue_tile(t + S, cur); });
    ++t;
  }
  for (; t + 1 < KT; ++t) {
    tile_body();
    tile_next(t, [] {});
  }
  tile_body();
  mfma_frags<T>(f[1], acc);
}

// GENERIC = false: direct-to-LDS buffer loads; needs 2-byte-aligned A and B and per-tile byte
//                  offsets within 32 bits (dma_ok).  Rows that are not 16-byte aligned are read
//                  by unaligned buffer loads.  The last K tile of an unaligned problem
//                  (tail_regs) is loaded like the others with its chunks across K (A) and
//                  across N in B's last row patched from a copy gathered at the start, or,
//                  for operands narrower than the tile (ldb < BN or lda < 8), gathered
//                  through VGPRs.
// GENERIC = true : element-wise masked loads through VGPRs; any shape and alignment.
// CPOL: how C's 16-byte pieces are stored (CStore): plain, non-temporal or system-scope
//       write-through (sc0 sc1); the last two for 16-byte-aligned C rows only (see launch_nn).
// TAIL: the direct-to-LDS kernel handles an unaligned last K tile (p.tail_regs); launches
//       without one run the instantiation with TAIL = false, which carries none of that code.
// Launch bounds: the 64x64 tile declares the three workgroups per CU its LDS ring allows.  With
// one, the compiler kept that tile's accumulators in AGPRs and copied them to and from VGPRs
// every K tile of the instantiation without the tail code (20 copies per 8 MFMAs; 1024^2 x 2048
// ran 14.7 against 14.1 us); with three it keeps them in VGPRs.
template <class T>
constexpr int nn_launch_occupancy() {
  return T::BM == 64 && T::BN == 64 ? 3 : T::OCC;
}
template <class T, bool GENERIC, int CPOL = kStorePlain, bool TAIL = true>
__global__ __launch_bounds__(T::NT, nn_launch_occupancy<T>()) void gemm_nn_kernel(GemmProblem p, int tiles_m,
                                                                                  int tiles_n) {
  __shared__ __attribute__((aligned(1024))) char lds[T::STAGES * T::STAGE];
  // The last K tile's straddling chunks, gathered at the start: A's chunk across K of each
  // tile row (entry = row in the tile), then B's chunk across N in row K-1 (entry BM).
  constexpr int kSpare = TAIL && !GENERIC ? T::BM + 1 : 1;
  __shared__ half8 tail_spare[kSpare];
  static_assert(GENERIC || T::OCC * (T::STAGES * T::STAGE + kSpare * 16) <= 160 * 1024,
                "LDS rings and the tail copy must fit the 160 KB LDS");
  record_clock(p.clk, 0);

  // K split (direct-to-LDS path only).  Blocks [0, whole) compute tiles 0 .. whole-1 of the
  // XCD-aware order over their full K range; the last split_tiles tiles of that order are split:
  // block whole + q * split_tiles + j computes K range q of tile whole + j (each split layer
  // walks those tiles in the same order).
  const int ntiles = tiles_m * tiles_n;
  const int ksplit = (!GENERIC && p.k_splits > 1) ? p.k_splits : 1;
  const int whole = ksplit > 1 ? ntiles - p.split_tiles : ntiles;
  const bool split_block = (int)blockIdx.x >= whole;
  const int nsplit = split_block ? ksplit : 1;
  int q = 0, j = 0, bt = (int)blockIdx.x;
  if (split_block) {
    const int b2 = (int)blockIdx.x - whole;
    q = b2 / p.split_tiles;
    j = b2 - q * p.split_tiles;
    bt = whole + j;
  }
  q = __builtin_amdgcn_readfirstlane(q);
  int tm, tn;
  tile_of_block(bt, tiles_m, tiles_n, 4, &tm, &tn);
  // The tile origin is uniform; readfirstlane keeps it (and everything derived from it, such
  // as the buffer descriptors) in SGPRs -- the integer divisions above are expanded on the VALU.
  const int m0 = __builtin_amdgcn_readfirstlane(tm * T::BM), n0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;

  // ---- staging map.  Thread (w, lane) moves chunk slot s = r*NT + w*64 + lane of a stage
  // (r = 0..RA-1 for A, 0..RB-1 for B).  A round of NT slots covers RPA = NT/CA rows of A
  // and RPB = NT/CB rows of B, so slot rows are row0 + r*RP; RPA is a multiple of the rows
  // the A swizzle depends on and RPB of 4, so the logical chunk is the same every round.
  constexpr int RPA = T::NT / T::CA, RPB = T::NT / T::CB;
  static_assert(RPA % T::SWZ_A_ROWS == 0 && (!T::B_UNIFORM || RPB % T::SWZ_B_ROWS == 0),
                "round strides must preserve the swizzle");
  static_assert(!GENERIC || T::B_UNIFORM, "the register-staged path uses the uniform B map");
  const int a_row0 = w * (64 / T::CA) + lane / T::CA;
  const int a_kc = 8 * ((lane % T::CA) ^ T::swz_a(a_row0));
  const int b_row0 = T::B_UNIFORM ? w * (64 / T::CB) + lane / T::CB : 0;
  const int b_nc = T::B_UNIFORM ? 8 * ((lane % T::CB) ^ T::swz_bk(b_row0)) : 0;
  // B row and column of slot r (any CB)
  auto b_row_of = [&](int r) {
    if constexpr (T::B_UNIFORM) return b_row0 + r * RPB;
    else return (r * T::NT + w * 64 + lane) / T::CB;
  };
  auto b_col_of = [&](int r) {
    if constexpr (T::B_UNIFORM) return b_nc;
    else {
      const int sl = r * T::NT + w * 64 + lane;
      return 8 * ((sl % T::CB) ^ T::swz_bk(sl / T::CB));
    }
  };

  // ---- fragment read offsets (bytes within a stage).  MF = 32: lane l reads row l % 32 of
  // A, k chunk l / 32 of each 16-deep step; B rows 8*(l/32) + (l/4)%4 (+4), columns
  // 16*((l/16)%2) + 4*(l%4) of each 32-column fragment.  MF = 16: row l % 16 of A, k chunk
  // l / 16 of each 32-deep step; B rows 8*(l/16) + (l/4)%4 (+4), columns 4*(l%4) of each
  // 16-column fragment.
  uint32_t a_off[kMaxOff] = {};
#pragma unroll
  for (int kk = 0; kk < T::KSTEPS; ++kk)
#pragma unroll
    for (int ph = 0; ph < T::APAR; ++ph) {
      const int m = wm * T::TM + ph * T::MF + (lane % T::MF);
      const int chunk = (T::KK / 8) * kk + lane / T::MF;
      a_off[kk * T::APAR + ph] = m * T::BK * 2 + (chunk ^ T::swz_a(m)) * 16;
    }
  uint32_t b_off[kMaxOff] = {};
  {
    const int k = 8 * (lane / T::MF) + ((lane >> 2) & 3);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
      const int n = T::MF == 32 ? wn * T::TN + 32 * nb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)
                                : wn * T::TN + 16 * nb + 4 * (lane & 3);
      b_off[nb] = k * T::BN * 2 + (((n >> 3) ^ T::swz_bk(k)) * 16) + (n & 7) * 2;
    }
  }

  AccT<T> acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = AccT<T>{};

  const int KT_all = (K + T::BK - 1) / T::BK;
  const int t_begin = __builtin_amdgcn_readfirstlane((q * KT_all) / nsplit);
  const int t_end = __builtin_amdgcn_readfirstlane(((q + 1) * KT_all) / nsplit);
  const int KT = t_end - t_begin;  // K tiles of this block
  char LDS_AS* lds_base = (char LDS_AS*)lds;

  if constexpr (!GENERIC) {
    const uint32_t a_goff = (uint32_t)((a_row0 * lda + a_kc) * 2);
    const uint32_t b_goff = (uint32_t)((b_row0 * ldb + b_nc) * 2);
    const uint32_t a_rstep = (uint32_t)(RPA * lda * 2), b_rstep = (uint32_t)(RPB * ldb * 2);
    uint32_t b_goffr[T::B_UNIFORM ? 1 : T::RB];  // per-slot B offsets (non-uniform map)
    if constexpr (!T::B_UNIFORM) {
#pragma unroll
      for (int r = 0; r < T::RB; ++r) b_goffr[r] = (uint32_t)((b_row_of(r) * ldb + b_col_of(r)) * 2);
    }

    // The last K tile of an unaligned problem (p.tail_regs: K or N not a multiple of 8, or rows
    // not 16-byte aligned), in the block that holds it.  When B's rows are at least a tile wide
    // and A's at least a chunk (dma_tail), no chunk of any tile reaches across a descriptor's
    // range end other than two of the last tile: A's chunk across K in row M-1 and B's chunk
    // across N in row K-1.  The last tile's ranges end before those two, so they read as zero
    // like every chunk past the ends, and its chunks across K (every row of A: past K they hold
    // the next row's values) and across N in B's row K-1 are overwritten from tail_spare before
    // the tile is published (tail_fix).  Narrower operands gather the whole last tile through
    // VGPRs instead (tail_regs).
    const bool tail_block = TAIL && p.tail_regs && t_end == KT_all;
    const bool dma_tail = ldb >= T::BN && lda >= 8;
    const bool tail_regs = tail_block && !dma_tail;
    const bool tail_fix = tail_block && dma_tail;

    // DMA of K tile t into ring slot `stage`: RA + RB buffer_load_dwordx4 ... lds per thread.
    // Each range ends at the operand's last element (row M-1, column K-1 of A; row K-1,
    // column N-1 of B), so nothing past the caller's data is ever fetched; rows past the end
    // read as zero.  With N, K multiples of 8 no chunk straddles a range end.  K tiles are
    // issued in order (t = 0, 1, ...), so bases and remaining byte counts advance by a
    // constant per tile instead of being recomputed.
    const char* a_ptr = (const char*)(p.A + (int64_t)m0 * lda + (int64_t)t_begin * T::BK);
    const char* b_ptr = (const char*)(p.B + (int64_t)t_begin * T::BK * ldb + n0);
    int64_t a_left = ((int64_t)(M - 1 - m0) * lda + K - (int64_t)t_begin * T::BK) * 2;
    int64_t b_left = ((int64_t)(K - 1 - t_begin * T::BK) * ldb + N - n0) * 2;
    const int64_t b_step = (int64_t)T::BK * ldb * 2;
    // A K tile's loads: descriptors and bases (prep; advances the running state), then the
    // LPT loads, j = 0 .. RA-1 for A and RA .. LPT-1 for B (dma_one).
    struct TileDma {
      i32x4 ra, rb;
      uint32_t a_dst, b_dst, a_base;
    };
    auto prep = [&](int t, int stage) {
      const int k0 = (t_begin + t) * T::BK;
      TileDma d;
      d.ra = make_rsrc(a_ptr, clip_records(a_left));
      d.rb = make_rsrc(b_ptr, clip_records(b_left));
      a_ptr += T::BK * 2, a_left -= T::BK * 2;
      b_ptr += b_step, b_left -= b_step;
      d.a_dst = lds_addr_of(lds_base) + stage * T::STAGE + w * 64 * 16;
      d.b_dst = d.a_dst + T::A_BYTES;
      // K tail: a chunk at or past K gets kOobOffset added, which puts it beyond the
      // descriptor's range so it reads as zero (no select: keeps the loads branch-free).
      const uint32_t a_dead = (uint32_t)(K - 1 - (k0 + a_kc)) >> 31;
      d.a_base = a_goff + ((0u - a_dead) & kOobOffset);
      return d;
    };
    auto dma_one = [&](const TileDma& d, int j) {
      if (j < T::RA)
        dma_b128(d.a_dst + j * T::NT * 16, d.ra, d.a_base + j * a_rstep);
      else
        dma_b128(d.b_dst + (j - T::RA) * T::NT * 16, d.rb,
                 T::B_UNIFORM ? b_goff + (j - T::RA) * b_rstep : b_goffr[T::B_UNIFORM ? 0 : j - T::RA]);
    };
    auto issue = [&](int t, int stage) {
      const TileDma d = prep(t, stage);
#pragma unroll
      for (int j = 0; j < T::LPT; ++j) dma_one(d, j);
    };

    // tail_regs: the last K tile gathered element by element through VGPRs into the same slot
    // layout.
    const _Float16* Ah = (const _Float16*)p.A;
    const _Float16* Bh = (const _Float16*)p.B;
    auto fill_regs = [&](int t, int stage) {
      const int k0 = (t_begin + t) * T::BK;
      char LDS_AS* a_dst = lds_base + stage * T::STAGE + (w * 64 + lane) * 16;
      char LDS_AS* b_dst = a_dst + T::A_BYTES;
      // Element loads under lane conditions, one memory round trip each: this path serves
      // operands narrower than the tile only, and it runs in the refill peeled off the K loop,
      // where the registers that would keep a chunk's loads in flight together are not free
      // (the 256x256 tile spilled; on the 64x64 tile, where they fit, the extra registers cost
      // its patched-tail launches 0.2-0.3 us per call, more than the gather gained).
#pragma unroll
      for (int r = 0; r < T::RA; ++r) {
        const int m = m0 + a_row0 + r * RPA, k = k0 + a_kc;
        half8 v = {};
        if (m < M) {
          const _Float16* src = Ah + (int64_t)m * lda + k;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k + e < K) v[e] = src[e];
        }
        *(half8 LDS_AS*)(a_dst + r * T::NT * 16) = v;
      }
#pragma unroll
      for (int r = 0; r < T::RB; ++r) {
        const int k = k0 + b_row_of(r), n = n0 + b_col_of(r);
        half8 v = {};
        if (k < K) {
          const _Float16* src = Bh + (int64_t)k * ldb + n;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) v[e] = src[e];
        }
        *(half8 LDS_AS*)(b_dst + r * T::NT * 16) = v;
      }
    };
    // tail_fix: the chunk of the last K tile across K (column k0t + a_kcs .. +7 of each row of
    // A, K % 8 of them valid) and across N in B's row K-1 (columns n0 + n_cs .. +7, N % 8
    // valid), gathered here (their loads overlap the first tiles'), kept in tail_spare from
    // the first tile's wait on, and copied over what the DMA put in their slots.  Thread
    // (w, lane) owns the same chunks in every tile: its A chunks when its chunk column is
    // a_kcs, and B slot r when that slot is row K-1, column n_cs.
    const int k0t = (KT_all - 1) * T::BK;
    const int a_kcs = (K - k0t) & ~7, n_cs = (N - n0) & ~7;
    const bool a_fix = tail_fix && (K & 7) != 0 && a_kc == a_kcs;
    // What the last tile needs, packed into one scalar that lives through the K loop: bit 0
    // tail_fix, then K % 8, N % 8, a_kcs (6 bits), K-1 as a row of the last tile (< 64) and n_cs
    // clamped to BN (no chunk of the tile when the tile does not reach N).  a_kcs is used only
    // when K % 8 != 0, where it is at most 56; with K a multiple of 64 it is 64 and is masked to
    // keep it out of the row field (whose low bit it would otherwise set: that field is then 63,
    // so the OR changed nothing, but the mask does not rely on that).
    const uint32_t tp = !TAIL ? 0u
                              : __builtin_amdgcn_readfirstlane(
                                    (uint32_t)tail_fix | (uint32_t)(K & 7) << 1 | (uint32_t)(N & 7) << 4 |
                                    (uint32_t)(a_kcs & 63) << 7 | (uint32_t)(K - 1 - k0t) << 13 |
                                    (uint32_t)(n_cs < T::BN ? n_cs : T::BN) << 19);
    // Both the gather and the store sit behind the scalar test of tp: the wait for the gathered
    // registers (a full vmcnt drain, the compiler not seeing the DMA loads) must not reach the
    // prologue of a launch without a patched tail.
    half8 a_fixv[T::RA];
    int b_fix_r = -1;
    half8 b_fixv = {};
    // Every lane loads (addresses clamped into the operands, values masked afterwards), so the
    // loads carry no branches and go out together: a load under a lane condition is merged
    // into its vector before the next one issues, one memory round trip each.
    if (tp & 1) {
      const int ka = K & 7, kb = N & 7;
      if (ka != 0) {
#pragma unroll
        for (int r = 0; r < T::RA; ++r) {
          const int m = m0 + a_row0 + r * RPA;
          const _Float16* src = Ah + (int64_t)(m < M ? m : M - 1) * lda + k0t + a_kcs;
          _Float16 x[7];
#pragma unroll
          for (int e = 0; e < 7; ++e) x[e] = src[e < ka ? e : ka - 1];  // columns below K
          half8 v = {};
#pragma unroll
          for (int e = 0; e < 7; ++e) v[e] = (e < ka && m < M) ? x[e] : (_Float16)0;
          a_fixv[r] = v;
        }
      }
      if (kb != 0) {
#pragma unroll
        for (int r = 0; r < T::RB; ++r)
          if (k0t + b_row_of(r) == K - 1 && b_col_of(r) == n_cs) b_fix_r = r;
        const _Float16* src = Bh + (int64_t)(K - 1) * ldb;
        const int c0 = n0 + n_cs;
        _Float16 x[7];
#pragma unroll
        for (int e = 0; e < 7; ++e) x[e] = src[c0 + e < N ? c0 + e : N - 1];
#pragma unroll
        for (int e = 0; e < 7; ++e) b_fixv[e] = e < kb ? x[e] : (_Float16)0;
      }
    }
    auto spare_store = [&] {
      if (tp & 1) {
        if (a_fix) {
#pragma unroll
          for (int r = 0; r < T::RA; ++r) tail_spare[a_row0 + r * RPA] = a_fixv[r];
        }
        if (b_fix_r >= 0) tail_spare[kSpare - 1] = b_fixv;  // entry BM
      }
    };
    // At the last tile the lane-derived values are rebuilt from a fresh lane index rather than
    // kept live through the K loop.
    auto tail_patch = [&](int slot) {
      if (!(tp & 1)) return;
      const int ln = lane_id_fresh();
      char LDS_AS* a_dst = lds_base + slot * T::STAGE + (w * 64 + ln) * 16;
      const int row0 = w * (64 / T::CA) + ln / T::CA;
      if ((tp >> 1 & 7) != 0 && 8 * ((ln % T::CA) ^ T::swz_a(row0)) == (int)(tp >> 7 & 63)) {
#pragma unroll
        for (int r = 0; r < T::RA; ++r) *(half8 LDS_AS*)(a_dst + r * T::NT * 16) = tail_spare[row0 + r * RPA];
      }
      if ((tp >> 4 & 7) != 0) {
#pragma unroll
        for (int r = 0; r < T::RB; ++r) {
          const int sl = r * T::NT + w * 64 + ln;
          const int row = sl / T::CB, col = 8 * ((sl % T::CB) ^ T::swz_bk(row));
          if (row == (int)(tp >> 13 & 63) && col == (int)(tp >> 19))
            *(half8 LDS_AS*)(a_dst + T::A_BYTES + r * T::NT * 16) = tail_spare[kSpare - 1];
        }
      }
    };

    // The last tile is issued by the prologue or by the refill peeled off the steady loop
    // (cross_stage), never by the steady loop's own refill.
    auto issue_tile = [&](int t, int stage) {
      if (tail_regs && t == KT - 1) {
        fill_regs(t, stage);
      } else {
        if ((tp & 1) && t == KT - 1) a_left -= (tp >> 1 & 7) * 2, b_left -= (tp >> 4 & 7) * 2;  // the cut ranges
        issue(t, stage);
      }
    };

    cross_stage<T, false>(lds_base, KT, tail_regs, a_off, b_off, acc, prep, dma_one, issue_tile, 0, spare_store,
                          tail_patch);
  } else {
    static_assert(!GENERIC || T::STAGES == 2, "the register-staged path double-buffers");
    (void)t_begin;
    u32x4 ra[T::RA], rb[T::RB];
    const _Float16* A = (const _Float16*)p.A;
    const _Float16* B = (const _Float16*)p.B;
    auto load = [&](int t) {
      const int k0 = t * T::BK;
#pragma unroll
      // Elements past the operands load from kZeroHalves: no load sits under a lane condition,
      // so a stage's loads go out together (a conditional load is merged into its vector before
      // the next one issues).
      for (int r = 0; r < T::RA; ++r) {
        const int m = m0 + a_row0 + r * RPA, k = k0 + a_kc;
        const _Float16* src = A + (int64_t)m * lda + k;
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = *(m < M && k + e < K ? src + e : kZeroHalves);
        ra[r] = __builtin_bit_cast(u32x4, v);
      }
#pragma unroll
      for (int r = 0; r < T::RB; ++r) {
        const int k = k0 + b_row0 + r * RPB, n = n0 + b_nc;
        const _Float16* src = B + (int64_t)k * ldb + n;
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = *(k < K && n + e < N ? src + e : kZeroHalves);
        rb[r] = __builtin_bit_cast(u32x4, v);
      }
    };
    auto store = [&](int stage) {
      char LDS_AS* a_dst = lds_base + stage * T::STAGE + (w * 64 + lane) * 16;
      char LDS_AS* b_dst = lds_base + stage * T::STAGE + T::A_BYTES + (w * 64 + lane) * 16;
#pragma unroll
      for (int r = 0; r < T::RA; ++r) *(u32x4 LDS_AS*)(a_dst + r * T::NT * 16) = ra[r];
#pragma unroll
      for (int r = 0; r < T::RB; ++r) *(u32x4 LDS_AS*)(b_dst + r * T::NT * 16) = rb[r];
    };

    load(0);
    store(0);
    block_sync();
    for (int t = 0; t + 1 < KT; ++t) {
      const int cur = t & 1;
      load(t + 1);
      compute_stage<T, false>(lds_base + cur * T::STAGE, lds_base + cur * T::STAGE + T::A_BYTES, a_off, b_off, acc,
                              NoHook{});
      store(cur ^ 1);
      block_sync();
    }
    {
      const int cur = (KT - 1) & 1;
      compute_stage<T, false>(lds_base + cur * T::STAGE, lds_base + cur * T::STAGE + T::A_BYTES, a_off, b_off, acc,
                              NoHook{});
    }
  }

  // ---- epilogue: lane owns row m, columns n..n+3 for each (mb, nb, q).  MF = 32: m = l % 32,
  // n = 32*nb + 8*q + 4*(l/32) (q = 0..3); MF = 16: m = l % 16, n = 16*nb + 4*(l/16) (q = 0).
  constexpr int NQ = T::MF == 32 ? 4 : 1;  // float4 groups per accumulator
  static_assert(NQ * 4 == sizeof(AccT<T>) / 4, "accumulator groups");
  auto col_of = [&](int nb, int qq) {
    return T::MF == 32 ? 32 * nb + 8 * qq + 4 * (lane >> 5) : 16 * nb + 4 * (lane >> 4);
  };
  if (nsplit > 1) {  // K split: the whole tile (rows/columns past M/N included) to the partials
    float* part = p.partials + ((int64_t)j * nsplit + q) * (T::BM * T::BN);
    // Whole lines, written through (sc0 sc1): reduce_tiles_kernel, next on the stream, reads
    // them on other XCDs.  Measured on MI355X (interleaved, against L2-allocating half lines):
    // 256 x 4096 x 4096 +9.2%, 1024^2 x 8192 +5.9%, 1024 x 2048 x 4096 +4.7%, 128 x 14336 x 4096
    // +3.3%, 1536^2 x 12288 +2.6%, 2304^2 x 8192 +1.9%; non-temporal lines -4% to +6%.
    if constexpr (c_lines_ok<T>()) {
      store_wave_tile_lines<T, kStoreWriteThrough>(part + wm * T::TM * T::BN + wn * T::TN, T::BN, acc);
      record_clock(p.clk, 2);
      return;
    }
#pragma unroll
    for (int mb = 0; mb < T::FM; ++mb) {
      float* prow = part + (wm * T::TM + T::MF * mb + (lane % T::MF)) * T::BN + wn * T::TN;
#pragma unroll
      for (int nb = 0; nb < T::FN; ++nb)
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq)
          *(f32x4*)(prow + col_of(nb, qq)) = f32x4{acc[mb][nb][4 * qq + 0], acc[mb][nb][4 * qq + 1],
                                                   acc[mb][nb][4 * qq + 2], acc[mb][nb][4 * qq + 3]};
    }
    record_clock(p.clk, 2);
    return;
  }
  float* C = p.C;
  const int64_t ldc = p.ldc;
  const bool vec_ok = p.c_vec4;
  // Interior tiles store whole lines with every store policy here (plain ones too: the ragged
  // configuration +0.7-1%, other plain grids +-0.5%).
  if constexpr (c_lines_ok<T>()) {
    if (vec_ok && m0 + T::BM <= M && n0 + T::BN <= N) {  // interior tile (uniform)
      store_wave_tile_lines<T, CPOL>(C + (int64_t)(m0 + wm * T::TM) * ldc + n0 + wn * T::TN, ldc, acc);
      record_clock(p.clk, 2);
      return;
    }
  }
#pragma unroll
  for (int mb = 0; mb < T::FM; ++mb) {
    const int m = m0 + wm * T::TM + T::MF * mb + (lane % T::MF);
    if (m >= M) continue;
    float* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int n = n0 + wn * T::TN + col_of(nb, q);
        f32x4 v = {acc[mb][nb][4 * q + 0], acc[mb][nb][4 * q + 1], acc[mb][nb][4 * q + 2], acc[mb][nb][4 * q + 3]};
        if (vec_ok && n + 3 < N) {
          store_c4<CPOL>(crow + n, v);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) crow[n + e] = v[e];
        }
      }
    }
  }
  record_clock(p.clk, 2);
}

// ------------------------------------------------------------------------------------
// Persistent direct-to-LDS tile kernel, for grids of whole interior tiles (M and N multiples
// of the tile, aligned operands and C; a K split of the last round runs as
// gemm_nn_persistent_split_kernel instead) over more than one round: grid =
// min(tiles, 256) workgroups; workgroup b computes tiles b, b + grid, b + 2*grid, ... of the
// XCD-aware order (grid % 8 == 0 keeps it on one XCD, walking that XCD's tile patches in
// order).  Between two tiles it waits for every wave to finish reading the ring, issues the
// next tile's first S K tiles, and only then stores the finished tile's C: the stores drain
// while those loads are in flight, and the next tile's first wait lets the NST stores
// (issued after the loads) stay outstanding, since vector-memory operations retire in issue
// order.
// ------------------------------------------------------------------------------------
template <class T, bool NT>
__global__ __launch_bounds__(T::NT, T::OCC) void gemm_nn_persistent_kernel(GemmProblem p, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) char lds[T::STAGES * T::STAGE];
  record_clock(p.clk, 0);
  constexpr int S = T::STAGES;
  constexpr int NQ = T::MF == 32 ? 4 : 1;       // float4 groups per accumulator
  constexpr int NST = T::FM * T::FN * NQ;       // C stores per thread per tile
  const int ntiles = tiles_m * tiles_n;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;

  // staging map and fragment offsets: as gemm_nn_kernel
  constexpr int RPA = T::NT / T::CA, RPB = T::NT / T::CB;
  static_assert(RPA % T::SWZ_A_ROWS == 0 && (!T::B_UNIFORM || RPB % T::SWZ_B_ROWS == 0),
                "round strides must preserve the swizzle");
  // Fragment offsets (as gemm_nn_kernel), rebuilt at every tile from a freshly read lane index:
  // kept from the kernel's start they would be live through the epilogue, whose line stores
  // need the registers.
  uint32_t a_off[kMaxOff], b_off[kMaxOff];
  auto frag_offsets = [&]() {
    const int ln = lane_id_fresh();
#pragma unroll
    for (int q = 0; q < kMaxOff; ++q) a_off[q] = b_off[q] = 0;
#pragma unroll
    for (int kk = 0; kk < T::KSTEPS; ++kk)
#pragma unroll
      for (int ph = 0; ph < T::APAR; ++ph) {
        const int m = wm * T::TM + ph * T::MF + (ln % T::MF);
        const int chunk = (T::KK / 8) * kk + ln / T::MF;
        a_off[kk * T::APAR + ph] = m * T::BK * 2 + (chunk ^ T::swz_a(m)) * 16;
      }
    const int k = 8 * (ln / T::MF) + ((ln >> 2) & 3);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
      const int n = T::MF == 32 ? wn * T::TN + 32 * nb + 16 * ((ln >> 4) & 1) + 4 * (ln & 3)
                                : wn * T::TN + 16 * nb + 4 * (ln & 3);
      b_off[nb] = k * T::BN * 2 + (((n >> 3) ^ T::swz_bk(k)) * 16) + (n & 7) * 2;
    }
  };

  const int KT = (K + T::BK - 1) / T::BK;
  char LDS_AS* lds_base = (char LDS_AS*)lds;
  const uint32_t a_rstep = (uint32_t)(RPA * lda * 2), b_rstep = (uint32_t)(RPB * ldb * 2);
  // Per-lane load offset bases (as gemm_nn_kernel; b_goffr: per-slot B offsets of a non-uniform
  // map), rebuilt at every tile from a freshly read lane index, so that they are not live
  // through a tile's last K step and epilogue, which run at the register limit.
  int a_kc_t;  // a_kc, for the K-tail test
  uint32_t a_goff, b_goff;
  uint32_t b_goffr[T::B_UNIFORM ? 1 : T::RB];
  auto dma_bases = [&]() {
    const int ln = lane_id_fresh();
    const int ar0 = w * (64 / T::CA) + ln / T::CA;
    a_kc_t = 8 * ((ln % T::CA) ^ T::swz_a(ar0));
    a_goff = (uint32_t)((ar0 * lda + a_kc_t) * 2);
    if constexpr (T::B_UNIFORM) {
      const int br0 = w * (64 / T::CB) + ln / T::CB;
      b_goff = (uint32_t)((br0 * ldb + 8 * ((ln % T::CB) ^ T::swz_bk(br0))) * 2);
    } else {
      b_goff = 0;
#pragma unroll
      for (int r = 0; r < T::RB; ++r) {
        const int sl = r * T::NT + w * 64 + ln;
        b_goffr[r] = (uint32_t)(((sl / T::CB) * ldb + 8 * ((sl % T::CB) ^ T::swz_bk(sl / T::CB))) * 2);
      }
    }
  };
  const int64_t b_step = (int64_t)T::BK * ldb * 2;
  // per-tile running load state (K tiles are prepared in order from 0)
  const char* a_ptr;
  const char* b_ptr;
  int64_t a_left, b_left;
  auto start_tile = [&](int tm0, int tn0) {
    dma_bases();
    a_ptr = (const char*)(p.A + (int64_t)tm0 * lda);
    b_ptr = (const char*)(p.B + tn0);
    a_left = ((int64_t)(p.M - 1 - tm0) * lda + K) * 2;
    b_left = ((int64_t)(K - 1) * ldb + p.N - tn0) * 2;
  };
  struct TileDma {
    i32x4 ra, rb;
    uint32_t a_dst, b_dst, a_base;
  };
  auto prep = [&](int t, int stage) {
    const int k0 = t * T::BK;
    TileDma d;
    d.ra = make_rsrc(a_ptr, clip_records(a_left));
    d.rb = make_rsrc(b_ptr, clip_records(b_left));
    a_ptr += T::BK * 2, a_left -= T::BK * 2;
    b_ptr += b_step, b_left -= b_step;
    d.a_dst = lds_addr_of(lds_base) + stage * T::STAGE + w * 64 * 16;
    d.b_dst = d.a_dst + T::A_BYTES;
    const uint32_t a_dead = (uint32_t)(K - 1 - (k0 + a_kc_t)) >> 31;
    d.a_base = a_goff + ((0u - a_dead) & kOobOffset);
    return d;
  };
  auto dma_one = [&](const TileDma& d, int j) {
    if (j < T::RA)
      dma_b128(d.a_dst + j * T::NT * 16, d.ra, d.a_base + j * a_rstep);
    else
      dma_b128(d.b_dst + (j - T::RA) * T::NT * 16, d.rb,
               T::B_UNIFORM ? b_goff + (j - T::RA) * b_rstep : b_goffr[T::B_UNIFORM ? 0 : j - T::RA]);
  };
  auto issue = [&](int t, int stage) {
    const TileDma d = prep(t, stage);
#pragma unroll
    for (int j = 0; j < T::LPT; ++j) dma_one(d, j);
  };

  int b = blockIdx.x;
  int tm, tn;
  tile_of_block(b, tiles_m, tiles_n, 4, &tm, &tn);
  int m0 = __builtin_amdgcn_readfirstlane(tm * T::BM), n0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
  start_tile(m0, n0);
#pragma unroll
  for (int s = 0; s < S; ++s) issue(s, s);
  int pre = 1;
  AccT<T> acc[T::FM][T::FN];
  while (true) {
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
      for (int jj = 0; jj < T::FN; ++jj) acc[i][jj] = AccT<T>{};
    frag_offsets();
    // again after the previous tile's line-store epilogue, which they need not live through
    if constexpr (use_c_lines<T, NT ? kStoreNonTemporal : kStorePlain>()) dma_bases();
    cross_stage<T, false, NST>(lds_base, KT, false, a_off, b_off, acc, prep, dma_one, issue, pre);
    const int nb = b + (int)gridDim.x;
    int nm0 = 0, nn0 = 0;
    if (nb < ntiles) {
      block_sync();  // every wave has read its last fragments of the ring
      tile_of_block(nb, tiles_m, tiles_n, 4, &tm, &tn);
      nm0 = __builtin_amdgcn_readfirstlane(tm * T::BM), nn0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
      start_tile(nm0, nn0);
#pragma unroll
      for (int s = 0; s < S; ++s) issue(s, s);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the stores below
    }
    // epilogue: interior tile, NST 16-byte stores per thread
    if constexpr (use_c_lines<T, NT ? kStoreNonTemporal : kStorePlain>()) {
      store_wave_tile_lines<T, NT ? kStoreNonTemporal : kStorePlain>(
          p.C + (int64_t)(m0 + wm * T::TM) * p.ldc + n0 + wn * T::TN, p.ldc, acc);
    } else
#pragma unroll
    for (int mb = 0; mb < T::FM; ++mb) {
      float* crow = p.C + (int64_t)(m0 + wm * T::TM + T::MF * mb + (lane % T::MF)) * p.ldc + n0 + wn * T::TN;
#pragma unroll
      for (int nb2 = 0; nb2 < T::FN; ++nb2)
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) {
          const int n = T::MF == 32 ? 32 * nb2 + 8 * qq + 4 * (lane >> 5) : 16 * nb2 + 4 * (lane >> 4);
          const f32x4 v = {acc[mb][nb2][4 * qq + 0], acc[mb][nb2][4 * qq + 1], acc[mb][nb2][4 * qq + 2],
                           acc[mb][nb2][4 * qq + 3]};
          if constexpr (NT)
            __builtin_nontemporal_store(v, (f32x4*)(crow + n));
          else
            *(f32x4*)(crow + n) = v;
        }
    }
    if (nb >= ntiles) break;
    b = nb, m0 = nm0, n0 = nn0, pre = 2;
  }
  record_clock(p.clk, 2);
}

// ------------------------------------------------------------------------------------
// Persistent grid over whole tiles and the last round's K-split pieces (same conditions as
// gemm_nn_persistent_kernel, plus a K split of an under-filled last round): the split pieces
// are the grid's final work items, so each workgroup's whole tiles keep the next-tile overlap
// and the split pieces follow without a kernel boundary; their partial tiles go to the
// workspace for reduce_tiles_kernel.  A separate kernel: folding the item bookkeeping into
// gemm_nn_persistent_kernel changed its register allocation (it spilled).
// ------------------------------------------------------------------------------------
template <class T, bool NT>
__global__ __launch_bounds__(T::NT, T::OCC) void gemm_nn_persistent_split_kernel(GemmProblem p, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) char lds[T::STAGES * T::STAGE];
  record_clock(p.clk, 0);
  constexpr int S = T::STAGES;
  constexpr int NQ = T::MF == 32 ? 4 : 1;       // float4 groups per accumulator
  constexpr int NST = T::FM * T::FN * NQ;       // C stores per thread per tile
  const int ntiles = tiles_m * tiles_n;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;

  // staging map and fragment offsets: as gemm_nn_kernel
  constexpr int RPA = T::NT / T::CA, RPB = T::NT / T::CB;
  static_assert(RPA % T::SWZ_A_ROWS == 0 && RPB % T::SWZ_B_ROWS == 0, "round strides must preserve the swizzle");
  const int a_row0 = w * (64 / T::CA) + lane / T::CA;
  const int a_kc = 8 * ((lane % T::CA) ^ T::swz_a(a_row0));
  const int b_row0 = w * (64 / T::CB) + lane / T::CB;
  const int b_nc = 8 * ((lane % T::CB) ^ T::swz_bk(b_row0));
  uint32_t a_off[kMaxOff] = {};
#pragma unroll
  for (int kk = 0; kk < T::KSTEPS; ++kk)
#pragma unroll
    for (int ph = 0; ph < T::APAR; ++ph) {
      const int m = wm * T::TM + ph * T::MF + (lane % T::MF);
      const int chunk = (T::KK / 8) * kk + lane / T::MF;
      a_off[kk * T::APAR + ph] = m * T::BK * 2 + (chunk ^ T::swz_a(m)) * 16;
    }
  uint32_t b_off[kMaxOff] = {};
  {
    const int k = 8 * (lane / T::MF) + ((lane >> 2) & 3);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
      const int n = T::MF == 32 ? wn * T::TN + 32 * nb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)
                                : wn * T::TN + 16 * nb + 4 * (lane & 3);
      b_off[nb] = k * T::BN * 2 + (((n >> 3) ^ T::swz_bk(k)) * 16) + (n & 7) * 2;
    }
  }

  const int KT_all = (K + T::BK - 1) / T::BK;
  // Work items: whole tiles 0 .. whole-1 of the XCD-aware order over all of K, then (K split)
  // item whole + q * split_tiles + j = K range q of tile whole + j, as gemm_nn_kernel numbers
  // its blocks.  Workgroup b takes items b, b + grid, ...: whole tiles first, split pieces last.
  const int ksplit = p.k_splits > 1 ? p.k_splits : 1;
  const int whole = ksplit > 1 ? ntiles - p.split_tiles : ntiles;
  const int nitems = whole + (ksplit > 1 ? p.split_tiles * ksplit : 0);
  struct Item {
    int m0, n0, kt0, kt, q, j;  // tile origin, first K tile and K tiles, split index, split tile
  };
  auto item_of = [&](int it) {
    Item r;
    int bt = it, nsplit = 1;
    r.q = 0, r.j = 0;
    if (it >= whole) {
      const int i2 = it - whole;
      r.q = i2 / p.split_tiles, r.j = i2 - r.q * p.split_tiles;
      bt = whole + r.j, nsplit = ksplit;
    }
    int tmi, tni;
    tile_of_block(bt, tiles_m, tiles_n, 4, &tmi, &tni);
    r.m0 = __builtin_amdgcn_readfirstlane(tmi * T::BM), r.n0 = __builtin_amdgcn_readfirstlane(tni * T::BN);
    r.kt0 = __builtin_amdgcn_readfirstlane((r.q * KT_all) / nsplit);
    r.kt = __builtin_amdgcn_readfirstlane(((r.q + 1) * KT_all) / nsplit) - r.kt0;
    r.q = __builtin_amdgcn_readfirstlane(r.q), r.j = __builtin_amdgcn_readfirstlane(r.j);
    return r;
  };
  char LDS_AS* lds_base = (char LDS_AS*)lds;
  int a_kc_t = a_kc;  // a_kc for the K-tail test, made opaque per tile like the offset bases
  uint32_t a_goff = (uint32_t)((a_row0 * lda + a_kc) * 2);
  uint32_t b_goff = (uint32_t)((b_row0 * ldb + b_nc) * 2);
  const uint32_t a_rstep = (uint32_t)(RPA * lda * 2), b_rstep = (uint32_t)(RPB * ldb * 2);
  const int64_t b_step = (int64_t)T::BK * ldb * 2;
  // per-item running load state (an item's K tiles are prepared in order from its first)
  const char* a_ptr;
  const char* b_ptr;
  int64_t a_left, b_left;
  int kt0 = 0;  // the item's first K tile
  auto start_tile = [&](const Item& it) {
    // The per-lane offset bases pass through an empty asm each tile, so the offsets of a tile's
    // first loads are recomputed from them rather than kept live across the K loop (which
    // runs at the register limit).
    asm volatile("" : "+v"(a_goff), "+v"(b_goff), "+v"(a_kc_t));
    kt0 = it.kt0;
    const int64_t k0 = (int64_t)kt0 * T::BK;
    a_ptr = (const char*)(p.A + (int64_t)it.m0 * lda + k0);
    b_ptr = (const char*)(p.B + k0 * ldb + it.n0);
    a_left = ((int64_t)(p.M - 1 - it.m0) * lda + K - k0) * 2;
    b_left = ((K - 1 - k0) * ldb + p.N - it.n0) * 2;
  };
  struct TileDma {
    i32x4 ra, rb;
    uint32_t a_dst, b_dst, a_base;
  };
  auto prep = [&](int t, int stage) {
    const int k0 = (kt0 + t) * T::BK;
    TileDma d;
    d.ra = make_rsrc(a_ptr, clip_records(a_left));
    d.rb = make_rsrc(b_ptr, clip_records(b_left));
    a_ptr += T::BK * 2, a_left -= T::BK * 2;
    b_ptr += b_step, b_left -= b_step;
    d.a_dst = lds_addr_of(lds_base) + stage * T::STAGE + w * 64 * 16;
    d.b_dst = d.a_dst + T::A_BYTES;
    const uint32_t a_dead = (uint32_t)(K - 1 - (k0 + a_kc_t)) >> 31;
    d.a_base = a_goff + ((0u - a_dead) & kOobOffset);
    return d;
  };
  auto dma_one = [&](const TileDma& d, int j) {
    if (j < T::RA)
      dma_b128(d.a_dst + j * T::NT * 16, d.ra, d.a_base + j * a_rstep);
    else
      dma_b128(d.b_dst + (j - T::RA) * T::NT * 16, d.rb, b_goff + (j - T::RA) * b_rstep);
  };
  auto issue = [&](int t, int stage) {
    const TileDma d = prep(t, stage);
#pragma unroll
    for (int j = 0; j < T::LPT; ++j) dma_one(d, j);
  };

  int b = blockIdx.x;
  Item cur = item_of(b);
  start_tile(cur);
#pragma unroll
  for (int s = 0; s < S; ++s) issue(s, s);
  int pre = 1;
  AccT<T> acc[T::FM][T::FN];
  while (true) {
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
      for (int jj = 0; jj < T::FN; ++jj) acc[i][jj] = AccT<T>{};
    cross_stage<T, false, NST>(lds_base, cur.kt, false, a_off, b_off, acc, prep, dma_one, issue, pre);
    const int nb = b + (int)gridDim.x;
    Item nxt = cur;
    if (nb < nitems) {
      block_sync();  // every wave has read its last fragments of the ring
      nxt = item_of(nb);
      start_tile(nxt);
#pragma unroll
      for (int s = 0; s < S; ++s) issue(s, s);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the stores below
    }
    // epilogue: NST 16-byte stores per thread -- an interior tile of C, or a split piece's whole
    // partial tile, [split tile][split][BM][BN], for reduce_tiles_kernel
    const bool split_item = b >= whole;  // uniform
    float* base = split_item ? p.partials + ((int64_t)cur.j * ksplit + cur.q) * (T::BM * T::BN)
                             : p.C + (int64_t)cur.m0 * p.ldc + cur.n0;
    const int64_t ld = split_item ? T::BN : p.ldc;
    if constexpr (use_c_lines<T, NT ? kStoreNonTemporal : kStorePlain>()) {
      store_wave_tile_lines<T, NT ? kStoreNonTemporal : kStorePlain>(base + (int64_t)wm * T::TM * ld + wn * T::TN, ld,
                                                                      acc);
    } else
#pragma unroll
    for (int mb = 0; mb < T::FM; ++mb) {
      float* crow = base + (int64_t)(wm * T::TM + T::MF * mb + (lane % T::MF)) * ld + wn * T::TN;
#pragma unroll
      for (int nb2 = 0; nb2 < T::FN; ++nb2)
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) {
          const int n = T::MF == 32 ? 32 * nb2 + 8 * qq + 4 * (lane >> 5) : 16 * nb2 + 4 * (lane >> 4);
          const f32x4 v = {acc[mb][nb2][4 * qq + 0], acc[mb][nb2][4 * qq + 1], acc[mb][nb2][4 * qq + 2],
                           acc[mb][nb2][4 * qq + 3]};
          if constexpr (NT)
            __builtin_nontemporal_store(v, (f32x4*)(crow + n));
          else
            *(f32x4*)(crow + n) = v;
        }
    }
    if (nb >= nitems) break;
    b = nb, cur = nxt, pre = 2;
  }
  record_clock(p.clk, 2);
}

// ------------------------------------------------------------------------------------
// Folded (5-D contraction) kernel: each GEMM axis is a (hi, lo) pair of sub-indices with
// its own strides per operand (mmm.h, mmm_contract_desc).  Operands are gathered element by
// element into the same swizzled LDS stages and multiplied by the same MFMA core; the
// output is scattered through the C strides.  A lane owns 32 consecutive m across the wave,
// so an output whose low m sub-index is contiguous (the reference's Out[m][b][r], r
// contiguous, mmmTensor.cpp:251) is written in 128-byte runs.
// BKM = true stages B as [BN][64] (for operands whose k_lo stride is 1, e.g. the
// reference's TN Input[b][n][l]); BKM = false stages B as [64][BN].
// ------------------------------------------------------------------------------------
__device__ __forceinline__ int64_t fold_off(int i, int lo, int64_t s_hi, int64_t s_lo) {
  return (int64_t)(i / lo) * s_hi + (int64_t)(i % lo) * s_lo;
}

// X at the 8 consecutive fold indices i .. i+7 past base (index j at base + fold_off(j, ...)),
// with one division for i and the rest stepped (the low sub-index carrying into the high one);
// indices at or past `end` read as zero, from kZeroHalves (end = 0: all of them).
__device__ __forceinline__ half8 gather8(const _Float16* X, int64_t base, int i, int end, int lo, int64_t s_hi,
                                         int64_t s_lo) {
  half8 v;
  int l = i % lo;
  int64_t off = base + (int64_t)(i / lo) * s_hi + (int64_t)l * s_lo;
  const int64_t carry = s_hi - (int64_t)lo * s_lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = *(i + e < end ? X + off : kZeroHalves);
    off += s_lo;
    if (++l == lo) l = 0, off += carry;
  }
  return v;
}

// gather8 for a contiguous low sub-index (s_lo == 1) whose extent, high stride and row bases are
// multiples of G, with X + base 2G-byte aligned: groups of G elements never cross a block, so each
// is one 2G-byte load (end is then a multiple of G too: a group is wholly in or out).  A group
// past `end` loads zeros from kZeroHalves, as in gather8.
template <int G>
__device__ __forceinline__ half8 gather8_vec(const _Float16* X, int64_t base, int i, int end, int lo, int64_t s_hi) {
  typedef _Float16 halfG __attribute__((ext_vector_type(G)));
  half8 v;
  int l = i % lo;
  int64_t off = base + (int64_t)(i / lo) * s_hi + l;
#pragma unroll
  for (int j = 0; j < 8 / G; ++j) {
    const halfG g = *(const halfG*)(i + j * G < end ? X + off : kZeroHalves);
#pragma unroll
    for (int e = 0; e < G; ++e) v[j * G + e] = g[e];
    off += G, l += G;
    if (l == lo) l = 0, off += s_hi - lo;
  }
  return v;
}

// Widest group (8, 4, 2 or 1 elements) gather8_vec may use for an operand whose fold index
// (low extent lo, strides s_hi / s_lo) is contiguous, given every row base's strides r0, r1.
__device__ __forceinline__ int gather_width(const void* X, int lo, int64_t s_hi, int64_t s_lo, int64_t r0, int64_t r1) {
  if (s_lo != 1) return 1;
#pragma unroll
  for (int g = 8; g > 1; g /= 2)
    if (lo % g == 0 && s_hi % g == 0 && r0 % g == 0 && r1 % g == 0 && (uintptr_t)X % (2 * g) == 0) return g;
  return 1;
}

// gather8 at group width G (1: element by element through the strides).
template <int G>
__device__ __forceinline__ half8 gather8_g(const _Float16* X, int64_t base, int i, int end, int lo, int64_t s_hi,
                                           int64_t s_lo) {
  if constexpr (G == 1)
    return gather8(X, base, i, end, lo, s_hi, s_lo);
  else
    return gather8_vec<G>(X, base, i, end, lo, s_hi);
}

// f(std::integral_constant<int, gw>) for a uniform group width gw: the branch is scalar and is taken
// once per operand and stage, so each arm holds all of that operand's loads of the stage, which go
// out together (a branch per chunk kept each chunk's loads waiting in their own arm).
template <class F>
__device__ __forceinline__ void with_width(int gw, F&& f) {
  if (gw == 8)
    f(std::integral_constant<int, 8>{});
  else if (gw == 4)
    f(std::integral_constant<int, 4>{});
  else if (gw == 2)
    f(std::integral_constant<int, 2>{});
  else
    f(std::integral_constant<int, 1>{});
}

template <class T, bool BKM>
__global__ __launch_bounds__(T::NT, 1) void gemm_fold_kernel(FoldProblem p, int tiles_m, int tiles_n) {
  static_assert(T::MF == 32, "the folded kernels use 32x32 fragments");
  __shared__ __attribute__((aligned(1024))) char lds[2 * T::STAGE];
  static_assert(T::STAGES == 2 && T::BK == 64, "the folded path double-buffers 64-deep stages");
  static_assert(!BKM || T::BN * 8 % T::NT == 0, "K-major B chunks must divide over threads");
  constexpr int RBK = BKM ? T::BN * 8 / T::NT : T::RB;

  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, 4, &tm, &tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * T::BM), n0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int M = p.M, N = p.N, K = p.K;

  int a_row[T::RA], a_kc[T::RA];
  int64_t a_base[T::RA];
#pragma unroll
  for (int r = 0; r < T::RA; ++r) {
    const int s = r * T::NT + w * 64 + lane;
    const int m = s / T::CA;
    a_row[r] = m;
    a_kc[r] = 8 * ((s % T::CA) ^ T::swz_a(m));
    a_base[r] = (m0 + m < M) ? fold_off(m0 + m, p.m_lo, p.am[0], p.am[1]) : 0;
  }
  int b_row[RBK], b_c[RBK];
  int64_t b_base[RBK];
#pragma unroll
  for (int r = 0; r < RBK; ++r) {
    const int s = r * T::NT + w * 64 + lane;
    if constexpr (BKM) {
      const int n = s / 8;
      b_row[r] = n;  // tile column n; chunk holds 8 consecutive k
      b_c[r] = 8 * ((s % 8) ^ T::swz_a(n));
      b_base[r] = (n0 + n < N) ? fold_off(n0 + n, p.n_lo, p.bn[0], p.bn[1]) : 0;
    } else {
      const int k = s / T::CB;
      b_row[r] = k;  // tile row k; chunk holds 8 consecutive n
      b_c[r] = 8 * ((s % T::CB) ^ swz_b(k));
      b_base[r] = 0;
    }
  }

  uint32_t a_off[kMaxOff] = {};
  {
    const int m = wm * T::TM + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < T::KSTEPS; ++kk) a_off[kk] = m * T::BK * 2 + ((2 * kk + (lane >> 5)) ^ T::swz_a(m)) * 16;
  }
  uint32_t b_off[kMaxOff] = {};
  if constexpr (BKM) {
    const int n = wn * T::TN + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < T::KSTEPS; ++kk) b_off[kk] = n * T::BK * 2 + ((2 * kk + (lane >> 5)) ^ T::swz_a(n)) * 16;
  } else {
    const int k = 8 * (lane >> 5) + ((lane >> 2) & 3);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
      const int n = wn * T::TN + 32 * nb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      b_off[nb] = k * T::BN * 2 + (((n >> 3) ^ swz_b(k)) * 16) + (n & 7) * 2;
    }
  }

  AccT<T> acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = f32x16{};

  const _Float16* A = (const _Float16*)p.A;
  const _Float16* B = (const _Float16*)p.B;
  // group widths of the gathers: A along k (row bases from the m strides); B along k (K-major,
  // column bases from the n strides) or along n (row bases from the k strides)
  const int a_gw = gather_width(A, p.k_lo, p.ak[0], p.ak[1], p.am[0], p.am[1]);
  const int b_gw = BKM ? gather_width(B, p.k_lo, p.bk[0], p.bk[1], p.bn[0], p.bn[1])
                       : gather_width(B, p.n_lo, p.bn[0], p.bn[1], p.bk[0], p.bk[1]);
  u32x4 ra[T::RA], rb[RBK];
  auto load = [&](int t) {
    const int k0 = t * T::BK;
    // Rows, columns and K rows past the operands gather with end = 0 (every element from
    // kZeroHalves): no load sits under a lane condition.
    with_width(a_gw, [&](auto g) {
      constexpr int G = decltype(g)::value;
#pragma unroll
      for (int r = 0; r < T::RA; ++r) {
        const int k = k0 + a_kc[r];
        ra[r] = __builtin_bit_cast(
            u32x4, gather8_g<G>(A, a_base[r], k, m0 + a_row[r] < M ? K : 0, p.k_lo, p.ak[0], p.ak[1]));
      }
    });
    with_width(b_gw, [&](auto g) {
      constexpr int G = decltype(g)::value;
#pragma unroll
      for (int r = 0; r < RBK; ++r) {
        if constexpr (BKM) {
          const int k = k0 + b_c[r];
          rb[r] = __builtin_bit_cast(
              u32x4, gather8_g<G>(B, b_base[r], k, n0 + b_row[r] < N ? K : 0, p.k_lo, p.bk[0], p.bk[1]));
        } else {
          const int k = k0 + b_row[r], n = n0 + b_c[r];
          rb[r] = __builtin_bit_cast(u32x4, gather8_g<G>(B, fold_off(k < K ? k : 0, p.k_lo, p.bk[0], p.bk[1]), n,
                                                         k < K ? N : 0, p.n_lo, p.bn[0], p.bn[1]));
        }
      }
    });
  };
  char LDS_AS* lds_base = (char LDS_AS*)lds;
  auto store = [&](int stage) {
    char LDS_AS* a_dst = lds_base + stage * T::STAGE + (w * 64 + lane) * 16;
    char LDS_AS* b_dst = lds_base + stage * T::STAGE + T::A_BYTES + (w * 64 + lane) * 16;
#pragma unroll
    for (int r = 0; r < T::RA; ++r) *(u32x4 LDS_AS*)(a_dst + r * T::NT * 16) = ra[r];
#pragma unroll
    for (int r = 0; r < RBK; ++r) *(u32x4 LDS_AS*)(b_dst + r * T::NT * 16) = rb[r];
  };

  const int KT = (K + T::BK - 1) / T::BK;
  load(0);
  store(0);
  block_sync();
  for (int t = 0; t < KT; t += 2) {
    if (t + 1 < KT) load(t + 1);
    compute_stage<T, BKM>(lds_base, lds_base + T::A_BYTES, a_off, b_off, acc, NoHook{});
    if (t + 1 < KT) store(1);
    block_sync();
    if (t + 1 < KT) {
      if (t + 2 < KT) load(t + 2);
      compute_stage<T, BKM>(lds_base + T::STAGE, lds_base + T::STAGE + T::A_BYTES, a_off, b_off, acc, NoHook{});
      if (t + 2 < KT) store(0);
      block_sync();
    }
  }

  float* C = p.C;
#pragma unroll
  for (int mb = 0; mb < T::FM; ++mb) {
    const int m = m0 + wm * T::TM + 32 * mb + (lane & 31);
    if (m >= M) continue;
    const int64_t crow = fold_off(m, p.m_lo, p.cm[0], p.cm[1]);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = n0 + wn * T::TN + 32 * nb + 8 * q + 4 * (lane >> 5) + e;
          if (n < N) C[crow + fold_off(n, p.n_lo, p.cn[0], p.cn[1])] = acc[mb][nb][4 * q + e];
        }
  }
}

// ------------------------------------------------------------------------------------
// Folded problem on the direct-to-LDS path, for folds whose K sub-index is contiguous in
// both operands (k_lo stride 1) and whose K tiles never straddle a k_hi boundary -- the
// reference's contraction: G[r][n][m][l] x Input[b][n][l] -> Out[m][b][r] (mmmTensor.cpp).
//  * A row m = (m_hi, m_lo) starts at m_hi*am0 + m_lo*am1; a 64-deep K tile at k0 adds
//    (k0 / k_lo)*ak0 + k0 % k_lo and is contiguous from there, so each 16-byte chunk is one
//    DMA load at a per-lane row base plus a uniform tile offset.
//  * B is K-major (Input[b][n][l]: column b of B is contiguous in k), staged [BN][64] like A
//    and read with ds_read_b128 fragments.
//  * Rows past M and columns past N are pushed out of the descriptor range (read as zero).
//  * LANEK: folds whose K tiles cross k_hi blocks (k_lo a multiple of 8 but not of 64, e.g. an
//    rt_l of 120): each lane keeps its own chunk's (k_hi, k_rem) and offsets, advanced by one
//    tile per step; a 16-byte chunk never crosses a block.  K is then a multiple of 8 but may
//    end inside the last K tile: that tile's chunks at or past K are pushed out of the
//    descriptor range too.  Otherwise (and always with WIDE) K is a multiple of 64.
//  * WIDE: operands whose offsets pass the buffer's 32 bits (a G of more than 1 GiB) are read
//    through 64-bit per-lane addresses instead (global_load_lds_dwordx4).  Rows past M and
//    columns past N then load row M-1 / column N-1: they feed only accumulators of rows and
//    columns the epilogue never stores.
//  * Output scattered through the C strides: lanes own consecutive m, so an output whose
//    m_lo is contiguous (Out[m][b][r]) is written in 128-byte runs.
// ------------------------------------------------------------------------------------
template <class T, bool NT, bool WIDE, bool LANEK>
__global__ __launch_bounds__(T::NT, T::OCC) void gemm_fold_dma_kernel(FoldProblem p, int tiles_m, int tiles_n,
                                                                      uint32_t a_bytes, uint32_t b_bytes) {
  __shared__ __attribute__((aligned(1024))) char lds[T::STAGES * T::STAGE];
  static_assert(T::BN * T::CA % T::NT == 0, "K-major B chunks must divide over threads");
  constexpr int RBK = T::BN * T::CA / T::NT;  // K-major B chunks per thread
  static_assert(RBK == T::RB, "the K-major B stage holds as many chunks as the N-contiguous one");
  constexpr int RPA = T::NT / T::CA;  // rows per round (A and B alike)
  static_assert(RPA % T::SWZ_A_ROWS == 0, "round strides must preserve the swizzle");

  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, 4, &tm, &tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * T::BM), n0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int M = p.M, N = p.N, K = p.K;

  const int row0 = w * (64 / T::CA) + lane / T::CA;
  const int kc = 8 * ((lane % T::CA) ^ T::swz_a(row0));
  const int kc_row = LANEK ? 0 : kc;  // LANEK: the chunk's K offset is kept per lane, apart
  uint32_t a_voff[WIDE ? 1 : T::RA], b_voff[WIDE ? 1 : RBK];
  const char* a_src[WIDE ? T::RA : 1];
  const char* b_src[WIDE ? RBK : 1];
#pragma unroll
  for (int r = 0; r < T::RA; ++r) {
    const int m = m0 + row0 + r * RPA;
    if constexpr (WIDE)
      a_src[r] = (const char*)p.A + (fold_off(m < M ? m : M - 1, p.m_lo, p.am[0], p.am[1]) + kc_row) * 2;
    else
      a_voff[r] = m < M ? (uint32_t)((fold_off(m, p.m_lo, p.am[0], p.am[1]) + kc_row) * 2) : kOobOffset;
  }
#pragma unroll
  for (int r = 0; r < RBK; ++r) {
    const int n = n0 + row0 + r * RPA;
    if constexpr (WIDE)
      b_src[r] = (const char*)p.B + (fold_off(n < N ? n : N - 1, p.n_lo, p.bn[0], p.bn[1]) + kc_row) * 2;
    else
      b_voff[r] = n < N ? (uint32_t)((fold_off(n, p.n_lo, p.bn[0], p.bn[1]) + kc_row) * 2) : kOobOffset;
  }

  // fragment read offsets: A rows and K-major B columns share the layout (lane l reads row
  // l % MF, k chunk l / MF of each K-step)
  uint32_t a_off[kMaxOff] = {}, b_off[kMaxOff] = {};
#pragma unroll
  for (int kk = 0; kk < T::KSTEPS; ++kk)
#pragma unroll
    for (int ph = 0; ph < T::APAR; ++ph) {
      const int m = wm * T::TM + ph * T::MF + (lane % T::MF), n = wn * T::TN + ph * T::MF + (lane % T::MF);
      const int chunk = (T::KK / 8) * kk + lane / T::MF;
      a_off[kk * T::APAR + ph] = m * T::BK * 2 + (chunk ^ T::swz_a(m)) * 16;
      b_off[kk * T::APAR + ph] = n * T::BK * 2 + (chunk ^ T::swz_a(n)) * 16;
    }

  AccT<T> acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = AccT<T>{};

  char LDS_AS* lds_base = (char LDS_AS*)lds;
  const i32x4 ra = make_rsrc(p.A, a_bytes);
  const i32x4 rb = make_rsrc(p.B, b_bytes);
  // K tile t starts at k0 = t * BK = (k_hi, k_rem): uniform offsets k_hi * ak0 + k_rem (A) and
  // k_hi * bk0 + k_rem (B), advanced per tile (tiles are prepared in order).
  using KOff = std::conditional_t<WIDE, int64_t, uint32_t>;
  struct FoldDma {
    uint32_t a_dst, b_dst;
    KOff ka, kb;
  };
  // LANEK: k_rem is this lane's chunk position inside its k_hi block; the row offsets (or
  // addresses) carry the chunk's K offset and advance by one K tile per prep (tiles are
  // prepared in order, and each tile's loads are issued before the next prep).
  int k_hi = 0, k_rem = 0;
  KOff a_wrap = 0, b_wrap = 0;
  if constexpr (LANEK) {
    k_hi = kc / p.k_lo, k_rem = kc - k_hi * p.k_lo;
    const int64_t ka0 = ((int64_t)k_hi * p.ak[0] + k_rem) * 2, kb0 = ((int64_t)k_hi * p.bk[0] + k_rem) * 2;
#pragma unroll
    for (int r = 0; r < T::RA; ++r) {
      if constexpr (WIDE) a_src[r] += ka0;
      else a_voff[r] += (uint32_t)ka0;
    }
#pragma unroll
    for (int r = 0; r < RBK; ++r) {
      if constexpr (WIDE) b_src[r] += kb0;
      else b_voff[r] += (uint32_t)kb0;
    }
    a_wrap = (KOff)((p.ak[0] - p.k_lo) * 2), b_wrap = (KOff)((p.bk[0] - p.k_lo) * 2);
  }
  auto prep = [&](int t, int stage) {
    FoldDma d;
    if constexpr (LANEK) {
      d.ka = 0, d.kb = 0;
      if (t > 0) {
        KOff da = T::BK * 2, db = T::BK * 2;
        k_rem += T::BK;
        while (k_rem >= p.k_lo) k_rem -= p.k_lo, da += a_wrap, db += b_wrap;
#pragma unroll
        for (int r = 0; r < T::RA; ++r) {
          if constexpr (WIDE) a_src[r] += da;
          else a_voff[r] += da;
        }
#pragma unroll
        for (int r = 0; r < RBK; ++r) {
          if constexpr (WIDE) b_src[r] += db;
          else b_voff[r] += db;
        }
      }
      if constexpr (!WIDE) {
        // K tail (the last tile only; nothing is loaded after it, so the offsets may stay out
        // of range; a chunk past K may sit in a k_hi block past the fold's, whose offset means
        // nothing, so it is replaced, not moved)
        if (t * T::BK + kc >= K) {
#pragma unroll
          for (int r = 0; r < T::RA; ++r) a_voff[r] = kOobOffset;
#pragma unroll
          for (int r = 0; r < RBK; ++r) b_voff[r] = kOobOffset;
        }
      }
    } else {
      d.ka = (KOff)(((int64_t)k_hi * p.ak[0] + k_rem) * 2);
      d.kb = (KOff)(((int64_t)k_hi * p.bk[0] + k_rem) * 2);
      k_rem += T::BK;
      if (k_rem == p.k_lo) k_rem = 0, ++k_hi;
    }
    d.a_dst = lds_addr_of(lds_base) + stage * T::STAGE + w * 64 * 16;
    d.b_dst = d.a_dst + T::A_BYTES;
    return d;
  };
  auto dma_one = [&](const FoldDma& d, int j) {
    if constexpr (WIDE) {
      if (j < T::RA)
        dma_b128_flat(d.a_dst + j * T::NT * 16, a_src[j] + d.ka);
      else
        dma_b128_flat(d.b_dst + (j - T::RA) * T::NT * 16, b_src[j - T::RA] + d.kb);
    } else {
      if (j < T::RA)
        dma_b128(d.a_dst + j * T::NT * 16, ra, a_voff[j] + d.ka);
      else
        dma_b128(d.b_dst + (j - T::RA) * T::NT * 16, rb, b_voff[j - T::RA] + d.kb);
    }
  };
  auto issue_tile = [&](int t, int stage) {
    const FoldDma d = prep(t, stage);
#pragma unroll
    for (int j = 0; j < T::LPT; ++j) dma_one(d, j);
  };
  cross_stage<T, true>(lds_base, (K + T::BK - 1) / T::BK, false, a_off, b_off, acc, prep, dma_one, issue_tile);

  // epilogue: lane owns row m and columns n .. n+3 of each accumulator group, scattered
  // through the C strides (MF = 32: m = l % 32, n = 32*nb + 8*q + 4*(l/32); MF = 16:
  // m = l % 16, n = 16*nb + 4*(l/16)).  A group's first column n is a multiple of 4, so when
  // n_lo is too, its 4 columns share one n_hi block and sit cn[1] apart: one fold_off per
  // group (computed once per lane) instead of one division per element.
  constexpr int NQ = T::MF == 32 ? 4 : 1;
  float* C = p.C;
  const bool quad = p.n_lo % 4 == 0;  // uniform
  const int64_t cn1 = p.cn[1];
  int64_t coff[T::FN][NQ];
#pragma unroll
  for (int nb = 0; nb < T::FN; ++nb)
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int n = n0 + wn * T::TN + (T::MF == 32 ? 32 * nb + 8 * q + 4 * (lane >> 5) : 16 * nb + 4 * (lane >> 4));
      coff[nb][q] = n < N ? fold_off(n, p.n_lo, p.cn[0], p.cn[1]) : 0;
    }
#pragma unroll
  for (int mb = 0; mb < T::FM; ++mb) {
    const int m = m0 + wm * T::TM + T::MF * mb + (lane % T::MF);
    if (m >= M) continue;
    float* crow = C + fold_off(m, p.m_lo, p.cm[0], p.cm[1]);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb)
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int n = n0 + wn * T::TN + (T::MF == 32 ? 32 * nb + 8 * q + 4 * (lane >> 5) : 16 * nb + 4 * (lane >> 4));
        if (quad && n + 3 < N) {
          float* c = crow + coff[nb][q];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (NT)
              __builtin_nontemporal_store(acc[mb][nb][4 * q + e], c + e * cn1);
            else
              c[e * cn1] = acc[mb][nb][4 * q + e];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) crow[fold_off(n + e, p.n_lo, p.cn[0], p.cn[1])] = acc[mb][nb][4 * q + e];
        }
      }
  }
}

// ------------------------------------------------------------------------------------
// Host-side launch
// ------------------------------------------------------------------------------------
// C tile = sum over the K splits, in split order (fixed order: deterministic), of the partial
// tiles written by gemm_nn_kernel for split tile j (tile `first + j` of the XCD-aware order);
// one thread per 4 consecutive columns.
template <int BM, int BN>
__global__ __launch_bounds__(256) void reduce_tiles_kernel(GemmProblem p, int tiles_m, int tiles_n, int first,
                                                           int splits) {
  constexpr int F4 = BM * BN / 4;  // float4s per tile
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int j = (int)(g / F4), e = (int)(g % F4);
  int tm, tn;
  tile_of_block(first + j, tiles_m, tiles_n, 4, &tm, &tn);
  const int r = e / (BN / 4), c = 4 * (e % (BN / 4));
  const int m = tm * BM + r, n = tn * BN + c;
  if (m >= p.M || n >= p.N) return;
  const f32x4* src = (const f32x4*)(p.partials + (int64_t)j * splits * (BM * BN)) + e;
  f32x4 sum = src[0];
  for (int s = 1; s < splits; ++s) sum += src[(int64_t)s * F4];
  float* crow = p.C + (int64_t)m * p.ldc;
  if (p.c_vec4 && n + 3 < p.N) {
    *(f32x4*)(crow + n) = sum;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < p.N) crow[n + i] = sum[i];
  }
}

// Shortest K for which the multi-round kernels store C non-temporally in half lines (see their
// launches).
constexpr int kNtMinK = 4096;

template <class T, bool GENERIC>
static hipError_t launch_nn(const GemmProblem& p, hipStream_t stream) {
  const int tiles_m = (p.M + T::BM - 1) / T::BM;
  const int tiles_n = (p.N + T::BN - 1) / T::BN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int splits = p.k_splits > 1 ? p.k_splits : 1;
  const int64_t split_tiles = splits > 1 ? p.split_tiles : 0;
  if (split_tiles < 0 || split_tiles > tiles) return hipErrorInvalidValue;
  const int64_t blocks = tiles - split_tiles + split_tiles * splits;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  // A one-round grid writes all of C after its last K step, with nothing left to overlap, and
  // system-scope write-through stores (sc0 sc1) drain that burst faster.  As half lines they won
  // only where C outgrew the eight XCDs' L2 (32 MB; 256x256 tile: 8192 x 2048 x 2048 +3.1%,
  // 4096^3 +1.3%, but 2048^3 -4.7%, 1024^3 -7.5%); as whole lines (store_wave_tile_lines) they win
  // at every size measured on MI355X, against L2-allocating half lines: 2048^2 x 1024 +11%,
  // 2048^3 +6.7%, 1536^3 +5%, 2048^2 x 4096 +4.4%, 8192 x 1024 x 8192 +2.8%, 1024 x 8192 x 8192
  // +2.1%, 1024^3 +1.5-2.3%, 512^3 +-0.  Not with a K split (as half lines: 3072^3 on 128x256
  // -8.8%) or for rows of an odd ldc (-9%).
  const bool c16 = ((uintptr_t)p.C & 15) == 0 && p.ldc % 4 == 0;
  const bool wt = splits == 1 && blocks <= 256 * T::OCC && c16 &&
                  (c_lines_ok<T>() || (double)p.M * p.N * 4.0 > 32.0 * (1 << 20));
  // (Multi-round grids keep plain stores: non-temporal whole lines there measured -4.6% at
  // 5000^3, -1% at 4096^3 on 256x128, +7% at 8192^2 x 2048 on 256x128, +-0 elsewhere.)
  // the direct-to-LDS kernel with or without the unaligned-tail code
  auto launch_dma = [&](auto cpol) {
    constexpr int CP = decltype(cpol)::value;
    if (p.tail_regs)
      hipLaunchKernelGGL((gemm_nn_kernel<T, false, CP, true>), dim3((unsigned)blocks), dim3(T::NT), 0, stream, p,
                         tiles_m, tiles_n);
    else
      hipLaunchKernelGGL((gemm_nn_kernel<T, false, CP, false>), dim3((unsigned)blocks), dim3(T::NT), 0, stream, p,
                         tiles_m, tiles_n);
  };
  if constexpr (GENERIC) {
    (void)wt;
    (void)launch_dma;
    hipLaunchKernelGGL((gemm_nn_kernel<T, true>), dim3((unsigned)blocks), dim3(T::NT), 0, stream, p, tiles_m, tiles_n);
  } else if constexpr (c_lines_ok<T>() || (T::BM == 256 && T::BN == 256)) {
    if (wt)
      launch_dma(std::integral_constant<int, kStoreWriteThrough>{});
    else
      launch_dma(std::integral_constant<int, kStorePlain>{});
  } else {
    (void)wt;
    launch_dma(std::integral_constant<int, kStorePlain>{});
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const int64_t per_tile = T::BM * T::BN / 4 / 256;  // blocks of 256 float4s per tile
  hipLaunchKernelGGL((reduce_tiles_kernel<T::BM, T::BN>), dim3((unsigned)(split_tiles * per_tile)), dim3(256), 0,
                     stream, p, tiles_m, tiles_n, (int)(tiles - split_tiles), splits);
  return hipGetLastError();
}

// Direct-to-LDS path: K step, ring depth and wave grid (compile-time).  Measured on MI355X
// at 8192^3 (median TFLOP/s): 64 x 2 stages with 2 x 4 waves (two waves per SIMD, so one
// wave's MFMAs cover the other's barrier and LDS waits) 1126; the same with 2 x 2 waves
// 1077; 32 x 4 or 32 x 5 stages 1055-1106 -- deeper prefetch does not pay, latency of the
// operand fetch is not the limiter.  MFMA shape of the 256x256 tile: 16x16x32 (measured at
// 8192^3 under sustained load, it runs at a 16% higher power-limited clock than 32x32x16 -- a
// quarter of the accumulator traffic per instruction -- and is 2-9% faster across 4096^3 ..
// 16384^2 x 4096).
constexpr int kDmaBK = 64;
using Tile256 = Tile<256, 256, 2, 4, kDmaBK, 2, 1, 16>;
// The 128-wide tiles run eight 16x16x32 waves (two per SIMD) like the 256x256 tile.  Measured on
// MI355X against the four-wave 32x32x16 versions they replace (interleaved runs, same box):
//   128x256 (2 x 4 waves of 64x64, 3 x 48 KB ring): 2048 x 4096 x 4096 858 -> 939 TFLOP/s,
//     8192 x 1024 x 8192 1022 -> 1136, 1024 x 8192 x 8192 1030 -> 1145, 4096^3 1063 -> 1106,
//     8192^3 1120 -> 1136, 3072^3 830 -> 827;
//   256x128 (4 x 2 waves of 64x64, 3 x 48 KB ring): 2048 x 4096 x 4096 926 -> 1039,
//     8192 x 1024 x 8192 1023 -> 1160, 4096^3 1008 -> 1109, 8192^3 1034 -> 1137;
//   128x128 in multi-round grids (2 x 4 waves of 64x32, 2 x 32 KB ring, two workgroups per CU):
//     4096^3 971 -> 1007, 6144^2 x 2048 918 -> 952, 8192^3 1032 -> 1048, 3072^3 738 -> 764.
// With four waves a one-round launch holds one wave per SIMD, and nothing covers a wave's
// barrier and LDS waits.
template <int BM, int BN>
struct DmaCfg {  // 128x128
  using T = Tile<BM, BN, 2, 4, 64, 2, 2, 16>;
};
// 64x64: for grids too small to fill the chip with 128x128 tiles (1024^3 is 64 of those, 256
// of these).  Four waves of 32x32 (2 x 2 16x16x32 fragments each) on a 3-stage ring (48 KB).
// Measured on MI355X against the 128x128 tile (interleaved runs, same box): 1024^3 139 -> 200
// TFLOP/s, 512^3 23.8 -> 30.4, 768^3 67 -> 96, 1024^2 x 2048 207 -> 297; it loses where 128x128
// tiles fill a round or split well (1536^3 333 vs 365, 2048^3 515 vs 640).  8 stages (K = 512
// in flight at once) ran 3-7% slower than 3 or 4; two workgroups per CU at 2 stages, slower still.
template <>
struct DmaCfg<64, 64> {
  using T = Tile<64, 64, 2, 2, 64, 3, 1, 16>;
};
// 192x192: 16 x 16 tiles fill one round exactly at 3072 x 3072, where 256x256 tiles leave 112
// of the 256 CUs idle, and whole multiples of 256 tiles run as the persistent grid (6144^2 x
// 2048: 1024 tiles, four rounds, 1006 -> 1047 TFLOP/s over one workgroup per tile, against 926
// for 256x256 tiles' 2.25 rounds; 3072 x 6144 x 2048 996 -> 1030, against 888).  Eight waves of
// 96x48 (6 x 3 16x16x32 fragments), a 3-stage ring of 48 KB stages; rows of 24 chunks use the
// per-slot B staging map.  Measured on MI355X (interleaved runs, same box): 3072^3 763 -> 1007
// TFLOP/s against the 256x256 tile, 3072^2 x 8192 963 -> 1159, 4357 x 4095 x 4111 805 -> 885;
// 8192^3 1172 against 1380 (per-CU rate 0.85).
template <>
struct DmaCfg<192, 192> {
  using T = Tile<192, 192, 2, 4, 64, 3, 1, 16>;
};
template <>
struct DmaCfg<256, 256> {
  using T = Tile256;
};
template <>
struct DmaCfg<256, 128> {
  using T = Tile<256, 128, 4, 2, 64, 3, 1, 16>;
};
template <>
struct DmaCfg<128, 256> {
  using T = Tile<128, 256, 2, 4, 64, 3, 1, 16>;
};
template <int BM, int BN>
using DmaTile = typename DmaCfg<BM, BN>::T;
// The 128x128 tile in a launch of at most one round (one workgroup per CU): no second
// workgroup on the CU covers the load latency, so the ring is one stage deeper (3 x 32 KB).
// Measured on MI355X (interleaved runs, same box), first with four waves: 2048^3 567 -> 624
// TFLOP/s, 2048^2 x 4096 720 -> 791, 1024^2 x 8192 (K split) 508 -> 540, 4 stages no better
// than 3; then eight waves of 16x16x32 instead of four of 32x32x16: 2048^3 601 -> 645, 2048^2 x
// 4096 760 -> 822, 1024^2 x 8192 538 -> 564, 512 x 8192 x 8192 783 -> 852.
using DeepTile128 = Tile<128, 128, 2, 4, 64, 3, 1, 16>;
// The folded direct-to-LDS kernel: the 256x256 tile's waves and ring.
using FoldDmaTile = Tile256;
// Register-staged path: 64-deep stages, double-buffered.
template <int BM, int BN>
using RegTile = Tile<BM, BN, 2, 2, 64, 2>;

// True when the direct-to-LDS path can serve the problem: fp16 operands (2-byte aligned), and
// per-tile byte offsets that fit the 32-bit buffer offsets.  Rows that are not 16-byte aligned
// (odd lda or ldb, e.g. the 4097 x 4095 x 4111 configuration) are read by 16-byte buffer loads
// at 2-byte-aligned addresses: this relies on the unaligned buffer access the gfx9 family
// serves in ROCm's default (unaligned) memory mode, which MI355X boxes run -- the exact
// full-size ragged tests cover it.  A platform without unaligned buffer access must send
// 2-byte-aligned rows to the register-staged path (return false for them here).
static bool dma_ok(const GemmProblem& p, int bm) {
  const uintptr_t a = (uintptr_t)p.A, b = (uintptr_t)p.B;
  if ((a & 1) || (b & 1)) return false;
  if ((int64_t)bm * p.lda * 2 >= (int64_t)kOobOffset) return false;
  if ((int64_t)kDmaBK * p.ldb * 2 >= (int64_t)kOobOffset) return false;
  return true;
}

// True when every DMA chunk of the last K tile also lies wholly inside the operands (K and
// N multiples of 8, 16-byte aligned rows); otherwise gemm_nn_kernel patches that tile's
// straddling chunks or gathers it through VGPRs, and the persistent kernels do not run.
static bool tail_aligned(const GemmProblem& p) {
  const uintptr_t a = (uintptr_t)p.A, b = (uintptr_t)p.B;
  return !((a & 15) || (b & 15) || p.lda % 8 || p.ldb % 8 || p.K % 8 || p.N % 8);
}

bool gemm_nn_direct_to_lds(const GemmProblem& p, int tile_id) {
  return dma_ok(p, tile_bm(tile_id));
}

// K split for a tile launch whose last round of 256 workgroups (one per CU) is less than half
// full -- the whole grid when it is one small round: the last round's tiles each run as
// `splits` K ranges, enough to refill about one workgroup per CU (at least 8 64-deep K tiles
// each, at most 16, partial tiles within the stream workspace).  Taken only when the round
// time it saves exceeds the reduction's traffic (each split writes its partial tile; the
// reduction reads them and writes C) and launch.  Direct-to-LDS path only.
TileSplit gemm_nn_split(const GemmProblem& p, int tile_id) {
  if (!gemm_nn_direct_to_lds(p, tile_id)) return {1, 0};
  const int bm = tile_bm(tile_id), bn = tile_bn(tile_id);
  const int64_t tiles = (int64_t)((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
  // A round counts one workgroup per CU for every tile (counting the 128x128 tile's two per CU
  // measured 3072^3 -5.5%, 1536^2 x 12288 -5%, 2304^2 x 8192 -2%).
  const int64_t slots = 256;
  const int64_t last = tiles - (tiles - 1) / slots * slots;  // tiles in the last round (1 .. slots)
  if (last * 2 >= slots) return {1, 0};
  const int kt = (p.K + 63) / 64;  // 64-deep K tiles (the 32-deep tiles have twice as many)
  int64_t splits = slots / last;
  if (splits > kt / 8) splits = kt / 8;
  if (splits > 16) splits = 16;
  const int64_t cap = (int64_t)(kMaxWorkspaceBytes / ((size_t)bm * bn * 4)) / last;
  if (splits > cap) splits = cap;
  if (splits < 2) return {1, 0};
  // one tile's round at 4.8 TFLOP/s per CU (the 256x256 tile at 8192^3; smaller tiles run
  // slower, so this underestimates the saving); reduction traffic at kSplitTrafficBps plus 3 us
  const double round = 2.0 * bm * bn * (kt * 64.0) / 4.8e12;
  const double saved = round * (1.0 - 1.0 / (double)splits);
  const double cost = (double)last * bm * bn * 4.0 * (2.0 * splits + 1.0) / kSplitTrafficBps + 3e-6;
  // split only with a clear margin: near break-even the estimate's error decides (measured on
  // MI355X: 6144^2 x 1024 split in two -2%, 6150 x 6144 x 2048 +2.4%)
  if (saved <= 1.5 * cost) return {1, 0};
  return {(int)splits, (int)last};
}

int gemm_nn_splits(const GemmProblem& p, int tile_id) { return gemm_nn_split(p, tile_id).splits; }

size_t gemm_nn_workspace_bytes(const GemmProblem& p, int tile_id) {
  const TileSplit sp = gemm_nn_split(p, tile_id);
  if (sp.splits < 2) return 0;
  const size_t bm = tile_bm(tile_id), bn = tile_bn(tile_id);
  return (size_t)sp.tiles * sp.splits * bm * bn * 4;
}

// The persistent kernel's conditions: whole interior tiles (256x256, or 192x192 without a K
// split) over more than one round of 256 workgroups, aligned operands (no masked last K tile),
// 4-byte-aligned C, and at least S + 1 K tiles.  Measured against one workgroup per tile (same
// box): 8192^3 +1%, 8192^2 x 2048 +3.7%, 16384 x 8192 x 1024 +3.8%; 192x192 at 6144^2 x 2048 +4%.
template <class TP = DmaTile<256, 256>>
static bool persistent_ok(const GemmProblem& p) {
  if (!dma_ok(p, TP::BM) || p.tail_regs || !p.c_vec4) return false;
  if (p.M % TP::BM || p.N % TP::BN) return false;
  if ((int64_t)(p.M / TP::BM) * (p.N / TP::BN) <= 256) return false;
  return (p.K + TP::BK - 1) / TP::BK >= TP::STAGES + 1;
}

// Workgroups of a non-persistent tile launch (whole tiles plus the split tiles' K ranges).
static int64_t launch_blocks(const GemmProblem& p, int bm, int bn) {
  const int64_t tiles = (int64_t)((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
  return p.k_splits > 1 ? tiles - p.split_tiles + (int64_t)p.split_tiles * p.k_splits : tiles;
}

// ------------------------------------------------------------------------------------
// Operand-path probe (measurement only; entry point mmm_probe_lds_mfma).  The persistent 256x256
// kernel's K loop on operands that are already in LDS: each workgroup stages K tiles 0 and 1 of
// its first output tile into the two ring slots once (the kernels' staging map), then runs the
// kernel's own per-K-tile code -- ktile_body and ktile_last_step: the same MFMAs and fragment
// reads, at the same LDS addresses, in the same order -- over as many K tiles as its share of the
// M x N x K problem holds, alternating the slots as the ring does.  Left out: the refill loads (the
// last step's load hook is empty), their waits and the C stores.  With BARRIER the workgroup
// barrier stays where the kernel publishes the next K tile; without it the waves run
// unsynchronised (nothing writes the LDS after the staging, so nothing races).  Each thread
// writes the sum of its accumulators at the end.  A workgroup's accumulators see slot 0 (K 0..63
// of its first tile) and slot 1 (K 64..127) total/2 = tiles * K / 128 times each, so the sum of
// its threads' outputs is (total / 2) * (1^T A0)(B0 1), A0 = A[m0 .. m0+255][0 .. 127],
// B0 = B[0 .. 127][n0 .. n0+255] (exact for small integer inputs).
// ------------------------------------------------------------------------------------
template <class T, bool BARRIER>
__global__ __launch_bounds__(T::NT, T::OCC) void lds_mfma_probe_kernel(GemmProblem p, int tiles_m, int tiles_n,
                                                                       float* out) {
  __shared__ __attribute__((aligned(1024))) char lds[T::STAGES * T::STAGE];
  static_assert(T::STAGES == 2 && T::B_UNIFORM, "two ring slots, the uniform staging map");
  record_clock(p.clk, 0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / T::WGN, wn = w % T::WGN;
  const int K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  char LDS_AS* lds_base = (char LDS_AS*)lds;

  // staging of K tiles 0 and 1 of the first output tile, as the kernels stage them (thread
  // (w, lane) moves chunk slot r * NT + w * 64 + lane of each operand's rounds r)
  constexpr int RPA = T::NT / T::CA, RPB = T::NT / T::CB;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, 4, &tm, &tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * T::BM), n0 = __builtin_amdgcn_readfirstlane(tn * T::BN);
  {
    const int a_row0 = w * (64 / T::CA) + lane / T::CA;
    const int a_kc = 8 * ((lane % T::CA) ^ T::swz_a(a_row0));
    const int b_row0 = w * (64 / T::CB) + lane / T::CB;
    const int b_nc = 8 * ((lane % T::CB) ^ T::swz_bk(b_row0));
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const i32x4 ra = make_rsrc(p.A + (int64_t)m0 * lda + s * T::BK,
                                 clip_records(((int64_t)(p.M - 1 - m0) * lda + K - s * T::BK) * 2));
      const i32x4 rb = make_rsrc(p.B + (int64_t)s * T::BK * ldb + n0,
                                 clip_records(((int64_t)(K - 1 - s * T::BK) * ldb + p.N - n0) * 2));
      const uint32_t a_dst = lds_addr_of(lds_base) + s * T::STAGE + w * 64 * 16, b_dst = a_dst + T::A_BYTES;
#pragma unroll
      for (int r = 0; r < T::RA; ++r)
        dma_b128(a_dst + r * T::NT * 16, ra, (uint32_t)(((a_row0 + r * RPA) * lda + a_kc) * 2));
#pragma unroll
      for (int r = 0; r < T::RB; ++r)
        dma_b128(b_dst + r * T::NT * 16, rb, (uint32_t)(((b_row0 + r * RPB) * ldb + b_nc) * 2));
    }
    wait_vmcnt<0>();
  }
  block_sync();

  // fragment read offsets (as gemm_nn_kernel)
  uint32_t a_off[kMaxOff] = {};
#pragma unroll
  for (int kk = 0; kk < T::KSTEPS; ++kk)
#pragma unroll
    for (int ph = 0; ph < T::APAR; ++ph) {
      const int m = wm * T::TM + ph * T::MF + (lane % T::MF);
      const int chunk = (T::KK / 8) * kk + lane / T::MF;
      a_off[kk * T::APAR + ph] = m * T::BK * 2 + (chunk ^ T::swz_a(m)) * 16;
    }
  uint32_t b_off[kMaxOff] = {};
  {
    const int k = 8 * (lane / T::MF) + ((lane >> 2) & 3);
#pragma unroll
    for (int nb = 0; nb < T::FN; ++nb) {
      const int n = wn * T::TN + 16 * nb + 4 * (lane & 3);
      b_off[nb] = k * T::BN * 2 + (((n >> 3) ^ T::swz_bk(k)) * 16) + (n & 7) * 2;
    }
  }
  static_assert(T::MF == 16, "the 16x16x32 tile's fragment map");

  // this workgroup's K tiles: its output tiles b, b + grid, ... times K / BK each
  const int mine = (tiles_m * tiles_n - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int total = __builtin_amdgcn_readfirstlane(mine * (K / T::BK));
  AccT<T> acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = AccT<T>{};
  Frags<T> f[2];
  load_frags<T, false>(lds_base, lds_base + T::A_BYTES, a_off, b_off, 0, f[0]);
  int cur = 0;
  for (int t = 0; t < total; ++t) {
    ktile_body<T, false>(lds_base + cur * T::STAGE, a_off, b_off, f, acc);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (BARRIER) block_sync();
    cur ^= 1;
    ktile_last_step<T, false>(lds_base + cur * T::STAGE, a_off, b_off, f, acc, 0, [](int, int) {});
  }
  float keep = 0.0f;
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) keep += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  out[(int64_t)blockIdx.x * T::NT + tid] = keep;
  record_clock(p.clk, 2);
}

hipError_t launch_lds_mfma_probe(const GemmProblem& p, bool barrier, float* out, hipStream_t stream) {
  using T = Tile256;
  const int tiles_m = p.M / T::BM, tiles_n = p.N / T::BN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int grid = (int)(tiles < 256 ? tiles : 256);
  if (barrier)
    hipLaunchKernelGGL((lds_mfma_probe_kernel<T, true>), dim3(grid), dim3(T::NT), 0, stream, p, tiles_m, tiles_n, out);
  else
    hipLaunchKernelGGL((lds_mfma_probe_kernel<T, false>), dim3(grid), dim3(T::NT), 0, stream, p, tiles_m, tiles_n, out);
  return hipGetLastError();
}

bool gemm_nn_persistent(const GemmProblem& p0, int tile_id) {
  if (tile_id != kTile256x256 && tile_id != kTile192x192) return false;
  GemmProblem p = p0;
  p.c_vec4 = (uintptr_t)p.C % 4 == 0;
  p.tail_regs = !tail_aligned(p);
  p.k_splits = gemm_nn_split(p, tile_id).splits;
  if (tile_id == kTile192x192) return p.k_splits <= 1 && persistent_ok<DmaTile<192, 192>>(p);
  return persistent_ok(p);
}

hipError_t launch_gemm_nn(const GemmProblem& p0, int tile_id, hipStream_t stream) {
  GemmProblem p = p0;
  // 16-byte stores of C need only 4-byte alignment on gfx950 (rows of an odd ldc included)
  p.c_vec4 = (uintptr_t)p.C % 4 == 0;
  p.tail_regs = !tail_aligned(p);
  p.k_splits = 1;
  p.split_tiles = 0;
  p.partials = nullptr;
  const TileSplit sp = gemm_nn_split(p, tile_id);
  if (sp.splits > 1 && p.ws && p.ws_bytes >= gemm_nn_workspace_bytes(p, tile_id))
    p.k_splits = sp.splits, p.split_tiles = sp.tiles, p.partials = p.ws;  // else unsplit
  switch (tile_id) {
    case kTile256x256:
      if (persistent_ok(p)) {
        using TP = DmaTile<256, 256>;
        // Non-temporal C stores: the persistent grid stores a tile's C while its next tile's
        // operand loads run, and L2-allocating stores would evict the operand panels other
        // workgroups of the XCD are about to read.  As half-line stores that won only when each
        // tile's K loop is long (measured on MI355X: 12288^2 x 4096 +6.7%, 8192^3 +1.6-2.8%,
        // 8192^2 x 2048 -7.1%, 16384 x 8192 x 1024 -9.3%); as whole lines (store_wave_tile_lines)
        // they win at every K (against L2-allocating half lines: 8192^2 x 2048 +8%, 12288^2 x
        // 2048 +5.2%, 8192^2 x 1024 +4.2-4.8%, 16384 x 8192 x 1024 +4.2%).  16-byte-aligned C
        // rows only.
        const int tiles_m = p.M / TP::BM, tiles_n = p.N / TP::BN;
        const bool nt = ((uintptr_t)p.C & 15) == 0 && p.ldc % 4 == 0 &&
                        (c_lines_all<TP>() || p.K >= kNtMinK);
        if (p.k_splits <= 1) {
          if (nt)
            hipLaunchKernelGGL((gemm_nn_persistent_kernel<TP, true>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                               tiles_n);
          else
            hipLaunchKernelGGL((gemm_nn_persistent_kernel<TP, false>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                               tiles_n);
          return hipGetLastError();
        }
        if (nt)
          hipLaunchKernelGGL((gemm_nn_persistent_split_kernel<TP, true>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                             tiles_n);
        else
          hipLaunchKernelGGL((gemm_nn_persistent_split_kernel<TP, false>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                             tiles_n);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // the last round's K-split pieces ran as the grid's final items: sum their partials
        const int64_t tiles = (int64_t)tiles_m * tiles_n;
        constexpr int64_t per_tile = TP::BM * TP::BN / 4 / 256;  // blocks of 256 float4s per tile
        hipLaunchKernelGGL((reduce_tiles_kernel<TP::BM, TP::BN>), dim3((unsigned)(p.split_tiles * per_tile)), dim3(256),
                           0, stream, p, tiles_m, tiles_n, (int)(tiles - p.split_tiles), p.k_splits);
        return hipGetLastError();
      }
      return dma_ok(p, 256) ? launch_nn<DmaTile<256, 256>, false>(p, stream)
                            : launch_nn<RegTile<256, 256>, true>(p, stream);
    case kTile128x256:
      return dma_ok(p, 128) ? launch_nn<DmaTile<128, 256>, false>(p, stream)
                            : launch_nn<RegTile<128, 256>, true>(p, stream);
    case kTile256x128:
      return dma_ok(p, 256) ? launch_nn<DmaTile<256, 128>, false>(p, stream)
                            : launch_nn<RegTile<256, 128>, true>(p, stream);
    case kTile128x128:
      if (!dma_ok(p, 128)) return launch_nn<RegTile<128, 128>, true>(p, stream);
      return launch_blocks(p, 128, 128) <= 256 ? launch_nn<DeepTile128, false>(p, stream)
                                                : launch_nn<DmaTile<128, 128>, false>(p, stream);
    case kTile64x64:
      return dma_ok(p, 64) ? launch_nn<DmaTile<64, 64>, false>(p, stream) : launch_nn<RegTile<64, 64>, true>(p, stream);
    case kTile192x192:
      if (p.k_splits <= 1 && persistent_ok<DmaTile<192, 192>>(p)) {
        using TP = DmaTile<192, 192>;
        const int tiles_m = p.M / TP::BM, tiles_n = p.N / TP::BN;
        // non-temporal C as for the 256x256 tile; this tile's third block of a row is stored as
        // half lines, and at short K its non-temporal stores lose (6144^2 x 2048 -2.9%,
        // 3072 x 6144 x 2048 -3.7% with them at every K; long K: 6144^3 +1.2%)
        const bool nt = ((uintptr_t)p.C & 15) == 0 && p.ldc % 4 == 0 &&
                        (c_lines_all<TP>() || p.K >= kNtMinK);
        if (nt)
          hipLaunchKernelGGL((gemm_nn_persistent_kernel<TP, true>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                             tiles_n);
        else
          hipLaunchKernelGGL((gemm_nn_persistent_kernel<TP, false>), dim3(256), dim3(TP::NT), 0, stream, p, tiles_m,
                             tiles_n);
        return hipGetLastError();
      }
      // the register-staged path has no 192x192 instantiation: 128x128 tiles compute the same C
      return dma_ok(p, 192) ? launch_nn<DmaTile<192, 192>, false>(p, stream)
                            : launch_nn<RegTile<128, 128>, true>(p, stream);
    default:
      return hipErrorInvalidValue;
  }
}

// Largest element offset (+1) an operand's fold can address, or -1 if a stride is negative.
static int64_t fold_extent(int64_t e_hi, int64_t e_lo, int64_t s_hi, int64_t s_lo, int64_t f_hi, int64_t f_lo,
                           int64_t t_hi, int64_t t_lo) {
  if (s_hi < 0 || s_lo < 0 || t_hi < 0 || t_lo < 0) return -1;
  return (e_hi - 1) * s_hi + (e_lo - 1) * s_lo + (f_hi - 1) * t_hi + (f_lo - 1) * t_lo + 1;
}

template <bool NT, bool WIDE>
static void launch_fold_dma(const FoldProblem& p, bool lanek, int tiles_m, int tiles_n, uint32_t a_bytes,
                            uint32_t b_bytes, hipStream_t stream) {
  using TD = FoldDmaTile;
  const dim3 grid((unsigned)((int64_t)tiles_m * tiles_n)), block(TD::NT);
  if (lanek)
    hipLaunchKernelGGL((gemm_fold_dma_kernel<TD, NT, WIDE, true>), grid, block, 0, stream, p, tiles_m, tiles_n, a_bytes,
                       b_bytes);
  else
    hipLaunchKernelGGL((gemm_fold_dma_kernel<TD, NT, WIDE, false>), grid, block, 0, stream, p, tiles_m, tiles_n, a_bytes,
                       b_bytes);
}

hipError_t launch_gemm_fold(const FoldProblem& p, hipStream_t stream) {
  // direct-to-LDS fold path: K contiguous in both operands, 16-byte-aligned chunks; K tiles
  // inside one k_hi block (k_lo % 64 == 0) or, per lane, crossing blocks (k_lo % 8 == 0);
  // buffer loads when the offsets fit 32 bits, else 64-bit addresses (K % 64 == 0: no range
  // check masks a K tail there)
  using TD = FoldDmaTile;
  const int m_hi = (p.M + p.m_lo - 1) / p.m_lo, n_hi = (p.N + p.n_lo - 1) / p.n_lo, k_hi = p.K / p.k_lo;
  const int64_t a_ext = fold_extent(m_hi, p.m_lo, p.am[0], p.am[1], k_hi, p.k_lo, p.ak[0], p.ak[1]);
  const int64_t b_ext = fold_extent(n_hi, p.n_lo, p.bn[0], p.bn[1], k_hi, p.k_lo, p.bk[0], p.bk[1]);
  const bool lanek = p.k_lo % TD::BK != 0;
  const bool wide = a_ext * 2 >= (int64_t)kOobOffset / 2 || b_ext * 2 >= (int64_t)kOobOffset / 2;
  const bool fast = TD::BK == 64 && p.ak[1] == 1 && p.bk[1] == 1 && p.k_lo % 8 == 0 && p.K % p.k_lo == 0 &&
                    (p.K % TD::BK == 0 || !wide) &&
                    p.am[0] % 8 == 0 && p.am[1] % 8 == 0 && p.bn[0] % 8 == 0 && p.bn[1] % 8 == 0 &&
                    p.ak[0] % 8 == 0 && p.bk[0] % 8 == 0 && ((uintptr_t)p.A & 15) == 0 && ((uintptr_t)p.B & 15) == 0 &&
                    a_ext > 0 && b_ext > 0 && p.M % p.m_lo == 0 && p.N % p.n_lo == 0;
  if (fast) {
    const int tiles_m = (p.M + TD::BM - 1) / TD::BM;
    const int tiles_n = (p.N + TD::BN - 1) / TD::BN;
    // Non-temporal C stores when the grid has more than one round and K is long: later tiles'
    // operand loads then run while earlier tiles' C is written, and L2-allocating stores would
    // evict operand panels (measured on MI355X at the reference's M = N = K = 8192: +13-15%).  A
    // one-round grid writes all of C after its last K step, where L2-allocating stores drain
    // faster (plain-GEMM tiles: 4096^3 -5.5%, 8192 x 2048 x 2048 -6.7% with non-temporal stores).
    const int64_t blocks = (int64_t)tiles_m * tiles_n;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const bool nt = blocks > 256 && p.K >= kNtMinK;
    const uint32_t ab = wide ? 0u : (uint32_t)(a_ext * 2), bb = wide ? 0u : (uint32_t)(b_ext * 2);
    if (wide && nt)
      launch_fold_dma<true, true>(p, lanek, tiles_m, tiles_n, ab, bb, stream);
    else if (wide)
      launch_fold_dma<false, true>(p, lanek, tiles_m, tiles_n, ab, bb, stream);
    else if (nt)
      launch_fold_dma<true, false>(p, lanek, tiles_m, tiles_n, ab, bb, stream);
    else
      launch_fold_dma<false, false>(p, lanek, tiles_m, tiles_n, ab, bb, stream);
    return hipGetLastError();
  }
  using T = RegTile<128, 128>;
  const int tiles_m = (p.M + T::BM - 1) / T::BM;
  const int tiles_n = (p.N + T::BN - 1) / T::BN;
  const int64_t blocks = (int64_t)tiles_m * tiles_n;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const bool bkm = (p.bk[1] == 1) || (p.k_lo == 1 && p.bk[0] == 1);
  if (bkm)
    hipLaunchKernelGGL((gemm_fold_kernel<T, true>), dim3((unsigned)blocks), dim3(T::NT), 0, stream, p, tiles_m, tiles_n);
  else
    hipLaunchKernelGGL((gemm_fold_kernel<T, false>), dim3((unsigned)blocks), dim3(T::NT), 0, stream, p, tiles_m, tiles_n);
  return hipGetLastError();
}

}  // namespace mmm
