// Streaming GEMM for M <= 64 (decode-shaped, e.g. 16 x 8192 x 8192): HBM-bound, so the design
// goal is to stream B once at full bandwidth with the MFMA work hidden underneath.  Two kernels:
//
//  * gemm_stream_wide_kernel<MR, NS> (MR = 1, 2, 4 groups of 16 rows): one workgroup per
//    NS-column strip (128; 256 for long K streams) and K range; every wave streams the
//    strip's full 256- or 512-byte rows of B over its quarter of the range; K partials summed
//    through LDS, K ranges across workgroups summed by reduce_splits_kernel in a fixed order.
//  * gemm_skinny_kernel (M <= 16 without a caller workspace): one workgroup per
//    32-column strip, XCD-contiguous; the four waves split K; partials summed through LDS.
//
// Common to both: each wave streams through its own LDS ring with direct-to-LDS buffer loads
// and only reads what it loaded itself, so the loop has no workgroup barrier (a wave waits on
// its own vmcnt only).  A slot holds a KS-deep K step: A [16][KS] (rows swizzled so 16 rows
// at one chunk hit 16 bank groups) and B [KS][NS] (N contiguous).  Math:
// v_mfma_f32_16x16x32_f16, A fragment by ds_read_b128, B fragment by two ds_read_b64_tr_b16
// (transposing 4x16 blocks into the K-contiguous operand layout).  All sums run in fixed
// orders, so results are deterministic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mmm.h"
#include "mmm_dma.h"
#include "mmm_kernels.h"
#include "mmm_tile_map.h"

namespace mmm {

namespace {

constexpr int kNS = 32;     // columns per workgroup
constexpr int kKS = 64;     // K rows per ring slot
constexpr int kSlots = 6;   // ring slots per wave
constexpr int kWaves = 4;
constexpr int kABytes = 16 * kKS * 2;   // A [16][KS]
constexpr int kBBytes = kKS * kNS * 2;  // B [KS][NS]
constexpr int kSlot = kABytes + kBBytes;
constexpr int kLoadsPerSlot = kABytes / 1024 + kBBytes / 1024;  // 1 KB per wave-wide DMA
constexpr int kNT = kNS / 16;           // 16-column MFMA tiles per strip
constexpr int kCPR = kNS / 8;           // 16-byte chunks per B row
static_assert(kKS == 32 || kKS == 64, "K rows per slot");
static_assert(kNS == 32 || kNS == 64, "strip width");
static_assert(kWaves * kSlots * kSlot <= 160 * 1024, "rings must fit the LDS");

// A-slot swizzle: 16 rows at one logical chunk land in 16 distinct 16-byte bank groups.
// Rows of 128 B (KS = 64): chunk ^ ((row >> 1) & 7).  Rows of 64 B (KS = 32): four rows
// share a 256-byte window, so chunk ^ ((row >> 2) & 3).
__device__ __forceinline__ int swz_a(int row) { return kKS == 64 ? ((row >> 1) & 7) : ((row >> 2) & 3); }

}  // namespace

// Streams K steps [s_begin, s_end) of the 32-column strip at n0 through this wave's private
// LDS ring and accumulates the 16 x 32 product into acc (16x16 tiles j, lane (fr, fg) holding
// rows 4*fg .. 4*fg+3 of column 16*j + fr).  No barrier: the wave waits on its own loads only.
__device__ __forceinline__ void stream_columns(const GemmProblem& p, int n0, int s_begin, int s_end, int nst_all,
                                               char LDS_AS* ring, int lane, f32x4 (&acc)[kNT]) {
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int nst = s_end - s_begin;
  const uint32_t ring_addr = (uint32_t)(uintptr_t)ring;

  // DMA map.  A [16][KS]: CA = KS/8 chunks per row; one wave-wide instruction covers
  // 64/CA rows, lane -> row lane/CA (+ 64/CA per instruction), slot chunk lane%CA holding
  // logical chunk (lane%CA) ^ swz(row).  B [KS][NS]: lane -> row lane/CPR (+ 64/CPR per
  // instruction), slot chunk lane%CPR holding logical chunk (lane%CPR) ^ 2*((row >> 3) & 1):
  // a pass of a 16x16x32 transposing read takes rows k .. k+3 and k+8 .. k+11, and with
  // 64-byte rows, rows 8 apart sit on the same banks unless their chunk pairs are swapped.
  constexpr int CA = kKS / 8, RPI_A = 64 / CA, NA = kABytes / 1024;
  const int a_row = lane / CA;
  uint32_t a_goff[NA];
  int a_kc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int row = a_row + i * RPI_A;
    a_kc[i] = 8 * ((lane % CA) ^ swz_a(row));
    a_goff[i] = (uint32_t)((row * lda + a_kc[i]) * 2);
  }
  static_assert(kCPR == 4 && (64 / kCPR) % 16 == 0, "the B swizzle's row bit 3 is fixed per lane across loads");
  const int b_sw = 2 * (((lane / kCPR) >> 3) & 1);  // rows of load i: lane/CPR + 16i, same bit 3
  const uint32_t b_goff = (uint32_t)(((lane / kCPR) * ldb + 8 * ((lane % kCPR) ^ b_sw)) * 2);
  const uint32_t b_rstep = (uint32_t)((64 / kCPR) * ldb * 2);
  const i32x4 rb_full = make_rsrc(p.B + n0, clip_records(((int64_t)(K - 1) * ldb + N - n0) * 2));

  auto issue = [&](int s, int slot) {
    const int k0 = (s_begin + s) * kKS;
    const i32x4 ra = make_rsrc(p.A + k0, clip_records(((int64_t)(M - 1) * lda + K - k0) * 2));
    const uint32_t dst = ring_addr + slot * kSlot;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      // K tail: chunks at or past K are pushed out of the descriptor's range (read as zero)
      const uint32_t dead = (uint32_t)(K - 1 - (k0 + a_kc[i])) >> 31;
      dma_b128(dst + i * 1024, ra, a_goff[i] + dead * kOobOffset);
    }
    const uint32_t bk = (uint32_t)((int64_t)k0 * ldb * 2);
#pragma unroll
    for (int i = 0; i < kBBytes / 1024; ++i) dma_b128(dst + kABytes + i * 1024, rb_full, bk + b_goff + i * b_rstep);
  };

  // The globally last K slot of an unaligned problem (K or N not a multiple of 8, or rows
  // not 16-byte aligned) is gathered element by element through VGPRs into the same layout:
  // its chunks may straddle K, N or the end of an operand.  Every earlier slot lies wholly
  // inside both operands.  The ring is private to the wave, so LDS ordering within the wave
  // is all the gathered slot needs.
  const _Float16* Ah = (const _Float16*)p.A;
  const _Float16* Bh = (const _Float16*)p.B;
  // Every element is loaded from an address clamped into its operand and masked afterwards, all
  // loads before any store: a load under a lane condition would be merged into its vector before
  // the next one issued, one memory round trip per element.
  auto gather = [&](int s, int slot) {
    const int k0 = (s_begin + s) * kKS;
    char LDS_AS* dst = ring + slot * kSlot + lane * 16;
    constexpr int NB = kBBytes / 1024;
    _Float16 xa[NA][8], xb[NB][8];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int row = a_row + i * RPI_A, k = k0 + a_kc[i];
      const _Float16* src = Ah + (int64_t)(row < M ? row : M - 1) * lda;
#pragma unroll
      for (int e = 0; e < 8; ++e) xa[i][e] = src[k + e < K ? k + e : K - 1];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int k = k0 + i * (64 / kCPR) + lane / kCPR, n = n0 + 8 * ((lane % kCPR) ^ b_sw);
      const _Float16* src = Bh + (int64_t)(k < K ? k : K - 1) * ldb;
#pragma unroll
      for (int e = 0; e < 8; ++e) xb[i][e] = src[n + e < N ? n + e : N - 1];
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int row = a_row + i * RPI_A, k = k0 + a_kc[i];
      half8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (row < M && k + e < K) ? xa[i][e] : (_Float16)0;
      *(half8 LDS_AS*)(dst + i * 1024) = v;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int k = k0 + i * (64 / kCPR) + lane / kCPR, n = n0 + 8 * ((lane % kCPR) ^ b_sw);
      half8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (k < K && n + e < N) ? xb[i][e] : (_Float16)0;
      *(half8 LDS_AS*)(dst + kABytes + i * 1024) = v;
    }
  };
  const bool gather_last = p.tail_regs && s_end == nst_all && nst > 0;  // uniform
  auto fill = [&](int s, int slot) {
    if (gather_last && s == nst - 1)
      gather(s, slot);
    else
      issue(s, slot);
  };

  // fragment offsets within a slot
  const int fr = lane & 15, fg = lane >> 4;
  constexpr int KQ = kKS / 32;  // 32-deep MFMA steps per slot
  uint32_t a_off[KQ];
#pragma unroll
  for (int q = 0; q < KQ; ++q) a_off[q] = fr * (kKS * 2) + (((4 * q + fg) ^ swz_a(fr)) * 16);
  // B rows 8fg + (fr >> 2) (+4, +32q): row bit 3 = fg & 1, which swaps the two 16-column tiles'
  // chunk pairs
  const uint32_t b_off = kABytes + (8 * fg + (fr >> 2)) * (kNS * 2) + 4 * (fr & 3) * 2;
  const int b_js = fg & 1;

  auto compute = [&](int slot) {
    const char LDS_AS* sl = ring + slot * kSlot;
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
      const half8 af = *(const half8 LDS_AS*)(sl + a_off[q]);
#pragma unroll
      for (int j = 0; j < kNT; ++j) {
        const char LDS_AS* bp = sl + b_off + (32 * q) * (kNS * 2) + 16 * (j ^ b_js) * 2;
        fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)bp);
        fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)(bp + 4 * kNS * 2));
        const half8 bf = __builtin_shufflevector(__builtin_bit_cast(half4, lo), __builtin_bit_cast(half4, hi), 0, 1,
                                                 2, 3, 4, 5, 6, 7);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[j], 0, 0, 0);
      }
    }
  };

  constexpr int P = kSlots - 1;
  for (int s = 0; s < P; ++s)
    if (s < nst) fill(s, s);
  int cur = 0, nxt = P;
  int t = 0;
  for (; t + P < nst - 1; ++t) {            // refills a slot that is not the last
    wait_vmcnt<(P - 1) * kLoadsPerSlot>();  // step t landed (this wave's own loads)
    wait_lgkm0();                           // this wave's reads of slot nxt (step t-1) are done
    issue(t + P, nxt);
    compute(cur);
    cur = cur + 1 == kSlots ? 0 : cur + 1;
    nxt = nxt + 1 == kSlots ? 0 : nxt + 1;
  }
  if (t + P == nst - 1) {  // refills the last slot (possibly gathered)
    wait_vmcnt<(P - 1) * kLoadsPerSlot>();
    wait_lgkm0();
    fill(t + P, nxt);
    compute(cur);
    cur = cur + 1 == kSlots ? 0 : cur + 1;
    ++t;
  }
  for (; t < nst; ++t) {  // a gathered last slot leaves nothing outstanding: drain everything
    wait_vmcnt<0>();
    compute(cur);
    cur = cur + 1 == kSlots ? 0 : cur + 1;
  }
}

__global__ __launch_bounds__(256, 1) void gemm_skinny_kernel(GemmProblem p, int strips) {
  __shared__ __attribute__((aligned(1024))) char lds[kWaves * kSlots * kSlot];
  const int strip = __builtin_amdgcn_readfirstlane(xcd_compact(blockIdx.x, strips));
  const int n0 = strip * kNS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = p.M, N = p.N, K = p.K;

  // this wave's K steps (the four waves split K; their partials are summed through LDS)
  const int nst_all = (K + kKS - 1) / kKS;
  const int s_begin = __builtin_amdgcn_readfirstlane((w * nst_all) / kWaves);
  const int s_end = __builtin_amdgcn_readfirstlane(((w + 1) * nst_all) / kWaves);
  f32x4 acc[kNT];
#pragma unroll
  for (int j = 0; j < kNT; ++j) acc[j] = f32x4{};
  stream_columns(p, n0, s_begin, s_end, nst_all, (char LDS_AS*)lds + w * kSlots * kSlot, lane, acc);
  const int fr = lane & 15, fg = lane >> 4;

  // K-partials -> LDS (after every wave is done with its ring), fixed-order sum, store.
  __syncthreads();
  float LDS_AS* part = (float LDS_AS*)lds;  // [wave][16][NS]
#pragma unroll
  for (int j = 0; j < kNT; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(w * 16 + 4 * fg + v) * kNS + 16 * j + fr] = acc[j][v];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 16 * kNS / 256; ++e) {
    const int idx = tid + 256 * e;  // -> (row, col)
    const int row = idx / kNS, col = idx % kNS;
    const float sum = ((part[(0 * 16 + row) * kNS + col] + part[(1 * 16 + row) * kNS + col]) +
                       part[(2 * 16 + row) * kNS + col]) +
                      part[(3 * 16 + row) * kNS + col];
    if (row < M && n0 + col < N) p.C[(int64_t)row * p.ldc + n0 + col] = sum;
  }
}

// C[row][strip * NS + c] = sum over q = 0 .. splits-1 (in that order) of the strip's
// partials; one thread per 4 consecutive elements of the ROWS x NS strip tiles.  All of a
// thread's split loads are issued before the sum (splits <= kMaxSplits), so the kernel costs
// one memory round trip.
constexpr int kMaxSplits = 16;
template <int ROWS, int NS>
__global__ __launch_bounds__(256) void reduce_splits_kernel(GemmProblem p, int strips, int splits,
                                                            const float* partials) {
  constexpr int TILE = ROWS * NS;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int strip = idx / (TILE / 4), e = 4 * (idx % (TILE / 4)), row = e / NS, col = strip * NS + e % NS;
  if (strip >= strips) return;
  const f32x4* base = (const f32x4*)(partials + (int64_t)strip * splits * TILE + e);
  f32x4 v[kMaxSplits];
#pragma unroll
  for (int q = 0; q < kMaxSplits; ++q)
    if (q < splits) v[q] = base[q * (TILE / 4)];
  f32x4 sum = v[0];
#pragma unroll
  for (int q = 1; q < kMaxSplits; ++q)
    if (q < splits) sum += v[q];
  if (row >= p.M) return;
  float* c = p.C + (int64_t)row * p.ldc + col;
  if (p.c_vec4 && col + 3 < p.N) {
    *(f32x4*)c = sum;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (col + i < p.N) c[i] = sum[i];
  }
}

// ------------------------------------------------------------------------------------
// Split streaming kernel (M <= 64, enough K): one workgroup per NS-column strip and K range
// q of `splits`.  Each wave streams the whole strip -- NS * 2 contiguous bytes of every B row
// -- over its own quarter of the workgroup's K range, through a private LDS ring (no barrier in
// the loop); the four K partials are summed through LDS in wave order.  With splits == 1 the
// sum goes to C; otherwise to the workspace, and reduce_splits_kernel, launched next on the
// same stream, sums the splits of every strip in split order (fixed orders throughout:
// deterministic; the kernel boundary orders the partial stores before their reads).  B slots
// [KS][NS] have 256- or 512-byte rows -- one or two rows of the 64 banks each -- so a chunk's
// banks depend only on its slot position (mod 16 chunks).  One pass of a 16x16x32 transposing
// read takes rows k .. k+3 and k+8 .. k+11 at two chunks each; chunk c of row k sits at
// c ^ swz_b(k), swz_b(k) = {0,6,10,12}[k & 3] ^ 2 * ((k >> 3) & 1): eight distinct XOR values
// below 16, so the pass's 16 chunks hit all 64 banks once (without the k >> 3 term rows k and
// k+8 collide: measured 45% of the LDS cycles in bank conflicts).  MR 16-row groups of A
// (MR = 1, 2, 4 for up to 16, 32, 64 rows) share every B fragment: MR MFMAs per B read.
// 512-byte row pieces stream faster from HBM than 256-byte ones (16 x 8192 x 8192: 23.9 against
// 25.1 us for the streaming kernel), at twice the partial sums per workgroup.
// ------------------------------------------------------------------------------------
template <int MR, int NSW>
struct Wide {
  static constexpr int NS = NSW;  // columns per strip: 128 (256-byte rows) or 256 (512-byte rows)
  static constexpr int ROWS = 16 * MR;
  static constexpr int KS = MR == 4 || NS == 256 ? 32 : 64;  // K rows per slot
  static constexpr int SLOTS = MR == 4 && NS == 128 ? 3 : 2;  // ring slots per wave
  static constexpr int ABYTES = ROWS * KS * 2, BBYTES = KS * NS * 2, SLOT = ABYTES + BBYTES;
  static constexpr int NA = ABYTES / 1024, NB = BBYTES / 1024, LOADS = NA + NB;
  static constexpr int NT = NS / 16, CPR = NS / 8, RPI = 64 / CPR;  // tiles, chunks per row, rows per load
  // B rows of load i are RPI * i + (lane / CPR); their swz_b takes PH values, by phase(i)
  static constexpr int PH = RPI == 4 ? 2 : 4;
  __host__ __device__ static constexpr int phase(int i) { return RPI == 4 ? (i >> 1) & 1 : (i & 1) | ((i >> 2) & 1) << 1; }
  __host__ __device__ static constexpr int phase_load(int ph) { return RPI == 4 ? 2 * ph : (ph & 1) | (ph >> 1) << 2; }
  static constexpr int CA = KS / 8, RPI_A = 64 / CA;
  static constexpr int RING_BYTES = kWaves * SLOTS * SLOT;
  // [wave][ROWS][PS] fp32 partial sums; rows padded by 4 floats so the four 4-row lane groups of
  // an accumulator store (rows 4 apart) land 16 banks apart instead of on the same banks
  static constexpr int PS = NS + 4;
  // partial sums pass through the LDS in PASSES row blocks of PR rows when all of them do not fit
  static constexpr int PASSES = kWaves * ROWS * PS * 4 > 160 * 1024 ? 2 : 1, PR = ROWS / PASSES;
  static constexpr int PART_BYTES = kWaves * PR * PS * 4;
  static constexpr int LDS_BYTES = RING_BYTES > PART_BYTES ? RING_BYTES : PART_BYTES;
  static_assert(KS == 32 || KS == 64, "K rows per slot");
  static_assert(NS == 128 || NS == 256, "strip widths");
  static_assert(LDS_BYTES <= 160 * 1024, "rings and partials must fit the LDS");
  __device__ static __forceinline__ int swz_a(int row) { return KS == 64 ? ((row >> 1) & 7) : ((row >> 2) & 3); }
  __device__ static __forceinline__ int swz_b(int k) { return ((0xCA60 >> (4 * (k & 3))) & 15) ^ (((k >> 3) & 1) << 1); }
};

// NTB: B's loads are non-temporal (launch_wide: B of at least kNtStreamBytes).
template <int MR, int NSW, bool NTB>
__global__ __launch_bounds__(256, 1) void gemm_stream_wide_kernel(GemmProblem p, int strips, int splits,
                                                                  float* partials) {
  using W = Wide<MR, NSW>;
  constexpr int NS = W::NS, ROWS = W::ROWS, KS = W::KS, SLOTS = W::SLOTS, ABYTES = W::ABYTES, SLOT = W::SLOT;
  constexpr int NA = W::NA, NB = W::NB, LOADS = W::LOADS, NT = W::NT, CPR = W::CPR, RPI = W::RPI;
  constexpr int CA = W::CA, RPI_A = W::RPI_A;
  __shared__ __attribute__((aligned(1024))) char lds[W::LDS_BYTES];
  const int b = blockIdx.x;
  const int strip = b % strips, q = b / strips;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int n0 = strip * NS;
  const int nst_all = (K + KS - 1) / KS;
  // the workgroup's K slots, then this wave's quarter of them
  const int g_begin = (q * nst_all) / splits, g_end = ((q + 1) * nst_all) / splits;
  const int s_begin = __builtin_amdgcn_readfirstlane(g_begin + (w * (g_end - g_begin)) / kWaves);
  const int s_end = __builtin_amdgcn_readfirstlane(g_begin + ((w + 1) * (g_end - g_begin)) / kWaves);
  const int nst = s_end - s_begin;
  char LDS_AS* ring = (char LDS_AS*)lds + w * SLOTS * SLOT;
  const uint32_t ring_addr = (uint32_t)(uintptr_t)ring;

  // DMA map.  A [ROWS][KS]: lane -> row lane/CA (+ RPI_A per instruction), slot chunk lane%CA
  // holding logical chunk (lane%CA) ^ swz_a(row).  B [KS][128]: lane -> row lane/CPR (+ RPI
  // per instruction), slot chunk lane%CPR holding logical chunk (lane%CPR) ^ swz_b(row).
  // Rows of A at or past M lie past the A descriptor's range (lda >= K) and read as zero.
  const int a_row = lane / CA;
  uint32_t a_goff[NA];
  int a_kc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int row = a_row + i * RPI_A;
    a_kc[i] = 8 * ((lane % CA) ^ W::swz_a(row));
    a_goff[i] = (uint32_t)((row * lda + a_kc[i]) * 2);
  }
  // B rows of load i are RPI * i + b_row, and swz_b of them depends on W::phase(i) only: chunk
  // slot c holds logical chunk c ^ swz_b(row of that phase)
  const int b_row = lane / CPR;
  int b_nc[W::PH];
  uint32_t b_goff[W::PH];
#pragma unroll
  for (int ph = 0; ph < W::PH; ++ph) {
    b_nc[ph] = 8 * ((lane % CPR) ^ W::swz_b(W::phase_load(ph) * RPI + b_row));
    b_goff[ph] = (uint32_t)((b_row * ldb + b_nc[ph]) * 2);
  }
  const uint32_t b_rstep = (uint32_t)(RPI * ldb * 2);
  const i32x4 rb_full = make_rsrc(p.B + n0, clip_records(((int64_t)(K - 1) * ldb + N - n0) * 2));

  auto issue = [&](int s, int slot) {
    const int k0 = (s_begin + s) * KS;
    const i32x4 ra = make_rsrc(p.A + k0, clip_records(((int64_t)(M - 1) * lda + K - k0) * 2));
    const uint32_t dst = ring_addr + slot * SLOT;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const uint32_t dead = (uint32_t)(K - 1 - (k0 + a_kc[i])) >> 31;
      dma_b128(dst + i * 1024, ra, a_goff[i] + dead * kOobOffset);
    }
    const uint32_t bk = (uint32_t)((int64_t)k0 * ldb * 2);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const uint32_t voff = bk + b_goff[W::phase(i)] + i * b_rstep;
      if constexpr (NTB)
        dma_b128_nt(dst + ABYTES + i * 1024, rb_full, voff);
      else
        dma_b128(dst + ABYTES + i * 1024, rb_full, voff);
    }
  };
  // globally last K slot of an unaligned problem: gathered element by element (same layout)
  const _Float16* Ah = (const _Float16*)p.A;
  const _Float16* Bh = (const _Float16*)p.B;
  // No load sits under a lane condition (that would cost a memory round trip per element).
  // Elements past the operands load from kZeroHalves, and every load is issued before the first
  // store, so the compiler keeps as many in flight as the registers allow.  The 4 x 16-row
  // instantiations clamp their addresses into the operands instead, mask the values, and store
  // each chunk after its own eight loads: the 256-column one, already at 512 registers, spilled
  // with the other form, and the 128-column one's K loop then copied its accumulators between
  // AGPRs and VGPRs (144 copies per iteration against 20).
  auto gather = [&](int s, int slot) {
    const int k0 = (s_begin + s) * KS;
    char LDS_AS* dst = ring + slot * SLOT + lane * 16;
    if constexpr (MR == 4) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int row = a_row + i * RPI_A, k = k0 + a_kc[i];
        const _Float16* src = Ah + (int64_t)(row < M ? row : M - 1) * lda;
        _Float16 x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = src[k + e < K ? k + e : K - 1];
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (row < M && k + e < K) ? x[e] : (_Float16)0;
        *(half8 LDS_AS*)(dst + i * 1024) = v;
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int k = k0 + i * RPI + b_row, n = n0 + b_nc[W::phase(i)];
        const _Float16* src = Bh + (int64_t)(k < K ? k : K - 1) * ldb;
        _Float16 x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = src[n + e < N ? n + e : N - 1];
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (k < K && n + e < N) ? x[e] : (_Float16)0;
        *(half8 LDS_AS*)(dst + ABYTES + i * 1024) = v;
      }
    } else {
      half8 va[NA], vb[NB];
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int row = a_row + i * RPI_A, k = k0 + a_kc[i];
        const _Float16* src = Ah + (int64_t)row * lda + k;
#pragma unroll
        for (int e = 0; e < 8; ++e) va[i][e] = *(row < M && k + e < K ? src + e : kZeroHalves);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int k = k0 + i * RPI + b_row, n = n0 + b_nc[W::phase(i)];
        const _Float16* src = Bh + (int64_t)k * ldb + n;
#pragma unroll
        for (int e = 0; e < 8; ++e) vb[i][e] = *(k < K && n + e < N ? src + e : kZeroHalves);
      }
#pragma unroll
      for (int i = 0; i < NA; ++i) *(half8 LDS_AS*)(dst + i * 1024) = va[i];
#pragma unroll
      for (int i = 0; i < NB; ++i) *(half8 LDS_AS*)(dst + ABYTES + i * 1024) = vb[i];
    }
  };
  const bool gather_last = p.tail_regs && s_end == nst_all && nst > 0;
  auto fill = [&](int s, int slot) {
    if (gather_last && s == nst - 1)
      gather(s, slot);
    else
      issue(s, slot);
  };

  // fragments: A row 16*g + fr, k 8*fg..; B column 16*j + fr, k rows 8*fg + (fr>>2) (+4)
  const int fr = lane & 15, fg = lane >> 4;
  constexpr int KQ = KS / 32;
  uint32_t a_off[KQ];
#pragma unroll
  for (int qq = 0; qq < KQ; ++qq) a_off[qq] = fr * (KS * 2) + (((4 * qq + fg) ^ W::swz_a(fr)) * 16);
  const int bk_row = 8 * fg + (fr >> 2);
  const int bsw = W::swz_b(bk_row);  // same for the +4 row
  f32x4 acc[MR][NT];
#pragma unroll
  for (int g = 0; g < MR; ++g)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[g][j] = f32x4{};
  auto compute = [&](int slot) {
    const char LDS_AS* sl = ring + slot * SLOT;
#pragma unroll
    for (int qq = 0; qq < KQ; ++qq) {
      half8 af[MR];
#pragma unroll
      for (int g = 0; g < MR; ++g) af[g] = *(const half8 LDS_AS*)(sl + g * 16 * KS * 2 + a_off[qq]);
      const char LDS_AS* brow = sl + ABYTES + (32 * qq + bk_row) * (NS * 2);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int n = 16 * j + 4 * (fr & 3);
        const char LDS_AS* bp = brow + (((n >> 3) ^ bsw) * 16) + (n & 7) * 2;
        fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)bp);
        fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 LDS_AS*)(bp + 4 * NS * 2));
        const half8 bf = __builtin_shufflevector(__builtin_bit_cast(half4, lo), __builtin_bit_cast(half4, hi), 0, 1,
                                                 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int g = 0; g < MR; ++g) acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[g], bf, acc[g][j], 0, 0, 0);
      }
    }
  };

  constexpr int P = SLOTS - 1;
  for (int s = 0; s < P; ++s)
    if (s < nst) fill(s, s);
  int cur = 0, nxt = P;
  int t = 0;
  // The next slot's loads go out before the wait for the current one, so P to P + 1 slots are
  // in flight per wave, not P - 1 to P (16 x 8192 x 8192: 25.5 -> 24.8 us on 128-column strips).
  for (; t + P < nst - 1; ++t) {
    wait_lgkm0();  // the previous compute's reads of slot nxt are done
    issue(t + P, nxt);
    wait_vmcnt<P * LOADS>();  // slot cur has landed; the P slots after it may stay in flight
    compute(cur);
    cur = cur + 1 == SLOTS ? 0 : cur + 1;
    nxt = nxt + 1 == SLOTS ? 0 : nxt + 1;
  }
  if (t + P == nst - 1) {
    wait_vmcnt<(P - 1) * LOADS>();
    wait_lgkm0();
    fill(t + P, nxt);
    compute(cur);
    cur = cur + 1 == SLOTS ? 0 : cur + 1;
    ++t;
  }
  for (; t < nst; ++t) {
    wait_vmcnt<0>();
    compute(cur);
    cur = cur + 1 == SLOTS ? 0 : cur + 1;
  }

  // four K partials -> LDS, summed in wave order, to C (one split) or the workspace
  constexpr int PS = W::PS, PR = W::PR, GP = MR / W::PASSES;  // rows and 16-row groups per pass
  float LDS_AS* part = (float LDS_AS*)lds;  // [wave][PR][PS]
  float* mine = splits > 1 ? partials + (int64_t)(strip * splits + q) * (ROWS * NS) : nullptr;
#pragma unroll
  for (int h = 0; h < W::PASSES; ++h) {
    __syncthreads();  // the ring's last reads (h = 0), the previous pass's sums (h = 1)
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[(w * PR + 16 * g + 4 * fg + v) * PS + 16 * j + fr] = acc[h * GP + g][j][v];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < PR * NS / 256; ++e) {
      const int idx = tid + 256 * e, rl = idx / NS, col = idx % NS, row = h * PR + rl;
      const float sum = ((part[(0 * PR + rl) * PS + col] + part[(1 * PR + rl) * PS + col]) +
                         part[(2 * PR + rl) * PS + col]) +
                        part[(3 * PR + rl) * PS + col];
      if (mine)  // written through (sc0 sc1): the reduction reads them on other XCDs (+0.2-1.4% per call)
        asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(mine + h * PR * NS + idx), "v"(sum) : "memory");
      else if (row < M && n0 + col < N)
        p.C[(int64_t)row * p.ldc + n0 + col] = sum;
    }
  }
}

// ---- launch shape.  Split kernel: 128-column strips (256 on the long streams that
// stream_shape names) x `splits` K ranges.  Every variant
// holds one workgroup per CU (LDS), so the grid is kept to one round of 256 workgroups:
// splits = the most that fit (at most 16, at least four 64-deep K steps each).  A second,
// partly filled round costs more than the extra parallelism gains (measured: 112 strips run
// 1.2-1.4x faster at 2 splits than at 3).  A split count of 1 needs no workspace.  For
// M <= 16 with one split and fewer than 128 strips the wave-split kernel (32-column strips,
// four times the workgroups) runs instead; for 16 < M <= 64 the split kernel runs with one
// split when no workspace is to be had.
constexpr int kWsTiles = 512;  // partial tiles of up to 64 x 128 fp32 (16 MiB of workspace)
static_assert((size_t)kWsTiles * 64 * 128 * 4 <= kMaxWorkspaceBytes, "partials must fit the workspace");

struct StreamShape {
  int mr;              // 16-row groups of the split kernel (1, 2, 4)
  int ns;              // split kernel: columns per strip (128, or 256 for mr == 1)
  int strips, splits;  // split kernel: grid strips * splits; splits == 0: wave-split kernel
};

static int stream_mr(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }

static StreamShape stream_shape(const GemmProblem& p) {
  const int mr = stream_mr(p.M);
  const int strips = (p.N + 127) / 128;
  // M <= 16 on B rows that are not 16-byte aligned: the split kernel's 256-byte row pieces load
  // misaligned and its reduction is a second dependent launch.  The wave-split kernel ran
  // 1 x 4095 x 4111 in 14.6 us against 19.8 (split kernel + reduction), 2 x 4095 x 4111 in 15.0
  // against 19.8; on aligned rows the two tie at that size and the split kernel leads on larger
  // B (16 x 8192^2: 32.7 against 39.8 us).  Taken when its 32-column strips fill at least half
  // the chip and B is at most 64 MiB.
  const bool b_unaligned = ((uintptr_t)p.B & 15) || p.ldb % 8;
  if (mr == 1 && b_unaligned && (p.N + kNS - 1) / kNS >= 128 && (int64_t)p.K * p.ldb * 2 <= ((int64_t)64 << 20))
    return {mr, 128, strips, 0};
  const int nst_all = (p.K + 63) / 64;  // 64-deep K steps
  auto splits_for = [&](int ns, int nstrips) {
    int splits = 256 / nstrips;
    splits = splits < kMaxSplits ? splits : kMaxSplits;
    splits = splits < nst_all / 4 ? splits : nst_all / 4;
    if (splits > kWsTiles * 128 / ns / nstrips) splits = kWsTiles * 128 / ns / nstrips;
    return splits < 1 ? 1 : splits;
  };
  const int splits = splits_for(128, strips);
  if (splits == 1 && strips < 128 && mr == 1) return {mr, 128, strips, 0};
  // Aligned B, a workspace, and a 128-column grid already split: 256-column strips (512-byte
  // row pieces) when K >= 8192 and every wave still streams at least 256 K rows (512 for more
  // than 16 rows).  Measured per call (B rotating through HBM, 256- against 128-column
  // strips): 16 x 8192 x 8192 +2.8%, 16 x 16384 x 8192 +6.4%, 16 x 8192 x 28672 +8.7%, 1 x 8192 x
  // 8192 +4.5%; with shorter streams per wave they lose: 16 x 4096 x 8192 (128 rows per wave)
  // -4.8%, 16 x 4096 x 4096 -25%, 16 x 4096 x 14336 (224) -0.4%, 16 x 14336 x 4096 (K 4096)
  // -1.8%; from an unsplit grid (no reduction) 16 x 32768 x 4096 -4.3%, 16 x 28672 x 8192 -1.0%.
  // 17 to 32 rows: 32 x 12288 x 16384 (819 rows per wave) +8.8%, 17 x 16384 x 16384 (1024)
  // +5.2%, 32 x 8192 x 28672 (896) +3.8%, 24 x 8192 x 16384 (512) +2.3%, 32 x 16384 x 8192 (512)
  // +0.9%; 32 x 8192 x 12288 (384) +-0, 32 x 6144 x 16384 (410) -2.2%, 32 x 8192 x 8192 (256)
  // -1.3%, 32 x 4096 x 8192 (128) -11%.  33 to 64 rows: 48 x 12288 x 16384 (819) +19.5% (240
  // workgroups instead of 192), 64 x 8192 x 28672 (896) +4.2%, 64 x 8192 x 16384 (512) +1.9%,
  // 40 x 16384 x 16384 (1024) +1.2%, 64 x 16384 x 8192 (512) +1.0%; 48 x 8192 x 12288 (384)
  // -2.5%, 64 x 4096 x 14336 (224) -1.0%, 64 x 8192 x 8192 (256) -0.4%.  From an unsplit
  // 128-column grid only 33 to 64 rows, whose 128-column slots are one third A: 64 x 28672 x 8192
  // +6.6% (1024 rows per wave), 48 x 28672 x 8192 +2.7% (16 rows: -1.0%, above).
  if (!p.ws_absent && !b_unaligned && (splits >= 2 || mr == 4) && p.K >= 8192) {
    const int strips2 = (p.N + 255) / 256, splits2 = splits_for(256, strips2);
    if (splits2 >= 2 && strips2 * splits2 >= strips * splits && p.K / (4 * splits2) >= (mr == 1 ? 256 : 512))
      return {mr, 256, strips2, splits2};
  }
  return {mr, 128, strips, splits};
}

int skinny_splits(const GemmProblem& p) { return stream_shape(p).splits; }

int skinny_columns(const GemmProblem& p) { return stream_shape(p).splits ? stream_shape(p).ns : kNS; }

// More 128-column strips than CUs, on B rows that are not 16-byte aligned or with rounds less than
// 2/3 filled on average: the tile kernels run the problem faster.  Measured (B rotating through
// HBM, auto-picked tiles against the streaming kernel): unaligned 16 x 33001 x 8192 129 us against
// 207.6, 16 x 50257 x 4096 92.0 against 140.7, 64 x 50257 x 4096 100.3 against 155.9; aligned
// 16 x 33000 x 8192 (258 strips) 118.1 against 140.1, 16 x 40000 x 8192 (313) 121.8 against 128.2.
// Fuller rounds stream faster: 16 x 49152 x 8192 (384 strips) 150.4 against 172.1, 32 x 81920 x
// 4096 (640) 134.9 against 151.0, 16 x 151936 x 4096 (1187) 204.2 against 233.3, 16 x 65536 x
// 8192 174.4 against 186.7 (16 x 100000 x 4096, 782 strips: 184.9 streamed, 163.0 on tiles).
// Without a workspace the tiles run their last round unsplit, and on aligned rows the
// threshold rises to 1.8 (measured: 16 x 33000 x 8192, 1.98, tiles 130.2 against 165.5 streamed;
// 16 x 40000 x 8192, 1.64, tiles 129.4 against 123.3-125.2 streamed); unaligned rows still go to
// tiles (16 x 33001 x 8192 147.2 against 201.6; 16 x 50257 x 4096 96.0 against 126.9-130.2;
// 64 x 50257 x 4096 97.2 against 152.0).
bool skinny_prefers_tiles(const GemmProblem& p) {
  const StreamShape sh = stream_shape(p);
  if (sh.splits == 0) return false;  // the wave-split kernel
  const int wgs = sh.strips * sh.splits;
  if (wgs <= 256) return false;
  const bool b_unaligned = ((uintptr_t)p.B & 15) || p.ldb % 8;
  const double fill = (double)((wgs + 255) / 256) * 256.0 / wgs;  // rounds' slots per workgroup
  return b_unaligned || fill > (p.ws_absent ? 1.8 : 1.5);
}

// 33 to 64 rows on a 128-column grid of 2 or 3 K splits with K <= 4096 (many strips, short
// streams): the 64 x 64 tile kernel, whose B panels the M <= 64 rows share, runs them faster.
// Measured (B rotating through HBM, whole calls): 64 x 14336 x 4096 225.1 against 214.4 TFLOP/s
// streamed, 64 x 16384 x 4096 264.2 against 236.0, 64 x 11008 x 4096 190.5 against 180.8,
// 56 x 14336 x 4096 200.7 against 191.4, 48 x 14336 x 4096 174.3 against 166.7, 40 x 11008 x
// 4096 124.9 against 121.9.  At K = 8192 the same grids stream faster than the tile picked for
// them (64 x 10240 x 8192: 249.7 streamed, 175 on 64 x 64 tiles).
bool skinny_tiles_faster(const GemmProblem& p) {
  const StreamShape sh = stream_shape(p);
  return !p.ws_absent && sh.mr == 4 && sh.ns == 128 && sh.splits >= 2 && sh.splits <= 3 && p.K <= 4096;
}

size_t skinny_workspace_bytes(const GemmProblem& p) {
  const StreamShape sh = stream_shape(p);
  return sh.splits > 1 ? (size_t)sh.strips * sh.splits * (16 * sh.mr) * sh.ns * 4 : 0;
}

int skinny_workgroups(const GemmProblem& p) {
  const StreamShape sh = stream_shape(p);
  return sh.splits ? sh.strips * sh.splits : (p.N + kNS - 1) / kNS;
}

bool skinny_ok(const GemmProblem& p) {
  const uintptr_t a = (uintptr_t)p.A, b = (uintptr_t)p.B;
  if (p.M > kStreamMaxRows || p.M < 1) return false;
  if ((a & 1) || (b & 1)) return false;
  if ((int64_t)16 * stream_mr(p.M) * p.lda * 2 >= (int64_t)kOobOffset) return false;
  // B offsets are taken from the strip base: the whole operand must fit a 32-bit offset (a
  // larger B goes to the tile kernels, whose descriptors are rebased per K tile; with per-slot
  // descriptors here, 16 x 33001 x 66000 ran 1005 us against 915 on 64 x 64 tiles)
  if (((int64_t)p.K * p.ldb + 256) * 2 >= (int64_t)kOobOffset) return false;
  return true;
}

// B operands this large are streamed with non-temporal loads.  Measured on MI355X (interleaved,
// three B buffers rotating): 16 x 8192 x 8192 32.9 -> 30.8 us per call, 32 x 8192 x 8192 34.8 ->
// 32.7, 64 x 14336 x 4096 (112 MiB) 36.6 -> 35.4; with 64 MiB of B (16 x 4096 x 8192: three
// buffers fit the 256 MB Infinity Cache) 17.5 -> 18.4, slower, so smaller B keeps cached loads.
// The in-workgroup kernel's 64-byte strips ran 30-40% slower with them (not used there).
constexpr int64_t kNtStreamBytes = 96ll << 20;

template <int MR, int NS>
static hipError_t launch_wide(const GemmProblem& p, int strips, int splits, float* ws, hipStream_t stream) {
  if ((int64_t)p.K * p.N * 2 >= kNtStreamBytes)
    hipLaunchKernelGGL((gemm_stream_wide_kernel<MR, NS, true>), dim3(strips * splits), dim3(256), 0, stream, p, strips,
                       splits, ws);
  else
    hipLaunchKernelGGL((gemm_stream_wide_kernel<MR, NS, false>), dim3(strips * splits), dim3(256), 0, stream, p,
                       strips, splits, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  constexpr int ROWS = 16 * MR;
  hipLaunchKernelGGL((reduce_splits_kernel<ROWS, NS>), dim3(strips * (ROWS * NS / 4 / 256)), dim3(256), 0, stream, p,
                     strips, splits, (const float*)ws);
  return hipGetLastError();
}

hipError_t launch_gemm_skinny(const GemmProblem& p0, hipStream_t stream) {
  GemmProblem p = p0;
  const uintptr_t a = (uintptr_t)p.A, b = (uintptr_t)p.B;
  p.tail_regs = (a & 15) || (b & 15) || p.lda % 8 || p.ldb % 8 || p.K % 8 || p.N % 8;
  p.c_vec4 = (uintptr_t)p.C % 4 == 0;
  StreamShape sh = stream_shape(p);
  float* ws = sh.splits > 1 && p.ws && p.ws_bytes >= skinny_workspace_bytes(p) ? p.ws : nullptr;
  if (sh.splits > 1 && !ws && sh.mr > 1) sh.splits = 1;  // no workspace: one split
  if (sh.splits == 1 || ws) {
    switch (sh.mr) {
      case 1:
        return sh.ns == 256 ? launch_wide<1, 256>(p, sh.strips, sh.splits, ws, stream)
                            : launch_wide<1, 128>(p, sh.strips, sh.splits, ws, stream);
      case 2:
        return sh.ns == 256 ? launch_wide<2, 256>(p, sh.strips, sh.splits, ws, stream)
                            : launch_wide<2, 128>(p, sh.strips, sh.splits, ws, stream);
      default:
        return sh.ns == 256 ? launch_wide<4, 256>(p, sh.strips, sh.splits, ws, stream)
                            : launch_wide<4, 128>(p, sh.strips, sh.splits, ws, stream);
    }
  }
  // wave-split kernel (M <= 16): no caller workspace
  const int strips = (p.N + kNS - 1) / kNS;
  hipLaunchKernelGGL(gemm_skinny_kernel, dim3(strips), dim3(256), 0, stream, p, strips);
  return hipGetLastError();
}

}  // namespace mmm
