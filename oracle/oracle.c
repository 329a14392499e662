/*
 * oracle.c -- CPU restatement of the reference's FP16->FP32 GEMM / 5-D contraction path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or as the timed CPU
 * baseline).  The product library never links, loads or calls anything in oracle/.
 *
 * Reference: thrasos-g/RDNA4-GEMM-WMMA (files mmm.cpp, mmmTensor.cpp).  Every function
 * below cites the reference lines it restates, or says what pins it when the reference
 * has nothing to restate (the input generator and the fp64 truth are ours).
 *
 * fp16 values travel as uint16_t bit patterns (IEEE binary16).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>
#include <stdatomic.h>
#include <unistd.h>
#include <immintrin.h>

/* ------------------------------------------------------------------------------------ */
/* Minimal pthread parallel-for (no OpenMP: the oracle is loaded into processes that also  */
/* carry torch's own OpenMP runtime, and two OpenMP runtimes in one process are unsafe).   */
/* Thread count: ORACLE_THREADS, else OMP_NUM_THREADS, else online CPUs; capped at 256.     */
/* ------------------------------------------------------------------------------------ */
typedef void (*orc_body_fn)(int64_t begin, int64_t end, void* ctx);

int orc_max_threads(void) {
    const char* e = getenv("ORACLE_THREADS");
    if (!e || !*e) e = getenv("OMP_NUM_THREADS");
    long n = e && *e ? strtol(e, NULL, 10) : sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    return (int)n;
}

typedef struct {
    atomic_llong next;
    int64_t n, chunk;
    orc_body_fn body;
    void* ctx;
} pf_job;

static void* pf_worker(void* arg) {
    pf_job* j = (pf_job*)arg;
    for (;;) {
        int64_t b = (int64_t)atomic_fetch_add(&j->next, j->chunk);
        if (b >= j->n) break;
        int64_t e = b + j->chunk < j->n ? b + j->chunk : j->n;
        j->body(b, e, j->ctx);
    }
    return NULL;
}

/* Runs body over [0, n) in chunks of `chunk`, dynamically scheduled over `threads`
 * threads (<= 0: orc_max_threads()). */
static void parallel_for(int64_t n, int64_t chunk, int threads, orc_body_fn body, void* ctx) {
    if (n <= 0) return;
    if (chunk < 1) chunk = 1;
    if (threads <= 0) threads = orc_max_threads();
    int64_t nchunks = (n + chunk - 1) / chunk;
    if (threads > nchunks) threads = (int)nchunks;
    pf_job j;
    atomic_init(&j.next, 0);
    j.n = n, j.chunk = chunk, j.body = body, j.ctx = ctx;
    if (threads <= 1) {
        pf_worker(&j);
        return;
    }
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)(threads - 1));
    int started = 0;
    for (int t = 0; t < threads - 1; ++t)
        if (pthread_create(&tids[t], NULL, pf_worker, &j) == 0) started++;
        else break;
    pf_worker(&j);
    for (int t = 0; t < started; ++t) pthread_join(tids[t], NULL);
    free(tids);
}

/* ------------------------------------------------------------------------------------ */
/* fp16 <-> fp32/fp64 conversions (bit exact, round-to-nearest-even).                    */
/* Pinned by tests against numpy's float16 casts over every fp16 value and random floats. */
/* ------------------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: value = mant * 2^-24, exact in fp32 */
            float v = (float)mant * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    int32_t e = (int32_t)(ax >> 23) - 127;
    if (e >= -14) {
        uint32_t mant = ax & 0x7fffffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return sign | (uint16_t)h;
    }
    if (ax == 0) return sign;
    /* half subnormal: h = round(value / 2^-24) */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    if (e < -127 + 1) { /* fp32 subnormal input: far below half range */
        return sign;
    }
    int shift = -(e + 1); /* value = mant * 2^(e-23); h = mant * 2^(e+1) */
    if (shift > 24) return sign;
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

uint16_t orc_f64_to_f16(double d) {
    uint64_t x;
    memcpy(&x, &d, 8);
    uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    uint64_t ax = x & 0x7fffffffffffffffull;
    if (ax >= 0x7ff0000000000000ull) {
        if (ax == 0x7ff0000000000000ull) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 42) & 0x3ffu);
    }
    if (ax >= 0x40effe0000000000ull) return sign | 0x7c00u; /* >= 65520 */
    int32_t e = (int32_t)(ax >> 52) - 1023;
    if (e >= -14) {
        uint64_t mant = ax & 0xfffffffffffffull;
        uint64_t h = ((uint64_t)(e + 15) << 10) | (mant >> 42);
        uint64_t rem = mant & ((1ull << 42) - 1ull);
        uint64_t half = 1ull << 41;
        if (rem > half || (rem == half && (h & 1ull))) h++;
        return sign | (uint16_t)h;
    }
    if (ax == 0) return sign;
    if (e < -1022) return sign; /* fp64 subnormal */
    uint64_t mant = (ax & 0xfffffffffffffull) | (1ull << 52);
    int shift = 28 - e; /* value = mant*2^(e-52); h = mant*2^(e-28) */
    if (shift > 53) return sign;
    uint64_t h = mant >> shift;
    uint64_t rem = mant & ((1ull << shift) - 1ull);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (h & 1ull))) h++;
    return sign | (uint16_t)h;
}

/* Array forms of the conversions (for tests that sweep many values). */
void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}
void orc_f64_to_f16_array(const double* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f64_to_f16(in[i]);
}
void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

static float g_f16_lut[65536];
static int g_lut_ready = 0;

static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;

static void lut_fill(void) {
    for (uint32_t i = 0; i < 65536u; ++i) g_f16_lut[i] = orc_f16_to_f32((uint16_t)i);
    g_lut_ready = 1;
}

static void lut_init(void) { pthread_once(&g_lut_once, lut_fill); }

/* ------------------------------------------------------------------------------------ */
/* Seeded input generator.  The reference draws unseeded rand()/RAND_MAX in [0,1)        */
/* (mmm.cpp:1409-1414, srand(time) at mmm.cpp:1455; mmmTensor.cpp:271-276), which is not  */
/* reproducible; this build defines a counter-based stream instead so that the CPU and     */
/* the GPU produce the same tensors:                                                      */
/*   key   = splitmix64(seed * 0x9E3779B97F4A7C15 + tensor_id + 1)                        */
/*   x_i   = splitmix64(key + i)                                                          */
/*   uniform[-1,1):  v = (x_i >> 40) * 2^-23 - 1   (exact in fp32), then fp16 RNE          */
/*   normal*scale:   Box-Muller in fp64 on u1 = ((x_{2i} >> 11) + 1) * 2^-53,             */
/*                   u2 = (x_{2i+1} >> 11) * 2^-53; v = sqrt(-2 ln u1) cos(2 pi u2) * scale */
/*                   rounded once from fp64 to fp16 RNE.                                   */
/* Pinned by committed known-answer vectors and by the mathematics of splitmix64 (its     */
/* published first outputs for seed 0).                                                   */
/* ------------------------------------------------------------------------------------ */

uint64_t orc_splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint32_t tensor_id) {
    return orc_splitmix64(seed * 0x9E3779B97F4A7C15ull + (uint64_t)tensor_id + 1ull);
}

typedef struct {
    uint16_t* out;
    uint64_t key;
    double scale;
} fill_ctx;

static void fill_uniform_body(int64_t b, int64_t e, void* vctx) {
    fill_ctx* c = (fill_ctx*)vctx;
    for (int64_t i = b; i < e; ++i) {
        uint64_t x = orc_splitmix64(c->key + (uint64_t)i);
        float v = (float)(uint32_t)(x >> 40) * 1.1920928955078125e-07f - 1.0f;
        c->out[i] = orc_f32_to_f16(v);
    }
}

static void fill_normal_body(int64_t b, int64_t e, void* vctx) {
    fill_ctx* c = (fill_ctx*)vctx;
    for (int64_t i = b; i < e; ++i) {
        uint64_t x1 = orc_splitmix64(c->key + 2ull * (uint64_t)i);
        uint64_t x2 = orc_splitmix64(c->key + 2ull * (uint64_t)i + 1ull);
        double u1 = (double)((x1 >> 11) + 1ull) * 1.1102230246251565e-16;
        double u2 = (double)(x2 >> 11) * 1.1102230246251565e-16;
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        c->out[i] = orc_f64_to_f16(z * c->scale);
    }
}

void orc_fill_uniform_f16(uint16_t* out, int64_t n, uint64_t seed, uint32_t tensor_id) {
    fill_ctx c = {out, stream_key(seed, tensor_id), 0.0};
    parallel_for(n, 1 << 16, 0, fill_uniform_body, &c);
}

void orc_fill_normal_f16(uint16_t* out, int64_t n, uint64_t seed, uint32_t tensor_id, double scale) {
    fill_ctx c = {out, stream_key(seed, tensor_id), scale};
    parallel_for(n, 1 << 15, 0, fill_normal_body, &c);
}

/* ------------------------------------------------------------------------------------ */
/* fp64 ground truth with the tolerance scale S = sum_k |a_ik * b_kj|.                   */
/* C[i][j] = sum_k A[i*lda + k] * B[k*ldb + j]  -- the GEMM definition of                 */
/* mmm.cpp:52-62 (row-major A [M][K], B [K][N]), evaluated in fp64 (fp16*fp16 products    */
/* are exact in fp64).  rows/cols select a sub-grid: C and S are [nr][nc].                */
/* b_kstride/b_nstride generalise B's layout so the TN operand of mmmTensor.cpp:168       */
/* (B[k][j] at j*ldb + k) uses the same routine.                                          */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    const uint16_t *A, *B;
    int64_t a_mstride, a_kstride, b_kstride, b_nstride, K;
    const int64_t *rows, *cols;
    int64_t nc;
    double *C, *S;
    float* Cf;
    int64_t lda, ldb;
} gemm_ctx;

static void gemm_f64_body(int64_t rb, int64_t re, void* vctx) {
    gemm_ctx* g = (gemm_ctx*)vctx;
    const int64_t nc = g->nc;
    double* acc = (double*)malloc(sizeof(double) * (size_t)nc);
    double* sab = (double*)malloc(sizeof(double) * (size_t)nc);
    double* brow = (double*)malloc(sizeof(double) * (size_t)nc);
    for (int64_t r = rb; r < re; ++r) {
        const int64_t i = g->rows[r];
        for (int64_t c = 0; c < nc; ++c) { acc[c] = 0.0; sab[c] = 0.0; }
        for (int64_t k = 0; k < g->K; ++k) {
            double a = (double)g_f16_lut[g->A[i * g->a_mstride + k * g->a_kstride]];
            if (a == 0.0) continue;
            const uint16_t* bk = g->B + k * g->b_kstride;
            for (int64_t c = 0; c < nc; ++c) brow[c] = (double)g_f16_lut[bk[g->cols[c] * g->b_nstride]];
            double aa = fabs(a);
            for (int64_t c = 0; c < nc; ++c) {
                acc[c] += a * brow[c];
                sab[c] += aa * fabs(brow[c]);
            }
        }
        for (int64_t c = 0; c < nc; ++c) {
            g->C[r * nc + c] = acc[c];
            if (g->S) g->S[r * nc + c] = sab[c];
        }
    }
    free(acc);
    free(sab);
    free(brow);
}

void orc_gemm_f64_sub(const uint16_t* A, int64_t a_mstride, int64_t a_kstride,
                      const uint16_t* B, int64_t b_kstride, int64_t b_nstride, int64_t K,
                      const int64_t* rows, int64_t nr, const int64_t* cols, int64_t nc,
                      double* C, double* S) {
    lut_init();
    gemm_ctx g = {A, B, a_mstride, a_kstride, b_kstride, b_nstride, K, rows, cols, nc, C, S, NULL, 0, 0};
    parallel_for(nr, 1, 0, gemm_f64_body, &g);
}

/* ------------------------------------------------------------------------------------ */
/* Restatements of the reference kernels' fp32 arithmetic.                               */
/* ------------------------------------------------------------------------------------ */

/* GEMM_Naive (mmm.cpp:52-62): one fp32 accumulator per output, k ascending,
 * acc += float(a) * float(b).  rows/cols select the sub-grid; C is [nr][nc]. */
static void gemm_naive_body(int64_t rb, int64_t re, void* vctx) {
    gemm_ctx* g = (gemm_ctx*)vctx;
    for (int64_t r = rb; r < re; ++r) {
        const int64_t i = g->rows[r];
        for (int64_t c = 0; c < g->nc; ++c) {
            const int64_t j = g->cols[c];
            float acc = 0.0f;
            for (int64_t k = 0; k < g->K; ++k) acc += g_f16_lut[g->A[i * g->lda + k]] * g_f16_lut[g->B[k * g->ldb + j]];
            g->Cf[r * g->nc + c] = acc;
        }
    }
}

void orc_gemm_naive_f32_sub(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, int64_t K,
                            const int64_t* rows, int64_t nr, const int64_t* cols, int64_t nc, float* C) {
    lut_init();
    gemm_ctx g = {A, B, 0, 0, 0, 0, K, rows, cols, nc, NULL, NULL, C, lda, ldb};
    parallel_for(nr, 1, 0, gemm_naive_body, &g);
}

/* WMMA_Swizzled_Full (mmm.cpp:1309-1356; bounds handling of mmmTensor.cpp:135-178):
 * K is walked in LDS tiles of 32 (k += LDS_K, mmm.cpp:1309), each split into two 16-deep
 * WMMA steps (tk = 0, 16, mmm.cpp:1323).  One WMMA step adds a 16-term dot product to the
 * fp32 accumulator (C = A*B + C, mmm.cpp:1353); the order of the 16 terms inside the
 * instruction is unspecified by the reference, and is taken here as ascending k in fp32.
 * Elements with k >= K are zero-filled exactly as the tensor variant's masked loads do
 * (mmmTensor.cpp:137-148, 164-175). */
static void gemm_refkernel_body(int64_t rb, int64_t re, void* vctx) {
    gemm_ctx* g = (gemm_ctx*)vctx;
    for (int64_t r = rb; r < re; ++r) {
        const int64_t i = g->rows[r];
        for (int64_t c = 0; c < g->nc; ++c) {
            const int64_t j = g->cols[c];
            float acc = 0.0f;
            for (int64_t k0 = 0; k0 < g->K; k0 += 32) {      /* LDS_K tile */
                for (int64_t tk = 0; tk < 32; tk += 16) { /* WMMA step */
                    float step = 0.0f;
                    for (int64_t e = 0; e < 16; ++e) {
                        int64_t k = k0 + tk + e;
                        float a = 0.0f, b = 0.0f;
                        if (k < g->K) {
                            a = g_f16_lut[g->A[i * g->a_mstride + k * g->a_kstride]];
                            b = g_f16_lut[g->B[k * g->b_kstride + j * g->b_nstride]];
                        }
                        step += a * b;
                    }
                    acc += step;
                }
            }
            g->Cf[r * g->nc + c] = acc;
        }
    }
}

void orc_gemm_refkernel_f32_sub(const uint16_t* A, int64_t a_mstride, int64_t a_kstride,
                                const uint16_t* B, int64_t b_kstride, int64_t b_nstride, int64_t K,
                                const int64_t* rows, int64_t nr, const int64_t* cols, int64_t nc,
                                float* C) {
    lut_init();
    gemm_ctx g = {A, B, a_mstride, a_kstride, b_kstride, b_nstride, K, rows, cols, nc, NULL, NULL, C, 0, 0};
    parallel_for(nr, 1, 0, gemm_refkernel_body, &g);
}

/* ------------------------------------------------------------------------------------ */
/* 5-D contractions as plain loop nests (independent of any GEMM fold).                   */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    const uint16_t *A, *B;
    int64_t d[5];
    const int64_t* sel;
    double *C, *S;
} contract_ctx;

/* Baseline layout: C[b,i,j] = sum_{k,l} A[b,i,k,l] * B[k,l,j]; all tensors dense in the
 * listed index order.  Not in the reference; it is the benchmark's contraction.  Output is
 * computed for the (b,i) pairs listed in bi (pairs b*ni + i) and every j; C, S are
 * [nbi][nj].  The loop nest walks k then l explicitly, never forming a folded index. */
static void contract_baseline_body(int64_t pb, int64_t pe, void* vctx) {
    contract_ctx* x = (contract_ctx*)vctx;
    const int64_t ni = x->d[0], nk = x->d[1], nl = x->d[2], nj = x->d[3];
    for (int64_t p = pb; p < pe; ++p) {
        const int64_t b = x->sel[p] / ni, i = x->sel[p] % ni;
        double* c = x->C + p * nj;
        double* s = x->S ? x->S + p * nj : NULL;
        for (int64_t j = 0; j < nj; ++j) {
            c[j] = 0.0;
            if (s) s[j] = 0.0;
        }
        for (int64_t k = 0; k < nk; ++k) {
            for (int64_t l = 0; l < nl; ++l) {
                double a = (double)g_f16_lut[x->A[((b * ni + i) * nk + k) * nl + l]];
                if (a == 0.0) continue;
                const uint16_t* brow = x->B + (k * nl + l) * nj;
                for (int64_t j = 0; j < nj; ++j) {
                    double bv = (double)g_f16_lut[brow[j]];
                    c[j] += a * bv;
                    if (s) s[j] += fabs(a * bv);
                }
            }
        }
    }
}

void orc_contract_baseline_f64(const uint16_t* A, const uint16_t* B, int64_t ni, int64_t nk, int64_t nl,
                               int64_t nj, const int64_t* bi, int64_t nbi, double* C, double* S) {
    lut_init();
    contract_ctx x = {A, B, {ni, nk, nl, nj, 0}, bi, C, S};
    parallel_for(nbi, 1, 0, contract_baseline_body, &x);
}

/* Reference layout (mmmTensor.cpp): Out[m][b][r] = sum_{n,l} G[r][n][m][l] * In[b][n][l]
 * with G of shape [rt][nt][mt][rt_l], In [bt][nt][rt_l], Out [mt][bt][rt].  This follows
 * the host pack (mmmTensor.cpp:329-340: A[(m*rt + r)][(n*rt_l + l)] = G[r][n][m][l]),
 * the TN read of Input (mmmTensor.cpp:168: B[k][j] = Input[j*DIM_K + k]) and the output
 * remap (mmmTensor.cpp:246-252: Out[m*bt*rt + b*rt + r]).  Computed for the (m, r) pairs
 * listed in mr (pairs m*rt + r) and every b; C, S are [nmr][bt] indexed [p][b]. */
static void contract_reference_body(int64_t pb, int64_t pe, void* vctx) {
    contract_ctx* x = (contract_ctx*)vctx;
    const int64_t mt = x->d[0], bt = x->d[1], rt = x->d[2], nt = x->d[3], rt_l = x->d[4];
    for (int64_t p = pb; p < pe; ++p) {
        const int64_t m = x->sel[p] / rt, r = x->sel[p] % rt;
        for (int64_t b = 0; b < bt; ++b) {
            double acc = 0.0, sab = 0.0;
            for (int64_t n = 0; n < nt; ++n) {
                for (int64_t l = 0; l < rt_l; ++l) {
                    double g = (double)g_f16_lut[x->A[((r * nt + n) * mt + m) * rt_l + l]];
                    double v = (double)g_f16_lut[x->B[(b * nt + n) * rt_l + l]];
                    acc += g * v;
                    sab += fabs(g * v);
                }
            }
            x->C[p * bt + b] = acc;
            if (x->S) x->S[p * bt + b] = sab;
        }
    }
}

void orc_contract_reference_f64(const uint16_t* G, const uint16_t* In, int64_t mt, int64_t bt, int64_t rt,
                                int64_t nt, int64_t rt_l, const int64_t* mr, int64_t nmr, double* C, double* S) {
    lut_init();
    contract_ctx x = {G, In, {mt, bt, rt, nt, rt_l}, mr, C, S};
    parallel_for(nmr, 1, 0, contract_reference_body, &x);
}

/* The reference's host-side pack of G into the GEMM operand A (mmmTensor.cpp:329-340),
 * single-threaded, in the reference's loop order. */
void orc_pack_reference_G(const uint16_t* G, uint16_t* hA, int64_t mt, int64_t rt, int64_t nt, int64_t rt_l) {
    const int64_t DIM_K = nt * rt_l;
    for (int64_t r = 0; r < rt; r++)
        for (int64_t m = 0; m < mt; m++)
            for (int64_t n = 0; n < nt; n++)
                for (int64_t k = 0; k < rt_l; k++) {
                    int64_t row_A = m * rt + r;
                    int64_t col_A = n * rt_l + k;
                    int64_t g_idx = (r * nt * mt * rt_l) + (n * mt * rt_l) + (m * rt_l) + k;
                    hA[row_A * DIM_K + col_A] = G[g_idx];
                }
}

/* ------------------------------------------------------------------------------------ */
/* Reference block remap (mmm.cpp:1219-1236 == mmmTensor.cpp:50-65).                     */
/* ------------------------------------------------------------------------------------ */
void orc_ref_block_remap(int bx, int by, int gx, int gy, int* sx, int* sy) {
    int S = 32;
    if (gx < S) S = gx;
    int block_id = by * gx + bx;
    int blocks_per_group = S * gy;
    int group_id = block_id / blocks_per_group;
    int group_lane = block_id % blocks_per_group;
    int x = group_id * S + (group_lane % S);
    int y = group_lane / S;
    if (x >= gx) { x = bx; y = by; }
    *sx = x;
    *sy = y;
}

/* ------------------------------------------------------------------------------------ */
/* Tolerance check: |C - T| <= rel * S elementwise (fp32 result C, fp64 truth T).         */
/* Returns the number of violations; *worst receives max |C-T| / max(S, tiny).            */
/* ------------------------------------------------------------------------------------ */
int64_t orc_check_tol(const float* C, int64_t c_stride_r, const double* T, const double* S, int64_t nr, int64_t nc,
                      double rel, double* worst) {
    int64_t bad = 0;
    double w = 0.0;
    for (int64_t r = 0; r < nr; ++r)
        for (int64_t c = 0; c < nc; ++c) {
            double d = fabs((double)C[r * c_stride_r + c] - T[r * nc + c]);
            double s = S[r * nc + c];
            if (!(d <= rel * s)) bad++; /* NaN counts as a violation */
            double q = d / (s > 1e-300 ? s : 1e-300);
            if (q > w || q != q) w = q;
        }
    if (worst) *worst = w;
    return bad;
}

/* ------------------------------------------------------------------------------------ */
/* Multithreaded CPU FP16->FP32 GEMM (the reported CPU baseline).  fp16 panels are        */
/* converted with F16C and multiplied by a 6x16 AVX2/FMA micro-kernel, fp32 accumulate.   */
/* C[M][N] (ldc) = A[M][K] (lda) * B[K][N] (ldb), row-major, overwrite.                   */
/* ------------------------------------------------------------------------------------ */
#define CB_MR 6
#define CB_NR 16
#define CB_KC 256
#define CB_MC 72

static void cb_kernel_6x16(int64_t kc, const float* ap, const float* bp, float* c, int64_t ldc) {
    __m256 c00 = _mm256_loadu_ps(c + 0 * ldc), c01 = _mm256_loadu_ps(c + 0 * ldc + 8);
    __m256 c10 = _mm256_loadu_ps(c + 1 * ldc), c11 = _mm256_loadu_ps(c + 1 * ldc + 8);
    __m256 c20 = _mm256_loadu_ps(c + 2 * ldc), c21 = _mm256_loadu_ps(c + 2 * ldc + 8);
    __m256 c30 = _mm256_loadu_ps(c + 3 * ldc), c31 = _mm256_loadu_ps(c + 3 * ldc + 8);
    __m256 c40 = _mm256_loadu_ps(c + 4 * ldc), c41 = _mm256_loadu_ps(c + 4 * ldc + 8);
    __m256 c50 = _mm256_loadu_ps(c + 5 * ldc), c51 = _mm256_loadu_ps(c + 5 * ldc + 8);
    for (int64_t k = 0; k < kc; ++k) {
        __m256 b0 = _mm256_loadu_ps(bp + k * CB_NR), b1 = _mm256_loadu_ps(bp + k * CB_NR + 8);
        __m256 a;
        a = _mm256_broadcast_ss(ap + k * CB_MR + 0); c00 = _mm256_fmadd_ps(a, b0, c00); c01 = _mm256_fmadd_ps(a, b1, c01);
        a = _mm256_broadcast_ss(ap + k * CB_MR + 1); c10 = _mm256_fmadd_ps(a, b0, c10); c11 = _mm256_fmadd_ps(a, b1, c11);
        a = _mm256_broadcast_ss(ap + k * CB_MR + 2); c20 = _mm256_fmadd_ps(a, b0, c20); c21 = _mm256_fmadd_ps(a, b1, c21);
        a = _mm256_broadcast_ss(ap + k * CB_MR + 3); c30 = _mm256_fmadd_ps(a, b0, c30); c31 = _mm256_fmadd_ps(a, b1, c31);
        a = _mm256_broadcast_ss(ap + k * CB_MR + 4); c40 = _mm256_fmadd_ps(a, b0, c40); c41 = _mm256_fmadd_ps(a, b1, c41);
        a = _mm256_broadcast_ss(ap + k * CB_MR + 5); c50 = _mm256_fmadd_ps(a, b0, c50); c51 = _mm256_fmadd_ps(a, b1, c51);
    }
    _mm256_storeu_ps(c + 0 * ldc, c00); _mm256_storeu_ps(c + 0 * ldc + 8, c01);
    _mm256_storeu_ps(c + 1 * ldc, c10); _mm256_storeu_ps(c + 1 * ldc + 8, c11);
    _mm256_storeu_ps(c + 2 * ldc, c20); _mm256_storeu_ps(c + 2 * ldc + 8, c21);
    _mm256_storeu_ps(c + 3 * ldc, c30); _mm256_storeu_ps(c + 3 * ldc + 8, c31);
    _mm256_storeu_ps(c + 4 * ldc, c40); _mm256_storeu_ps(c + 4 * ldc + 8, c41);
    _mm256_storeu_ps(c + 5 * ldc, c50); _mm256_storeu_ps(c + 5 * ldc + 8, c51);
}

static inline void cvt_f16_row(const uint16_t* src, float* dst, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(src + i))));
    for (; i < n; ++i) dst[i] = g_f16_lut[src[i]];
}

typedef struct {
    const uint16_t *A, *B;
    float* C;
    float* bpack;
    int64_t lda, ldb, ldc, M, N, k0, kc, np;
} cpu_gemm_ctx;

static void cb_zero_body(int64_t b, int64_t e, void* vctx) {
    cpu_gemm_ctx* g = (cpu_gemm_ctx*)vctx;
    for (int64_t i = b; i < e; ++i) memset(g->C + i * g->ldc, 0, sizeof(float) * (size_t)g->N);
}

/* pack B[k0:k0+kc][:] into slivers [np][kc][16] */
static void cb_packb_body(int64_t b, int64_t e, void* vctx) {
    cpu_gemm_ctx* g = (cpu_gemm_ctx*)vctx;
    for (int64_t p = b; p < e; ++p) {
        float* dst = g->bpack + p * CB_NR * CB_KC;
        const int64_t j0 = p * CB_NR;
        const int64_t w = (g->N - j0 < CB_NR) ? (g->N - j0) : CB_NR;
        for (int64_t k = 0; k < g->kc; ++k) {
            const uint16_t* src = g->B + (g->k0 + k) * g->ldb + j0;
            if (w == CB_NR) {
                cvt_f16_row(src, dst + k * CB_NR, CB_NR);
            } else {
                for (int64_t j = 0; j < CB_NR; ++j) dst[k * CB_NR + j] = j < w ? g_f16_lut[src[j]] : 0.0f;
            }
        }
    }
}

static void cb_main_body(int64_t b, int64_t e, void* vctx) {
    cpu_gemm_ctx* g = (cpu_gemm_ctx*)vctx;
    const int64_t M = g->M, N = g->N, kc = g->kc, k0 = g->k0, ldc = g->ldc;
    float* C = g->C;
    float* apack = (float*)aligned_alloc(64, sizeof(float) * CB_MC * CB_KC);
    float* arow = (float*)malloc(sizeof(float) * CB_KC);
    float ctmp[CB_MR * CB_NR];
    for (int64_t mb = b; mb < e; ++mb) {
        const int64_t i0 = mb * CB_MC;
        const int64_t mc = (M - i0 < CB_MC) ? (M - i0) : CB_MC;
        const int64_t ngroups = (mc + CB_MR - 1) / CB_MR;
        /* pack A[i0:i0+mc][k0:k0+kc] into groups [g][kc][6] */
        for (int64_t q = 0; q < ngroups; ++q)
            for (int64_t r = 0; r < CB_MR; ++r) {
                int64_t i = i0 + q * CB_MR + r;
                if (q * CB_MR + r < mc) cvt_f16_row(g->A + i * g->lda + k0, arow, kc);
                else memset(arow, 0, sizeof(float) * (size_t)kc);
                for (int64_t k = 0; k < kc; ++k) apack[q * CB_MR * CB_KC + k * CB_MR + r] = arow[k];
            }
        for (int64_t p = 0; p < g->np; ++p) {
            const int64_t j0 = p * CB_NR;
            const int64_t w = (N - j0 < CB_NR) ? (N - j0) : CB_NR;
            for (int64_t q = 0; q < ngroups; ++q) {
                const int64_t ib = i0 + q * CB_MR;
                const int64_t h = (mc - q * CB_MR < CB_MR) ? (mc - q * CB_MR) : CB_MR;
                if (h == CB_MR && w == CB_NR) {
                    cb_kernel_6x16(kc, apack + q * CB_MR * CB_KC, g->bpack + p * CB_NR * CB_KC, C + ib * ldc + j0, ldc);
                } else {
                    for (int64_t r = 0; r < CB_MR; ++r)
                        for (int64_t j = 0; j < CB_NR; ++j)
                            ctmp[r * CB_NR + j] = (r < h && j < w) ? C[(ib + r) * ldc + j0 + j] : 0.0f;
                    cb_kernel_6x16(kc, apack + q * CB_MR * CB_KC, g->bpack + p * CB_NR * CB_KC, ctmp, CB_NR);
                    for (int64_t r = 0; r < h; ++r)
                        for (int64_t j = 0; j < w; ++j) C[(ib + r) * ldc + j0 + j] = ctmp[r * CB_NR + j];
                }
            }
        }
    }
    free(apack);
    free(arow);
}

void orc_cpu_gemm_f16f32(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, float* C, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, int nthreads) {
    lut_init();
    if (nthreads <= 0) nthreads = orc_max_threads();
    cpu_gemm_ctx g = {A, B, C, NULL, lda, ldb, ldc, M, N, 0, 0, (N + CB_NR - 1) / CB_NR};
    g.bpack = (float*)aligned_alloc(64, sizeof(float) * (size_t)(g.np * CB_NR * CB_KC));
    parallel_for(M, 64, nthreads, cb_zero_body, &g);
    for (int64_t k0 = 0; k0 < K; k0 += CB_KC) {
        g.k0 = k0;
        g.kc = (K - k0 < CB_KC) ? (K - k0) : CB_KC;
        parallel_for(g.np, 8, nthreads, cb_packb_body, &g);
        parallel_for((M + CB_MC - 1) / CB_MC, 1, nthreads, cb_main_body, &g);
    }
    free(g.bpack);
}
