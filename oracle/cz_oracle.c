/*
 * cz_oracle.c - CPU restatement of colizig's block-FP8 MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle): used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product library.  Build: oracle/Makefile -> oracle/libczoracle.so.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add below is an
 * explicit fmaf()/_mm256_fmadd_ps where the reference uses @mulAdd, and every
 * `a * b + c` the reference writes without @mulAdd stays a separate multiply
 * and add (Zig's default strict float mode never contracts).
 *
 * Parity pins (checked in tests/test_oracle.py; none of them re-types a
 * formula from this file):
 *   czo_e4m3_decode / lut   closed form over all 256 bytes, torch.float8_e4m3fn
 *                           (a library decoder), and the reference's demo
 *                           bytes fp8.zig:263-271.
 *   czo_decode_lane /       bit-identical to lut[b]*scale for every byte
 *   czo_dequant_row         (the reference's own test fp8.zig:355-377).
 *   czo_dot_fp8_row(_scalar), czo_dot_f32(_scalar)
 *                           AVX2 == scalar lane emulation bit-for-bit; f64
 *                           brute force within the reference tolerances
 *                           (fp8.zig:273-353, matmul.zig:133-155); exact
 *                           results on integer-valued inputs.
 *   czo_expf                exhaustively within 1 ulp of the correctly
 *                           rounded exp (expl) and equal to it on all but a
 *                           counted handful of inputs.  The bits of Zig's @exp
 *                           itself cannot be observed here (no zig), so they
 *                           are "parity unpinned".
 *   czo_route               top-k against a brute-force stable argsort with
 *                           lowest-index ties; gates sum to 1 under norm_topk.
 *   czo_moe_forward         f64 brute force of the SwiGLU experts + combine at
 *                           1e-4 rel L2; grouped == per-token dense at 1e-3
 *                           abs (moe.zig:720-728); determinism.
 *   czo_cache_replay        hand-worked LRU traces (moe.zig:730-741).
 *   czo_chunk_bounds        disjoint cover of [0,n) (parallel.zig:348-375).
 *   czo_rms_unit /          float64 closed form x / sqrt(mean(x^2) + eps) at
 *   czo_chain_layer         1e-6; the reference's own rms tests
 *                           (rmsnorm.zig:67-100 restated as checks); the chain
 *                           step == rms, then moe.forward, then the residual add.
 */
#define _GNU_SOURCE
#include "cz_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define CZO_HAVE_X86 1
#else
#define CZO_HAVE_X86 0
#endif

/* ======================================================================= */
/* fp8.zig                                                                 */
/* ======================================================================= */

size_t czo_nblk(size_t x) { return (x + CZO_BLOCK - 1) / CZO_BLOCK; } /* fp8.zig:19-21 */

/* fp8.zig:55-64 pow2f: m * 2^k evaluated in f64 by repeated doubling/halving. */
static float czo_pow2f(float m, int k) {
    double r = m;
    int i = 0;
    if (k >= 0) {
        while (i < k) { r *= 2.0; i++; }
    } else {
        while (i > k) { r *= 0.5; i--; }
    }
    return (float)r;
}

/* fp8.zig:40-51 decodeE4M3 */
float czo_e4m3_decode(uint8_t byte) {
    const float sign = (byte & 0x80) ? -1.0f : 1.0f;
    const uint32_t e = (byte >> 3) & 0x0f;
    const uint32_t m = byte & 0x07;
    if (e == 0) {
        if (m == 0) return sign * 0.0f;
        return sign * czo_pow2f((float)m / 8.0f, 1 - 7);
    }
    if (e == 0x0f && m == 0x07) {
        const uint32_t nb = 0x7fc00000u;
        float nan;
        memcpy(&nan, &nb, 4);
        return sign * nan;
    }
    const float mm = 1.0f + (float)m / 8.0f;
    return sign * czo_pow2f(mm, (int)e - 7);
}

/* fp8.zig:33-38 e4m3_lut (comptime table of decodeE4M3) */
static float g_lut[256];
static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;
static void czo_build_lut(void) {
    for (int b = 0; b < 256; ++b) g_lut[b] = czo_e4m3_decode((uint8_t)b);
}
const float *czo_e4m3_lut(void) {
    pthread_once(&g_lut_once, czo_build_lut);
    return g_lut;
}

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* fp8.zig:80-106 decodeLane, one lane: the f32 bit pattern built
 * arithmetically, then ONE f32 multiply by the block scale. */
static inline float czo_decode_one(uint8_t byte, float sc) {
    const uint32_t b = byte;
    const uint32_t sign32 = (b >> 7) << 31;
    const uint32_t e = (b >> 3) & 0x0f;
    const uint32_t m = b & 0x07;
    const uint32_t normal_bits = sign32 | ((e + 120u) << 23) | (m << 20);
    const float mant_f = (float)m;
    const uint32_t subn_bits = f32_bits(mant_f * 0x1p-9f) | sign32;
    uint32_t bits = (e == 0) ? subn_bits : normal_bits;
    if (e == 15 && m == 7) bits = 0x7fc00000u;
    return bits_f32(bits) * sc;
}

void czo_decode_lane(const uint8_t *bytes, float sc, float *out8) {
    for (unsigned l = 0; l < CZO_LANES; ++l) out8[l] = czo_decode_one(bytes[l], sc);
}

/* fp8.zig:123-130 dequantRow: full L-lane chunks through decodeLane, tail
 * through the LUT (same single multiply). */
void czo_dequant_row(float *out, const uint8_t *w, const float *scale_row, size_t n) {
    const float *lut = czo_e4m3_lut();
    size_t i = 0;
    for (; i + CZO_LANES <= n; i += CZO_LANES) {
        const float sc = scale_row[i / CZO_BLOCK];
        czo_decode_lane(w + i, sc, out + i);
    }
    for (; i < n; ++i) out[i] = lut[w[i]] * scale_row[i / CZO_BLOCK];
}

void czo_dequant_matrix(float *out, const uint8_t *w, const float *scales, size_t rows, size_t cols) {
    const size_t nbi = czo_nblk(cols);
    for (size_t o = 0; o < rows; ++o)
        czo_dequant_row(out + o * cols, w + o * cols, scales + (o / CZO_BLOCK) * nbi, cols);
}

/* Sequential lane reduction: Zig's @reduce(.Add) in strict float mode is the
 * ordered LLVM reduction ((((-0 + v0) + v1) + ...) + v7). */
static inline float czo_reduce8(const float *v) {
    float s = -0.0f;
    for (unsigned l = 0; l < CZO_LANES; ++l) s = s + v[l];
    return s;
}

/* fp8.zig:137-160 dotFp8Row, scalar lane emulation (L = 8, two
 * accumulators: chunk i -> acc0, chunk i+L -> acc1). */
float czo_dot_fp8_row_scalar(const float *x, const uint8_t *w, const float *scale_row, size_t n) {
    const float *lut = czo_e4m3_lut();
    float acc0[CZO_LANES] = {0}, acc1[CZO_LANES] = {0};
    size_t i = 0;
    for (; i + 2 * CZO_LANES <= n; i += 2 * CZO_LANES) {
        const float sc0 = scale_row[i / CZO_BLOCK];
        for (unsigned l = 0; l < CZO_LANES; ++l)
            acc0[l] = fmaf(x[i + l], czo_decode_one(w[i + l], sc0), acc0[l]);
        const float sc1 = scale_row[(i + CZO_LANES) / CZO_BLOCK];
        for (unsigned l = 0; l < CZO_LANES; ++l)
            acc1[l] = fmaf(x[i + CZO_LANES + l], czo_decode_one(w[i + CZO_LANES + l], sc1), acc1[l]);
    }
    for (; i + CZO_LANES <= n; i += CZO_LANES) {
        const float sc = scale_row[i / CZO_BLOCK];
        for (unsigned l = 0; l < CZO_LANES; ++l)
            acc0[l] = fmaf(x[i + l], czo_decode_one(w[i + l], sc), acc0[l]);
    }
    float v[CZO_LANES];
    for (unsigned l = 0; l < CZO_LANES; ++l) v[l] = acc0[l] + acc1[l];
    float sum = czo_reduce8(v);
    for (; i < n; ++i) {
        const float prod = x[i] * (lut[w[i]] * scale_row[i / CZO_BLOCK]);
        sum = sum + prod;
    }
    return sum;
}

/* matmul.zig:60-82 dotF32, scalar lane emulation (L = 8, four accumulator
 * chains over 32-element steps, then 8-element steps into acc[0]). */
float czo_dot_f32_scalar(const float *a, const float *b, size_t n) {
    float acc[4][CZO_LANES];
    memset(acc, 0, sizeof acc);
    size_t i = 0;
    for (; i + 4 * CZO_LANES <= n; i += 4 * CZO_LANES)
        for (unsigned k = 0; k < 4; ++k)
            for (unsigned l = 0; l < CZO_LANES; ++l)
                acc[k][l] = fmaf(a[i + k * CZO_LANES + l], b[i + k * CZO_LANES + l], acc[k][l]);
    for (; i + CZO_LANES <= n; i += CZO_LANES)
        for (unsigned l = 0; l < CZO_LANES; ++l) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    float total[CZO_LANES];
    for (unsigned l = 0; l < CZO_LANES; ++l) total[l] = 0.0f;
    for (unsigned k = 0; k < 4; ++k)
        for (unsigned l = 0; l < CZO_LANES; ++l) total[l] = total[l] + acc[k][l];
    float sum = czo_reduce8(total);
    for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

#if CZO_HAVE_X86
/* AVX2 forms of the same three kernels: identical operation order, used for
 * speed (the CPU baseline).  tests check them bit-for-bit against the scalar
 * emulations above. */
__attribute__((target("avx2,fma"))) static inline __m256 czo_decode_lane_avx2(const uint8_t *bytes, __m256 sc) {
    const __m256i b = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)bytes));
    const __m256i sign32 = _mm256_slli_epi32(_mm256_srli_epi32(b, 7), 31);
    const __m256i e = _mm256_and_si256(_mm256_srli_epi32(b, 3), _mm256_set1_epi32(0x0f));
    const __m256i m = _mm256_and_si256(b, _mm256_set1_epi32(0x07));
    const __m256i normal = _mm256_or_si256(
        sign32, _mm256_or_si256(_mm256_slli_epi32(_mm256_add_epi32(e, _mm256_set1_epi32(120)), 23),
                                _mm256_slli_epi32(m, 20)));
    const __m256 mant_f = _mm256_cvtepi32_ps(m);
    const __m256i subn =
        _mm256_or_si256(_mm256_castps_si256(_mm256_mul_ps(mant_f, _mm256_set1_ps(0x1p-9f))), sign32);
    const __m256i e0 = _mm256_cmpeq_epi32(e, _mm256_setzero_si256());
    __m256i bits = _mm256_blendv_epi8(normal, subn, e0);
    const __m256i isnan = _mm256_and_si256(_mm256_cmpeq_epi32(e, _mm256_set1_epi32(15)),
                                           _mm256_cmpeq_epi32(m, _mm256_set1_epi32(7)));
    bits = _mm256_blendv_epi8(bits, _mm256_set1_epi32(0x7fc00000), isnan);
    return _mm256_mul_ps(_mm256_castsi256_ps(bits), sc);
}

__attribute__((target("avx2,fma"))) static float czo_dot_fp8_row_avx2(const float *x, const uint8_t *w,
                                                                        const float *scale_row, size_t n) {
    const float *lut = czo_e4m3_lut();
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        const __m256 w0 = czo_decode_lane_avx2(w + i, _mm256_set1_ps(scale_row[i / CZO_BLOCK]));
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), w0, acc0);
        const __m256 w1 = czo_decode_lane_avx2(w + i + 8, _mm256_set1_ps(scale_row[(i + 8) / CZO_BLOCK]));
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), w1, acc1);
    }
    for (; i + 8 <= n; i += 8) {
        const __m256 wv = czo_decode_lane_avx2(w + i, _mm256_set1_ps(scale_row[i / CZO_BLOCK]));
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), wv, acc0);
    }
    float v[8];
    _mm256_storeu_ps(v, _mm256_add_ps(acc0, acc1));
    float sum = czo_reduce8(v);
    for (; i < n; ++i) {
        const float prod = x[i] * (lut[w[i]] * scale_row[i / CZO_BLOCK]);
        sum = sum + prod;
    }
    return sum;
}

__attribute__((target("avx2,fma"))) static float czo_dot_f32_avx2(const float *a, const float *b, size_t n) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps(), acc2 = _mm256_setzero_ps(),
           acc3 = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), acc1);
        acc2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), acc2);
        acc3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), acc3);
    }
    for (; i + 8 <= n; i += 8) acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    __m256 total = _mm256_setzero_ps();
    total = _mm256_add_ps(total, acc0);
    total = _mm256_add_ps(total, acc1);
    total = _mm256_add_ps(total, acc2);
    total = _mm256_add_ps(total, acc3);
    float v[8];
    _mm256_storeu_ps(v, total);
    float sum = czo_reduce8(v);
    for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

static int czo_have_avx2(void) {
    static int cached = -1;
    if (cached < 0) {
        __builtin_cpu_init();
        cached = (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) ? 1 : 0;
        if (getenv("CZO_FORCE_SCALAR")) cached = 0;
    }
    return cached;
}
#endif

float czo_dot_fp8_row(const float *x, const uint8_t *w, const float *scale_row, size_t n) {
#if CZO_HAVE_X86
    if (czo_have_avx2()) return czo_dot_fp8_row_avx2(x, w, scale_row, n);
#endif
    return czo_dot_fp8_row_scalar(x, w, scale_row, n);
}

float czo_dot_f32(const float *a, const float *b, size_t n) {
#if CZO_HAVE_X86
    if (czo_have_avx2()) return czo_dot_f32_avx2(a, b, n);
#endif
    return czo_dot_f32_scalar(a, b, n);
}

/* ======================================================================= */
/* parallel.zig:50-76 chunks: contiguous split, serial below min_work, and  */
/* never nested (a chunk body running on a worker stays serial).            */
/* ======================================================================= */

#define CZO_MIN_WORK ((size_t)96 * 1024) /* parallel.zig:20 */
#define CZO_MAX_THREADS 256

typedef void (*czo_body_fn)(void *ctx, size_t lo, size_t hi);

static uint32_t g_max_tasks = 1;
static __thread int g_in_worker = 0;

typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_job;
    pthread_cond_t cv_done;
    uint64_t gen;
    int nthreads; /* worker threads started */
    /* current job */
    czo_body_fn body;
    void *ctx;
    size_t n, csize;
    uint32_t nchunks;
    uint32_t next_chunk;
    uint32_t done_chunks;
    int quit;
    pthread_t th[CZO_MAX_THREADS];
} czo_pool;

static czo_pool g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .cv_job = PTHREAD_COND_INITIALIZER,
                          .cv_done = PTHREAD_COND_INITIALIZER};

static void czo_run_chunk(uint32_t c) {
    const size_t lo = (size_t)c * g_pool.csize;
    size_t hi = lo + g_pool.csize;
    if (hi > g_pool.n) hi = g_pool.n;
    g_in_worker = 1;
    g_pool.body(g_pool.ctx, lo, hi);
    g_in_worker = 0;
}

static void *czo_worker(void *arg) {
    (void)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (!g_pool.quit && (g_pool.gen == seen || g_pool.next_chunk >= g_pool.nchunks))
            pthread_cond_wait(&g_pool.cv_job, &g_pool.mu);
        if (g_pool.quit) break;
        seen = g_pool.gen;
        while (g_pool.next_chunk < g_pool.nchunks) {
            const uint32_t c = g_pool.next_chunk++;
            pthread_mutex_unlock(&g_pool.mu);
            czo_run_chunk(c);
            pthread_mutex_lock(&g_pool.mu);
            g_pool.done_chunks++;
            if (g_pool.done_chunks == g_pool.nchunks) pthread_cond_broadcast(&g_pool.cv_done);
        }
    }
    pthread_mutex_unlock(&g_pool.mu);
    return NULL;
}

static void czo_pool_stop(void) {
    pthread_mutex_lock(&g_pool.mu);
    g_pool.quit = 1;
    pthread_cond_broadcast(&g_pool.cv_job);
    pthread_mutex_unlock(&g_pool.mu);
    for (int i = 0; i < g_pool.nthreads; ++i) pthread_join(g_pool.th[i], NULL);
    g_pool.nthreads = 0;
    g_pool.quit = 0;
}

void czo_parallel_enable(uint32_t max_tasks) {
    if (max_tasks == 0) {
        long n = sysconf(_SC_NPROCESSORS_ONLN);
        max_tasks = n > 0 ? (uint32_t)n : 1;
    }
    if (max_tasks > CZO_MAX_THREADS) max_tasks = CZO_MAX_THREADS;
    if (g_pool.nthreads) czo_pool_stop();
    g_max_tasks = max_tasks;
    for (uint32_t i = 0; i + 1 < max_tasks; ++i) {
        if (pthread_create(&g_pool.th[i], NULL, czo_worker, NULL) != 0) break;
        g_pool.nthreads++;
    }
}

void czo_parallel_disable(void) {
    if (g_pool.nthreads) czo_pool_stop();
    g_max_tasks = 1;
}

uint32_t czo_parallel_max_tasks(void) { return g_max_tasks; }

static int czo_serial(size_t n, size_t work) {
    const uint32_t tasks = g_max_tasks < n ? g_max_tasks : (uint32_t)n;
    return tasks <= 1 || work < CZO_MIN_WORK || g_in_worker || g_pool.nthreads == 0;
}

uint32_t czo_chunk_bounds(size_t n, size_t work, uint32_t *lo_hi, uint32_t max_out) {
    if (n == 0) return 0;
    const uint32_t tasks = g_max_tasks < n ? g_max_tasks : (uint32_t)n;
    if (tasks <= 1 || work < CZO_MIN_WORK) {
        if (max_out) { lo_hi[0] = 0; lo_hi[1] = (uint32_t)n; }
        return 1;
    }
    const size_t csize = (n + tasks - 1) / tasks;
    uint32_t c = 0;
    for (size_t lo = 0; lo < n; lo += csize, ++c) {
        if (c < max_out) {
            lo_hi[2 * c] = (uint32_t)lo;
            lo_hi[2 * c + 1] = (uint32_t)(lo + csize < n ? lo + csize : n);
        }
    }
    return c;
}

static void czo_chunks(size_t n, size_t work, void *ctx, czo_body_fn body) {
    if (n == 0) return;
    if (czo_serial(n, work)) {
        body(ctx, 0, n);
        return;
    }
    const uint32_t tasks = g_max_tasks < n ? g_max_tasks : (uint32_t)n;
    const size_t csize = (n + tasks - 1) / tasks;
    pthread_mutex_lock(&g_pool.mu);
    g_pool.body = body;
    g_pool.ctx = ctx;
    g_pool.n = n;
    g_pool.csize = csize;
    g_pool.nchunks = (uint32_t)((n + csize - 1) / csize);
    g_pool.next_chunk = 1; /* the caller runs chunk 0 */
    g_pool.done_chunks = 0;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.cv_job);
    pthread_mutex_unlock(&g_pool.mu);
    czo_run_chunk(0);
    pthread_mutex_lock(&g_pool.mu);
    g_pool.done_chunks++;
    /* help with any chunk nobody has picked up yet */
    while (g_pool.next_chunk < g_pool.nchunks) {
        const uint32_t c = g_pool.next_chunk++;
        pthread_mutex_unlock(&g_pool.mu);
        czo_run_chunk(c);
        pthread_mutex_lock(&g_pool.mu);
        g_pool.done_chunks++;
    }
    while (g_pool.done_chunks < g_pool.nchunks) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

/* ======================================================================= */
/* matmuls                                                                  */
/* ======================================================================= */

typedef struct {
    float *y;
    const float *x;
    const uint8_t *w;
    const float *scales;
    const float *wf;
    size_t S, I, O, nbi;
} czo_mm_ctx;

static void czo_fp8_s1_body(void *p, size_t o0, size_t o1) {
    const czo_mm_ctx *c = (const czo_mm_ctx *)p;
    for (size_t o = o0; o < o1; ++o)
        c->y[o] = czo_dot_fp8_row(c->x, c->w + o * c->I, c->scales + (o / CZO_BLOCK) * c->nbi, c->I);
}

static void czo_fp8_sn_body(void *p, size_t o0, size_t o1) {
    const czo_mm_ctx *c = (const czo_mm_ctx *)p;
    float *wf = (float *)malloc(c->I * sizeof(float));
    if (!wf) abort();
    for (size_t o = o0; o < o1; ++o) {
        czo_dequant_row(wf, c->w + o * c->I, c->scales + (o / CZO_BLOCK) * c->nbi, c->I);
        for (size_t s = 0; s < c->S; ++s) c->y[s * c->O + o] = czo_dot_f32(c->x + s * c->I, wf, c->I);
    }
    free(wf);
}

/* fp8.zig:215-257 matmulFp8Cpu: S==1 fused decode+dot per output row; S>1
 * dequantises each weight row once, then dotF32 against every input row. */
void czo_matmul_fp8(float *y, const float *x, const uint8_t *w, const float *scales, size_t S, size_t I,
                    size_t O) {
    czo_mm_ctx c = {y, x, w, scales, NULL, S, I, O, czo_nblk(I)};
    if (S == 1) {
        czo_chunks(O, O * I, &c, czo_fp8_s1_body);
        return;
    }
    czo_chunks(O, O * I * S, &c, czo_fp8_sn_body);
}

static void czo_f32_body(void *p, size_t o0, size_t o1) {
    const czo_mm_ctx *c = (const czo_mm_ctx *)p;
    for (size_t o = o0; o < o1; ++o) {
        const float *wr = c->wf + o * c->I;
        for (size_t s = 0; s < c->S; ++s) c->y[s * c->O + o] = czo_dot_f32(c->x + s * c->I, wr, c->I);
    }
}

/* matmul.zig:21-33 */
void czo_matmul_f32(float *y, const float *x, const float *w, size_t S, size_t I, size_t O) {
    czo_mm_ctx c = {y, x, NULL, NULL, w, S, I, O, 0};
    czo_chunks(O, O * I * S, &c, czo_f32_body);
}

/* ======================================================================= */
/* activation.zig                                                           */
/* ======================================================================= */

/* f32 exp.  Zig's @exp(f32) bits are not observable in this container, so
 * the oracle fixes one faithful f32 exp and states it: the f32 rounding of a
 * double-precision evaluation -
 *   k = nearest integer to x/ln2   (round-to-nearest-even shifter 0x1.8p52)
 *   r = x - k*ln2                  (two fma steps, ln2 split hi/lo)
 *   p = sum_{n=0}^{13} r^n/n!      (Horner with fma; truncation < 2^-57)
 *   y = p * 2^k                    (exact power-of-two scaling)
 *   return (float)y                (round to nearest even)
 * which is within 1 ulp of exp(x) everywhere and correctly rounded on all but
 * a handful of inputs (counted exhaustively in tests). */
float czo_expf(float xf) {
    if (xf != xf) return xf + xf;
    double x = (double)xf;
    if (x > 100.0) x = 100.0;   /* -> +inf after rounding */
    if (x < -120.0) x = -120.0; /* -> +0 after rounding */
    const double inv_ln2 = 0x1.71547652b82fep+0;
    const double ln2_hi = 0x1.62e42fefa39efp-1;
    const double ln2_lo = 0x1.abc9e3b39803fp-56;
    const double shifter = 0x1.8p52;
    const double t0 = x * inv_ln2;
    const double t1 = t0 + shifter;
    const double kd = t1 - shifter;
    double r = fma(-kd, ln2_hi, x);
    r = fma(-kd, ln2_lo, r);
    /* 1/n! for n = 13 .. 1 */
    double p = 0x1.6124613a86d09p-33; /* 1/13! */
    p = fma(p, r, 0x1.1eed8eff8d898p-29); /* 1/12! */
    p = fma(p, r, 0x1.ae64567f544e4p-26); /* 1/11! */
    p = fma(p, r, 0x1.27e4fb7789f5cp-22); /* 1/10! */
    p = fma(p, r, 0x1.71de3a556c734p-19); /* 1/9! */
    p = fma(p, r, 0x1.a01a01a01a01ap-16); /* 1/8! */
    p = fma(p, r, 0x1.a01a01a01a01ap-13); /* 1/7! */
    p = fma(p, r, 0x1.6c16c16c16c17p-10); /* 1/6! */
    p = fma(p, r, 0x1.1111111111111p-7);  /* 1/5! */
    p = fma(p, r, 0x1.5555555555555p-5);  /* 1/4! */
    p = fma(p, r, 0x1.5555555555555p-3);  /* 1/3! */
    p = fma(p, r, 0x1.0000000000000p-1);  /* 1/2! */
    p = fma(p, r, 1.0);                   /* 1/1! */
    p = fma(p, r, 1.0);                   /* 1/0! */
    const int k = (int)kd;
    const uint64_t sbits = (uint64_t)(int64_t)(k + 1023) << 52;
    double scale;
    memcpy(&scale, &sbits, 8);
    return (float)(p * scale);
}

void czo_expf_array(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = czo_expf(in[i]);
}

/* activation.zig:9-16 numerically stable sigmoid */
float czo_sigmoid(float x) {
    if (x >= 0) {
        const float z = czo_expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = czo_expf(x);
    return z / (1.0f + z);
}

/* activation.zig:18-20 */
float czo_silu(float x) { return x * czo_sigmoid(x); }

/* ======================================================================= */
/* moe.zig                                                                  */
/* ======================================================================= */

/* tensors.zig:114-119 NativeMatrix(f32).matmul -> matmul.zig:21-33 (S=1) */
void czo_router_logits(const czo_layer *L, const float *xs, float *logits) {
    czo_matmul_f32(logits, xs, L->router, 1, L->d.hidden, L->d.experts);
    /* optional per-expert bias, one f32 add after the dot: a workload-shaping
     * extension (skewed routing); the reference's route has no bias term */
    if (L->router_bias)
        for (uint32_t e = 0; e < L->d.experts; ++e) logits[e] = logits[e] + L->router_bias[e];
}

/* moe.zig:435-463 route */
void czo_route(const czo_layer *L, const float *xs, uint32_t *idx, float *gates, float *logits_out) {
    const uint32_t E = L->d.experts, K = L->d.topk;
    float *lg = (float *)malloc((size_t)E * sizeof(float));
    if (!lg) abort();
    czo_router_logits(L, xs, lg);
    float mx = lg[0];
    for (uint32_t e = 0; e < E; ++e) mx = fmaxf(mx, lg[e]); /* @max: the non-NaN operand */
    double all = 0;
    for (uint32_t e = 0; e < E; ++e) {
        lg[e] = czo_expf(lg[e] - mx);
        all += (double)lg[e];
    }
    double top = 0;
    for (uint32_t z = 0; z < K; ++z) {
        uint32_t best = 0;
        float bv = -1.0f;
        for (uint32_t e = 0; e < E; ++e) {
            int chosen = 0;
            for (uint32_t j = 0; j < z; ++j) chosen = chosen || (idx[j] == e);
            if (!chosen && lg[e] > bv) {
                bv = lg[e];
                best = e;
            }
        }
        idx[z] = best;
        top += (double)lg[best];
    }
    const double den = L->d.norm_topk ? top : all;
    for (uint32_t z = 0; z < K; ++z) gates[z] = (float)((double)lg[idx[z]] / den);
    if (logits_out) memcpy(logits_out, lg, (size_t)E * sizeof(float));
    free(lg);
}

/* moe.zig:467-479 addSharedExpert (no-op without a shared expert). */
static void czo_add_shared(const czo_layer *L, const float *xs, float *ys, float *sg, float *su, float *sh,
                           float *shared) {
    const czo_dims *d = &L->d;
    if (d->shared_inter == 0) return;
    const uint32_t H = d->hidden, SI = d->shared_inter;
    if (L->sh_native_gate) { /* NativeMatrix.matmul (tensors.zig:114-119) */
        czo_matmul_f32(sg, xs, L->sh_native_gate, 1, H, SI);
        czo_matmul_f32(su, xs, L->sh_native_up, 1, H, SI);
    } else {
        czo_matmul_fp8(sg, xs, L->sh_gate_proj.w, L->sh_gate_proj.s, 1, H, SI);
        czo_matmul_fp8(su, xs, L->sh_up_proj.w, L->sh_up_proj.s, 1, H, SI);
    }
    for (uint32_t j = 0; j < SI; ++j) sh[j] = czo_silu(sg[j]) * su[j];
    if (L->sh_native_down)
        czo_matmul_f32(shared, sh, L->sh_native_down, 1, SI, H);
    else
        czo_matmul_fp8(shared, sh, L->sh_down_proj.w, L->sh_down_proj.s, 1, SI, H);
    float sgate = 0;
    for (uint32_t dd = 0; dd < H; ++dd) {
        const float prod = xs[dd] * L->sh_gate[dd];
        sgate = sgate + prod;
    }
    sgate = czo_sigmoid(sgate);
    for (uint32_t dd = 0; dd < H; ++dd) {
        const float prod = sgate * shared[dd];
        ys[dd] = ys[dd] + prod;
    }
}

typedef struct {
    const czo_layer *L;
    const uint32_t *idx;
    const float *xs;
    const float *gates;
    float *eg, *eu, *eh, *eo;
} czo_eval_ctx;

/* moe.zig:556-570 evalExpertBody: one expert per task, disjoint eo rows,
 * eo *= g before the serial reduce. */
static void czo_eval_body(void *p, size_t z0, size_t z1) {
    const czo_eval_ctx *c = (const czo_eval_ctx *)p;
    const uint32_t H = c->L->d.hidden, I = c->L->d.inter;
    for (size_t z = z0; z < z1; ++z) {
        const czo_expert *ex = &c->L->experts[c->idx[z]];
        float *eg = c->eg + z * I, *eu = c->eu + z * I, *eh = c->eh + z * I, *eo = c->eo + z * H;
        czo_matmul_fp8(eg, c->xs, ex->gate.w, ex->gate.s, 1, H, I);
        czo_matmul_fp8(eu, c->xs, ex->up.w, ex->up.s, 1, H, I);
        for (uint32_t j = 0; j < I; ++j) eh[j] = czo_silu(eg[j]) * eu[j];
        czo_matmul_fp8(eo, eh, ex->down.w, ex->down.s, 1, I, H);
        const float g = c->gates[z];
        for (uint32_t dd = 0; dd < H; ++dd) eo[dd] = eo[dd] * g;
    }
}

/* moe.zig:481-539 forwardDense (the parallel form, par = true: every expert
 * resident, K <= 64; bit-identical to the serial form, moe.zig:510-514). */
static int czo_forward_dense(const czo_layer *L, const float *x, size_t S, float *out, uint32_t *r_idx,
                             float *r_gate) {
    const czo_dims *d = &L->d;
    const uint32_t H = d->hidden, K = d->topk, I = d->inter, SI = d->shared_inter;
    uint32_t *idx = (uint32_t *)malloc(K * sizeof(uint32_t));
    float *gates = (float *)malloc(K * sizeof(float));
    float *eg = (float *)malloc((size_t)K * I * sizeof(float));
    float *eu = (float *)malloc((size_t)K * I * sizeof(float));
    float *eh = (float *)malloc((size_t)K * I * sizeof(float));
    float *eo = (float *)malloc((size_t)K * H * sizeof(float));
    float *sbuf = (float *)malloc(((size_t)3 * SI + H + 1) * sizeof(float));
    int rc = 0;
    if (!idx || !gates || !eg || !eu || !eh || !eo || !sbuf) {
        rc = -1;
        goto done;
    }
    for (size_t s = 0; s < S; ++s) {
        const float *xs = x + s * H;
        float *ys = out + s * H;
        memset(ys, 0, H * sizeof(float));
        czo_route(L, xs, idx, gates, NULL);
        czo_eval_ctx c = {L, idx, xs, gates, eg, eu, eh, eo};
        czo_chunks(K, (size_t)K * 3 * I * H, &c, czo_eval_body);
        for (uint32_t z = 0; z < K; ++z)
            for (uint32_t dd = 0; dd < H; ++dd) ys[dd] = ys[dd] + eo[(size_t)z * H + dd];
        czo_add_shared(L, xs, ys, sbuf, sbuf + SI, sbuf + 2 * SI, sbuf + 3 * SI);
        if (r_idx) memcpy(r_idx + s * K, idx, K * sizeof(uint32_t));
        if (r_gate) memcpy(r_gate + s * K, gates, K * sizeof(float));
    }
done:
    free(idx);
    free(gates);
    free(eg);
    free(eu);
    free(eh);
    free(eo);
    free(sbuf);
    return rc;
}

static const uint32_t *g_sort_keys;
static int czo_slot_cmp(const void *a, const void *b) {
    const uint32_t sa = *(const uint32_t *)a, sb = *(const uint32_t *)b;
    const uint32_t ka = g_sort_keys[sa], kb = g_sort_keys[sb];
    if (ka != kb) return ka < kb ? -1 : 1;
    return sa < sb ? -1 : (sa > sb); /* tie order cannot change any result */
}

/* moe.zig:597-665 forwardGrouped: route all tokens (shared expert first),
 * order the S*K (token, slot) pairs by expert id, evaluate each distinct
 * expert once over its rows, scatter out[tok] += gate * row. */
static int czo_forward_grouped(const czo_layer *L, const float *x, size_t S, float *out, uint32_t *r_idx_out,
                               float *r_gate_out) {
    const czo_dims *d = &L->d;
    const uint32_t H = d->hidden, K = d->topk, I = d->inter, SI = d->shared_inter;
    const size_t M = S * K;
    uint32_t *r_idx = (uint32_t *)malloc(M * sizeof(uint32_t));
    float *r_gate = (float *)malloc(M * sizeof(float));
    uint32_t *ord = (uint32_t *)malloc(M * sizeof(uint32_t));
    float *xb = (float *)malloc(S * H * sizeof(float));
    float *bg = (float *)malloc(S * I * sizeof(float));
    float *bu = (float *)malloc(S * I * sizeof(float));
    float *bo = (float *)malloc(S * H * sizeof(float));
    float *sbuf = (float *)malloc(((size_t)3 * SI + H + 1) * sizeof(float));
    int rc = 0;
    if (!r_idx || !r_gate || !ord || !xb || !bg || !bu || !bo || !sbuf) {
        rc = -1;
        goto done;
    }
    for (size_t s = 0; s < S; ++s) {
        const float *xs = x + s * H;
        float *ys = out + s * H;
        memset(ys, 0, H * sizeof(float));
        czo_route(L, xs, r_idx + s * K, r_gate + s * K, NULL);
        czo_add_shared(L, xs, ys, sbuf, sbuf + SI, sbuf + 2 * SI, sbuf + 3 * SI);
    }
    for (size_t i = 0; i < M; ++i) ord[i] = (uint32_t)i;
    g_sort_keys = r_idx;
    qsort(ord, M, sizeof(uint32_t), czo_slot_cmp);
    for (size_t p = 0; p < M;) {
        const uint32_t eid = r_idx[ord[p]];
        size_t q = p;
        while (q < M && r_idx[ord[q]] == eid) q++;
        const size_t n = q - p;
        for (size_t k = 0; k < n; ++k) memcpy(xb + k * H, x + (size_t)(ord[p + k] / K) * H, H * sizeof(float));
        const czo_expert *ex = &L->experts[eid];
        czo_matmul_fp8(bg, xb, ex->gate.w, ex->gate.s, n, H, I);
        czo_matmul_fp8(bu, xb, ex->up.w, ex->up.s, n, H, I);
        for (size_t j = 0; j < n * I; ++j) bg[j] = czo_silu(bg[j]) * bu[j];
        czo_matmul_fp8(bo, bg, ex->down.w, ex->down.s, n, I, H);
        for (size_t k = 0; k < n; ++k) {
            const uint32_t slot = ord[p + k];
            const size_t tok = slot / K;
            const float g = r_gate[slot];
            float *ys = out + tok * H;
            const float *eo = bo + k * H;
            for (uint32_t dd = 0; dd < H; ++dd) {
                const float prod = g * eo[dd];
                ys[dd] = ys[dd] + prod;
            }
        }
        p = q;
    }
    if (r_idx_out) memcpy(r_idx_out, r_idx, M * sizeof(uint32_t));
    if (r_gate_out) memcpy(r_gate_out, r_gate, M * sizeof(float));
done:
    free(r_idx);
    free(r_gate);
    free(ord);
    free(xb);
    free(bg);
    free(bu);
    free(bo);
    free(sbuf);
    return rc;
}

/* moe.zig:409-426 forward */
int czo_moe_forward(const czo_layer *L, const float *x, size_t S, float *out, uint32_t *r_idx, float *r_gate) {
    if (S == 1) return czo_forward_dense(L, x, S, out, r_idx, r_gate);
    return czo_forward_grouped(L, x, S, out, r_idx, r_gate);
}

int czo_moe_forward_dense_each(const czo_layer *L, const float *x, size_t S, float *out, uint32_t *r_idx,
                               float *r_gate) {
    return czo_forward_dense(L, x, S, out, r_idx, r_gate);
}

/* ======================================================================= */
/* moe.zig:141-249 ExpertCache policy (LRU by use clock; victim = first    */
/* empty slot, else the first slot with the smallest `used`).              */
/* ======================================================================= */
uint32_t czo_cache_replay(uint32_t cap, const uint32_t *ids, size_t n, int32_t *slot_out, czo_cache_stats *st) {
    if (cap == 0) return 0;
    int64_t *id = (int64_t *)malloc(cap * sizeof(int64_t));
    uint64_t *used = (uint64_t *)calloc(cap, sizeof(uint64_t));
    if (!id || !used) abort();
    for (uint32_t i = 0; i < cap; ++i) id[i] = -1;
    uint64_t clock = 0;
    czo_cache_stats s;
    memset(&s, 0, sizeof s);
    for (size_t t = 0; t < n; ++t) {
        int32_t hit = -1;
        for (uint32_t i = 0; i < cap; ++i)
            if (id[i] == (int64_t)ids[t]) { hit = (int32_t)i; break; }
        if (hit >= 0) { /* moe.zig:221-231 */
            clock++;
            used[hit] = clock;
            s.hits++;
            if (slot_out) slot_out[t] = hit;
            continue;
        }
        s.misses++;
        uint32_t victim = 0; /* moe.zig:183-197 */
        int found_empty = 0;
        for (uint32_t i = 0; i < cap; ++i) {
            if (id[i] < 0) { victim = i; found_empty = 1; break; }
            if (used[i] < used[victim]) victim = i;
        }
        if (!found_empty) s.evictions++;
        id[victim] = ids[t]; /* moe.zig:199-217 fill */
        clock++;
        used[victim] = clock;
        s.loads++;
        if (slot_out) slot_out[t] = (int32_t)victim;
    }
    uint32_t resident = 0;
    for (uint32_t i = 0; i < cap; ++i) resident += id[i] >= 0;
    if (st) *st = s;
    free(id);
    free(used);
    return resident;
}

/* ExpertCache over (layer, expert) keys with pins and prefetch marks: the
 * library's HBM pool policy, restated from moe.zig:141-248 (see the header). */
int64_t czo_pool_replay(uint32_t nslots, const uint32_t *ops, size_t n, uint32_t *res_out, czo_pool_stats *st) {
    if (nslots == 0) return -1;
    uint64_t *key = (uint64_t *)calloc(nslots, sizeof(uint64_t)); /* 0 = empty, else 1 + (layer << 32 | expert) */
    uint64_t *used = (uint64_t *)calloc(nslots, sizeof(uint64_t));
    uint64_t *pin = (uint64_t *)calloc(nslots, sizeof(uint64_t));
    uint8_t *pref = (uint8_t *)calloc(nslots, 1);
    if (!key || !used || !pin || !pref) abort();
    uint64_t clock = 0, epoch = 0;
    czo_pool_stats s;
    memset(&s, 0, sizeof s);
    int64_t rc = 0;
    for (size_t t = 0; t < n && rc == 0; ++t) {
        const uint32_t op = ops[4 * t], layer = ops[4 * t + 1], e = ops[4 * t + 2];
        const uint64_t k = 1ull + (((uint64_t)layer << 32) | e);
        uint32_t res = 0;
        int32_t at = -1;
        for (uint32_t i = 0; i < nslots; ++i)
            if (key[i] == k) { at = (int32_t)i; break; }
        if (op == 0) {
            epoch++;
        } else if (op == 4) {
            for (uint32_t i = 0; i < nslots; ++i) { key[i] = 0; pref[i] = 0; }
        } else if (op == 1 && at >= 0) { /* get: hit */
            s.hits++;
            if (pref[at]) { s.prefetch_hits++; pref[at] = 0; }
            used[at] = ++clock;
            pin[at] = epoch;
            res = (uint32_t)at | 0x80000000u;
        } else if (op == 2 && at >= 0) { /* prefetch of a resident expert */
            res = 0xfffffffeu;
        } else {
            /* a fill: get miss, prefetch or warm */
            int32_t v = -1;
            for (uint32_t i = 0; i < nslots; ++i)
                if (key[i] == 0) { v = (int32_t)i; break; }
            if (v < 0 && op != 3) {
                for (uint32_t i = 0; i < nslots; ++i) {
                    if (pin[i] == epoch && epoch != 0) continue;
                    if (v < 0 || used[i] < used[v]) v = (int32_t)i;
                }
            }
            if (v < 0) {
                if (op == 1) { rc = -1; break; }
                res = 0xffffffffu; /* prefetch dropped / no free slot to warm */
            } else {
                if (key[v]) { s.evictions++; if (pref[v]) s.prefetch_wasted++; }
                key[v] = k;
                used[v] = ++clock;
                s.loads++;
                pref[v] = op != 1;
                if (op != 1) s.prefetch_issued++;
                if (op == 1) { s.misses++; pin[v] = epoch; }
                res = (uint32_t)v;
            }
        }
        if (res_out) res_out[t] = res;
    }
    int64_t resident = 0;
    for (uint32_t i = 0; i < nslots; ++i) resident += key[i] != 0;
    if (st) *st = s;
    free(key); free(used); free(pin); free(pref);
    return rc < 0 ? -1 : resident;
}

/* ======================================================================= */
/* the decode chain: x <- x + moe(rms(x)) per layer                        */
/* ======================================================================= */
/* rmsnorm.zig:32-40 `rms` with a unit weight, the norm qwen3moe/model.zig:228
 * applies before each MoE block: ss = sum of f64(v)*v over the row (each
 * square exact in f64), in row order; mean = f32(ss / n); r = 1 / sqrt(mean +
 * eps) in f32; out_i = x_i * r * w_i with w_i = 1 (an exact multiply). */
void czo_rms_unit(float *out, const float *x, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float mean = (float)(ss / (double)n);
    const float r = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * r * 1.0f;
}

int czo_chain_layer(const czo_layer *L, float *x, size_t S, float eps, float *xn_out, uint32_t *r_idx,
                    float *r_gate) {
    const uint32_t H = L->d.hidden;
    float *xn = (float *)calloc(S * H, sizeof(float));
    float *o = (float *)calloc(S * H, sizeof(float));
    if (!xn || !o) { free(xn); free(o); return -1; }
    for (size_t s = 0; s < S; ++s) czo_rms_unit(xn + s * H, x + s * H, H, eps);
    /* qwen3moe/model.zig:230-232: the MoE block's output added to the residual */
    int rc = czo_moe_forward(L, xn, S, o, r_idx, r_gate);
    if (rc == 0) {
        for (size_t i = 0; i < S * H; ++i) x[i] = x[i] + o[i];
        if (xn_out) memcpy(xn_out, xn, S * H * sizeof(float));
    }
    free(xn);
    free(o);
    return rc;
}
