/* Host C int8 path: the CPU baseline and the bit-level oracle. TEST
 * INFRASTRUCTURE ONLY (imported by tests/, smoke() and bench.py's CPU leg).
 *
 * The per-token int8 projection on the host, with the structure of the
 * reference's int8 recipe (schedules.py:303-323): weight rows outside tokens,
 * rows in blocks of 16 handed to a persistent thread pool (pool.c), and the
 * dot product in 32-byte VPDPBUSD groups with the +128 trick that lets an
 * unsigned-by-signed instruction multiply signed bytes (codegen_avx2.py:66-71,
 * loopir.Dp4 at loopir.py:137-150): sum (w + 128) * x, minus 128 * sum x.
 *
 * The ISA is picked at run time, so one build runs on any x86-64 host:
 * AVX-512 VNNI, else AVX-VNNI, else AVX2 (vpmaddwd on sign-extended bytes),
 * else scalar. Every form is exact in int32, so all of them produce the same
 * integers; nc_host_isa() says which one ran.
 *
 * Float code is compiled with -ffp-contract=off, as the reference's is
 * (codegen_c.py:50), so the epilogue rounds where the source says it does.
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <immintrin.h>

/* The same expf/sinf/cosf the GPU kernels use (one source for both). */
#include "../nanocompile_amd/csrc/nc_math.h"

#define EXPORT __attribute__((visibility("default")))

/* -- thread pool ----------------------------------------------------------- */

#include "nc_host.h"

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_start = PTHREAD_COND_INITIALIZER;
static pthread_cond_t g_done = PTHREAD_COND_INITIALIZER;
static int g_threads = 1;               /* workers + the caller */
static int g_spawned = 0;
static int64_t g_generation = 0;
static int g_pending = 0;
static task_fn g_fn;
static void *g_ctx;
static int64_t g_n;
static atomic_llong g_next;
static pthread_t g_workers[256];

static void run_tasks(void) {
    for (;;) {
        int64_t i = atomic_fetch_add(&g_next, 1);
        if (i >= g_n) return;
        g_fn(g_ctx, i);
    }
}

static void *worker(void *arg) {
    (void)arg;
    int64_t seen = 0;
    pthread_mutex_lock(&g_mu);
    for (;;) {
        while (g_generation == seen) pthread_cond_wait(&g_start, &g_mu);
        seen = g_generation;
        pthread_mutex_unlock(&g_mu);
        run_tasks();
        pthread_mutex_lock(&g_mu);
        if (--g_pending == 0) pthread_cond_signal(&g_done);
    }
    return NULL;
}

EXPORT int nc_host_set_threads(int n) {
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    pthread_mutex_lock(&g_mu);
    while (g_spawned < n - 1) {
        pthread_create(&g_workers[g_spawned], NULL, worker, NULL);
        pthread_detach(g_workers[g_spawned]);
        g_spawned++;
    }
    g_threads = n;
    pthread_mutex_unlock(&g_mu);
    return n;
}

EXPORT int nc_host_threads(void) { return g_threads; }

/* Runs fn(ctx, i) for i in [0, n) on g_threads threads; returns when all are done.
 * Spawned workers beyond g_threads - 1 take part too (they only claim tasks),
 * which is harmless: the task count, not the thread count, defines the work. */
void nc_pool_run(task_fn fn, void *ctx, int64_t n) {
    if (g_threads <= 1 || n <= 1) {
        for (int64_t i = 0; i < n; ++i) fn(ctx, i);
        return;
    }
    pthread_mutex_lock(&g_mu);
    g_fn = fn;
    g_ctx = ctx;
    g_n = n;
    atomic_store(&g_next, 0);
    g_pending = g_spawned;
    g_generation++;
    pthread_cond_broadcast(&g_start);
    pthread_mutex_unlock(&g_mu);
    run_tasks();
    pthread_mutex_lock(&g_mu);
    while (g_pending) pthread_cond_wait(&g_done, &g_mu);
    pthread_mutex_unlock(&g_mu);
}

/* -- exact int8 dot products ----------------------------------------------- */

static int32_t dot_scalar(const int8_t *w, const int8_t *x, int64_t k) {
    int32_t acc = 0;
    for (int64_t i = 0; i < k; ++i) acc += (int32_t)w[i] * (int32_t)x[i];
    return acc;
}

__attribute__((target("avx2"))) static int32_t dot_avx2(const int8_t *w, const int8_t *x, int64_t k) {
    __m256i acc = _mm256_setzero_si256();
    int64_t i = 0;
    for (; i + 16 <= k; i += 16) {
        __m256i a = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + i)));
        __m256i b = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(x + i)));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(a, b));
    }
    int32_t lanes[8];
    _mm256_storeu_si256((__m256i *)lanes, acc);
    int32_t sum = 0;
    for (int l = 0; l < 8; ++l) sum += lanes[l];
    return sum + dot_scalar(w + i, x + i, k - i);
}

/* sum x over k bytes, for the +128 correction */
static int32_t sum_bytes(const int8_t *x, int64_t k) {
    int32_t s = 0;
    for (int64_t i = 0; i < k; ++i) s += x[i];
    return s;
}

__attribute__((target("avx2,avxvnni"))) static int32_t dot_avxvnni(const int8_t *w, const int8_t *x, int64_t k,
                                                                   int32_t xsum) {
    const __m256i flip = _mm256_set1_epi8((char)0x80);
    __m256i acc = _mm256_setzero_si256();
    int64_t i = 0;
    for (; i + 32 <= k; i += 32) {
        __m256i a = _mm256_xor_si256(_mm256_loadu_si256((const __m256i *)(w + i)), flip);
        __m256i b = _mm256_loadu_si256((const __m256i *)(x + i));
        acc = _mm256_dpbusd_avx_epi32(acc, a, b);
    }
    int32_t lanes[8];
    _mm256_storeu_si256((__m256i *)lanes, acc);
    int32_t sum = 0;
    for (int l = 0; l < 8; ++l) sum += lanes[l];
    /* (w + 128) * x over the vector part, minus 128 * x over the same part */
    sum -= 128 * (xsum - sum_bytes(x + i, k - i));
    return sum + dot_scalar(w + i, x + i, k - i);
}

__attribute__((target("avx512f,avx512bw,avx512vnni"))) static int32_t dot_avx512vnni(const int8_t *w,
                                                                                      const int8_t *x, int64_t k,
                                                                                      int32_t xsum) {
    const __m512i flip = _mm512_set1_epi8((char)0x80);
    __m512i acc = _mm512_setzero_si512();
    int64_t i = 0;
    for (; i + 64 <= k; i += 64) {
        __m512i a = _mm512_xor_si512(_mm512_loadu_si512((const void *)(w + i)), flip);
        __m512i b = _mm512_loadu_si512((const void *)(x + i));
        acc = _mm512_dpbusd_epi32(acc, a, b);
    }
    int32_t sum = _mm512_reduce_add_epi32(acc);
    sum -= 128 * (xsum - sum_bytes(x + i, k - i));
    return sum + dot_scalar(w + i, x + i, k - i);
}

enum { ISA_SCALAR = 0, ISA_AVX2 = 1, ISA_AVXVNNI = 2, ISA_AVX512VNNI = 3 };
static int g_isa = -1;
static int g_isa_limit = 3;

static int detect_isa(void) {
    __builtin_cpu_init();
    int isa = ISA_SCALAR;
    if (__builtin_cpu_supports("avx2")) isa = ISA_AVX2;
    if (isa == ISA_AVX2 && __builtin_cpu_supports("avxvnni")) isa = ISA_AVXVNNI;
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw")) isa = ISA_AVX512VNNI;
    return isa;
}

/* The ISA the dot products use: 0 scalar, 1 AVX2, 2 AVX-VNNI, 3 AVX-512 VNNI. */
EXPORT int nc_host_isa(void) {
    if (g_isa < 0) g_isa = detect_isa();
    return g_isa < g_isa_limit ? g_isa : g_isa_limit;
}

/* Caps the ISA (for testing every form on one machine); returns the one in use. */
EXPORT int nc_host_limit_isa(int limit) {
    g_isa_limit = limit;
    return nc_host_isa();
}

static int32_t dot(const int8_t *w, const int8_t *x, int64_t k, int32_t xsum, int isa) {
    switch (isa) {
        case ISA_AVX512VNNI: return dot_avx512vnni(w, x, k, xsum);
        case ISA_AVXVNNI: return dot_avxvnni(w, x, k, xsum);
        case ISA_AVX2: return dot_avx2(w, x, k);
        default: return dot_scalar(w, x, k);
    }
}

/* -- the per-token int8 projection ----------------------------------------- */

#define ROW_BLOCK 16

typedef struct {
    float *y;
    int32_t *acc;          /* when set, the raw accumulators instead of y */
    const int8_t *xq;
    const float *xs;
    const int8_t *q;
    const float *ws;
    const float *bias;
    const float *residual;
    const int32_t *xsum;
    int64_t m, n, k;
    int isa;
} gemv_ctx;

static void gemv_task(void *arg, int64_t block) {
    const gemv_ctx *c = (const gemv_ctx *)arg;
    int64_t n0 = block * ROW_BLOCK, n1 = n0 + ROW_BLOCK < c->n ? n0 + ROW_BLOCK : c->n;
    for (int64_t n = n0; n < n1; ++n) {           /* rows outside tokens */
        const int8_t *row = c->q + n * c->k;
        for (int64_t m = 0; m < c->m; ++m) {
            int32_t acc = dot(row, c->xq + m * c->k, c->k, c->xsum[m], c->isa);
            int64_t at = m * c->n + n;
            if (c->acc) {
                c->acc[at] = acc;
                continue;
            }
            float v = ((float)acc * c->xs[m]) * c->ws[n];
            if (c->bias) v = v + c->bias[n];
            if (c->residual) v = c->residual[at] + v;
            c->y[at] = v;
        }
    }
}

static void gemv(float *y, int32_t *acc, const int8_t *xq, const float *xs, const int8_t *q, const float *ws,
                 const float *bias, const float *residual, int64_t m, int64_t n, int64_t k) {
    int32_t stack_sums[64];
    int32_t *xsum = m <= 64 ? stack_sums : (int32_t *)malloc(sizeof(int32_t) * (size_t)m);
    for (int64_t i = 0; i < m; ++i) xsum[i] = sum_bytes(xq + i * k, k);
    gemv_ctx c = {y, acc, xq, xs, q, ws, bias, residual, xsum, m, n, k, nc_host_isa()};
    nc_pool_run(gemv_task, &c, (n + ROW_BLOCK - 1) / ROW_BLOCK);
    if (xsum != stack_sums) free(xsum);
}

/* y[M,N] = ((f32(xq @ q.T) * xs[m]) * ws[n]) (+ bias[n]) (residual[m,n] + ...); y may alias residual. */
EXPORT void nc_host_matmul_i8_token(float *y, const int8_t *xq, const float *xs, const int8_t *q, const float *ws,
                                    const float *bias, const float *residual, int64_t m, int64_t n, int64_t k) {
    gemv(y, NULL, xq, xs, q, ws, bias, residual, m, n, k);
}

EXPORT void nc_host_matmul_i8_token_acc(int32_t *acc, const int8_t *xq, const int8_t *q, int64_t m, int64_t n,
                                        int64_t k) {
    gemv(NULL, acc, xq, NULL, q, NULL, NULL, NULL, m, n, k);
}

static double now(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + (double)t.tv_nsec * 1e-9;
}

/* Seconds for reps passes over `copies` weight copies laid out back to back
 * (q: copies * n * k bytes, ws: copies * n floats), one GEMV per copy. */
EXPORT double nc_host_time_matmul_i8_token(float *y, const int8_t *xq, const float *xs, const int8_t *q,
                                           const float *ws, int64_t m, int64_t n, int64_t k, int64_t copies,
                                           int64_t reps) {
    double t0 = now();
    for (int64_t r = 0; r < reps; ++r)
        for (int64_t c = 0; c < copies; ++c)
            gemv(y, NULL, xq, xs, q + c * n * k, ws + c * n, NULL, NULL, m, n, k);
    return now() - t0;
}

/* Streaming read bandwidth of the host, the reference's bench/probe.c nc_read
 * in spirit: GB/s summing `bytes` of int64 words, split over the pool. */
typedef struct { const int64_t *p; int64_t words; int64_t chunks; int64_t *out; } read_ctx;

static void read_task(void *arg, int64_t i) {
    const read_ctx *c = (const read_ctx *)arg;
    int64_t per = (c->words + c->chunks - 1) / c->chunks, lo = i * per, hi = lo + per < c->words ? lo + per : c->words;
    int64_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int64_t j = lo;
    for (; j + 4 <= hi; j += 4) { s0 += c->p[j]; s1 += c->p[j + 1]; s2 += c->p[j + 2]; s3 += c->p[j + 3]; }
    for (; j < hi; ++j) s0 += c->p[j];
    c->out[i] = s0 + s1 + s2 + s3;
}

EXPORT double nc_host_read_gbps(const void *buf, int64_t bytes, int64_t reps) {
    int64_t chunks = 256, sums[256];
    read_ctx c = {(const int64_t *)buf, bytes / 8, chunks, sums};
    nc_pool_run(read_task, &c, chunks);
    double t0 = now();
    for (int64_t r = 0; r < reps; ++r) nc_pool_run(read_task, &c, chunks);
    double dt = now() - t0;
    volatile int64_t sink = sums[0];
    (void)sink;
    return (double)bytes * (double)reps / dt / 1e9;
}

/* Elementwise transcendental functions, for pinning nc_math.h against the C
 * library the reference calls (codegen_c.py:58): kind 0-2 are nc_expf,
 * nc_sinf, nc_cosf; 3-5 are libm's expf, sinf, cosf. */
EXPORT void nc_host_math(int kind, float *out, const float *in, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x = in[i];
        switch (kind) {
            case 0: out[i] = nc_expf(x); break;
            case 1: out[i] = nc_sinf(x); break;
            case 2: out[i] = nc_cosf(x); break;
            case 3: out[i] = expf(x); break;
            case 4: out[i] = sinf(x); break;
            default: out[i] = cosf(x); break;
        }
    }
}
