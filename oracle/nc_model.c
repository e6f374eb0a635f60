/* Host C restatement of the GPU model kernels, in their exact operation
 * orders, and a whole Qwen2 forward built from them. TEST INFRASTRUCTURE ONLY.
 *
 * Every function here replays one HIP kernel of nanocompile_amd bit for bit
 * (same float32 operations, same order, the same nc_expf/nc_sinf/nc_cosf from
 * nc_math.h), so the GPU can be held to identical logits and tokens. Where a
 * kernel's order differs from the reference's (a tree where the reference sums
 * in index order), the kernel's header says so and the tests bound the
 * difference against the reference's own outputs (tests/golden).
 *
 * The arithmetic follows the reference: rms_norm nn.py:34-38, RoPE nn.py:69-106,
 * softmax nn.py:57-66 with the causal mask nn.py:123-135, silu nn.py:41-54,
 * attention models/qwen2.py:113-155, the model models/qwen2.py:167-224, the
 * LM head as the reference's matmul kernel lower.py:255-269.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

#include "nc_host.h"
#include "../nanocompile_amd/csrc/nc_math.h"

#define EXPORT __attribute__((visibility("default")))
#define THREADS 256

/* -- the row-sum order: 256 virtual threads, butterfly per 64, (w0+w1)+(w2+w3) -- */

static float row_sum_virtual(const float *partial /* [256] */) {
    float w[4];
    for (int g = 0; g < 4; ++g) {
        float v[64], t[64];
        memcpy(v, partial + 64 * g, sizeof v);
        for (int off = 32; off > 0; off >>= 1) {
            for (int i = 0; i < 64; ++i) t[i] = v[i] + v[i ^ off];
            memcpy(v, t, sizeof v);
        }
        w[g] = v[0];
    }
    return (w[0] + w[1]) + (w[2] + w[3]);
}

/* sum of f(row[k]) over k < n in the row-sum order */
static float row_sum_squares(const float *row, int64_t n) {
    float partial[THREADS];
    for (int t = 0; t < THREADS; ++t) {
        float s = 0.0f;
        for (int64_t k = t; k < n; k += THREADS) s = s + row[k] * row[k];
        partial[t] = s;
    }
    return row_sum_virtual(partial);
}

static float row_sum_values(const float *row, int64_t n) {
    float partial[THREADS];
    for (int t = 0; t < THREADS; ++t) {
        float s = 0.0f;
        for (int64_t k = t; k < n; k += THREADS) s = s + row[k];
        partial[t] = s;
    }
    return row_sum_virtual(partial);
}

/* -- rms_norm + per-token quantization ----------------------------------- */

/* max propagating NaN from either side (the reference's reduce_max, fusion.py:603-609) */
static float nan_max(float a, float b) { return (a < b || b != b) ? b : a; }

static void rms_row(float *normed, const float *x, const float *gamma, int64_t k, float eps) {
    const float ss = row_sum_squares(x, k);
    const float rcp = 1.0f / sqrtf(ss / (float)k + eps);
    for (int64_t i = 0; i < k; ++i) normed[i] = (x[i] * rcp) * gamma[i];
}

static float quantize_row(int8_t *xq, const float *x, int64_t k) {
    float mag = 0.0f;
    for (int64_t i = 0; i < k; ++i) mag = nan_max(mag, fabsf(x[i]));
    const float scale = mag <= 0.0f ? 1.0f : mag / 127.0f;
    for (int64_t i = 0; i < k; ++i) {
        float r = roundf(x[i] / scale);
        r = r <= 127.0f ? r : 127.0f;
        r = -127.0f <= r ? r : -127.0f;
        xq[i] = (int8_t)r;
    }
    return scale;
}

EXPORT void nc_host_rms_norm_quant(float *normed, int8_t *xq, float *xs, const float *x, const float *gamma,
                                   int64_t m, int64_t k, float eps) {
    float *tmp = normed ? NULL : (float *)malloc(sizeof(float) * (size_t)k);
    for (int64_t r = 0; r < m; ++r) {
        float *out = normed ? normed + r * k : tmp;
        rms_row(out, x + r * k, gamma, k, eps);
        if (xq) xs[r] = quantize_row(xq + r * k, out, k);
    }
    free(tmp);
}

/* The same rows spread over the host pool, ROWS_A_TASK rows a task (each row is independent, so
 * the bits are the serial function's): the CPU baseline's config 2 with its threads swept. */
#define ROWS_A_TASK 8
typedef struct { float *normed; int8_t *xq; float *xs; const float *x; const float *gamma; int64_t m, k; float eps; } rnq_ctx;

static void rnq_task(void *arg, int64_t t) {
    const rnq_ctx *c = (const rnq_ctx *)arg;
    const int64_t r0 = t * ROWS_A_TASK, n = c->m - r0 < ROWS_A_TASK ? c->m - r0 : ROWS_A_TASK;
    nc_host_rms_norm_quant(c->normed ? c->normed + r0 * c->k : NULL, c->xq + r0 * c->k, c->xs + r0, c->x + r0 * c->k,
                           c->gamma, n, c->k, c->eps);
}

EXPORT void nc_host_rms_norm_quant_pool(float *normed, int8_t *xq, float *xs, const float *x, const float *gamma,
                                        int64_t m, int64_t k, float eps) {
    rnq_ctx c = {normed, xq, xs, x, gamma, m, k, eps};
    nc_pool_run(rnq_task, &c, (m + ROWS_A_TASK - 1) / ROWS_A_TASK);
}

EXPORT void nc_host_quantize_token(int8_t *xq, float *xs, const float *x, int64_t m, int64_t k) {
    for (int64_t r = 0; r < m; ++r) xs[r] = quantize_row(xq + r * k, x + r * k, k);
}

/* -- RoPE, the cache, attention ------------------------------------------ */

static void rope_pair(float x0, float x1, float c, float s, float *y0, float *y1) {
    *y0 = (x0 * c) + ((-x1) * s);
    *y1 = (x1 * c) + (x0 * s);
}

EXPORT void nc_host_rope_append(float *qkv, float *kcache, float *vcache, const float *inv_freq, int64_t m,
                                int64_t heads, int64_t kv, int64_t d, int64_t past, int64_t capacity) {
    const int64_t half = d / 2, width = (heads + 2 * kv) * d;
    for (int64_t i = 0; i < m; ++i) {
        float *row = qkv + i * width;
        const int64_t pos = past + i;
        const float fpos = (float)pos;
        for (int64_t head = 0; head < heads + kv; ++head) {
            float *x = row + head * d;
            for (int64_t j = 0; j < half; ++j) {
                const float ang = fpos * inv_freq[j];
                float y0, y1;
                rope_pair(x[j], x[j + half], nc_cosf(ang), nc_sinf(ang), &y0, &y1);
                if (head < heads) {
                    x[j] = y0;
                    x[j + half] = y1;
                } else {
                    float *kk = kcache + ((head - heads) * capacity + pos) * d;
                    kk[j] = y0;
                    kk[j + half] = y1;
                }
            }
        }
        const float *v = row + (heads + kv) * d;
        for (int64_t u = 0; u < kv * d; ++u) vcache[((u / d) * capacity + pos) * d + u % d] = v[u];
    }
}

/* softmax of e[0..T) in place: max, nc_expf(z - max), the row-sum order, divide */
static void softmax_row(float *e, int64_t T) {
    float m = -INFINITY;
    for (int64_t t = 0; t < T; ++t) m = nan_max(m, e[t]);
    for (int64_t t = 0; t < T; ++t) e[t] = nc_expf(e[t] - m);
    const float sum = row_sum_values(e, T);
    for (int64_t t = 0; t < T; ++t) e[t] = e[t] / sum;
}

typedef struct {
    float *ctx;
    const float *qkv, *kcache, *vcache;
    int64_t m, heads, kv, d, past, capacity;
    float scale;
} attn_ctx;

/* Attention of one query row in the chunked order of the GPU kernels
 * (nanocompile_amd/csrc/nc_attend.h): per chunk of 64 keys the scores as an
 * fmaf chain in order of d, the chunk max, p = exp(s - max), the chunk sum as
 * the wavefront butterfly over 64 lanes (0 past the chunk), o as an fmaf chain
 * in key order; then
 * the chunks combined in order: m = max m_j, w_j = exp(m_j - m),
 * L = sum l_j w_j, O = sum o_j w_j, out = O / L. */
#define CHUNK 64

static float butterfly64(float *v /* [64], destroyed */) {
    float t[64];
    for (int off = 32; off > 0; off >>= 1) {
        for (int i = 0; i < 64; ++i) t[i] = v[i] + v[i ^ off];
        memcpy(v, t, sizeof t);
    }
    return v[0];
}

static void attend_row(float *out, const float *q, const float *K, const float *V, int64_t T, int64_t d,
                       float scale) {
    const int64_t J = (T + CHUNK - 1) / CHUNK;
    float *part = (float *)malloc(sizeof(float) * (size_t)(J * (d + 2)));
    for (int64_t j = 0; j < J; ++j) {
        const int64_t t0 = j * CHUNK, n = T - t0 < CHUNK ? T - t0 : CHUNK;
        float s[CHUNK], p[CHUNK];
        float m = -INFINITY;
        for (int64_t i = 0; i < n; ++i) {
            float acc = 0.0f;
            for (int64_t k = 0; k < d; ++k) acc = fmaf(q[k], K[(t0 + i) * d + k], acc);
            s[i] = (acc * scale) + 0.0f;
            m = nan_max(m, s[i]);
        }
        for (int64_t i = 0; i < CHUNK; ++i) p[i] = i < n ? nc_expf(s[i] - m) : 0.0f;
        float lanes[64];
        memcpy(lanes, p, sizeof lanes);
        float *pj = part + j * (d + 2);
        pj[0] = m;
        pj[1] = butterfly64(lanes);
        for (int64_t k = 0; k < d; ++k) {
            float o = 0.0f;
            for (int64_t i = 0; i < n; ++i) o = fmaf(p[i], V[(t0 + i) * d + k], o);
            pj[2 + k] = o;
        }
    }
    float m = -INFINITY;
    for (int64_t j = 0; j < J; ++j) m = nan_max(m, part[j * (d + 2)]);
    for (int64_t k = 0; k < d; ++k) {
        float L = 0.0f, O = 0.0f;
        for (int64_t j = 0; j < J; ++j) {
            const float *pj = part + j * (d + 2);
            const float w = nc_expf(pj[0] - m);
            L = L + pj[1] * w;
            O = O + pj[2 + k] * w;
        }
        out[k] = O / L;
    }
    free(part);
}

static void attention_task(void *arg, int64_t job) {
    const attn_ctx *a = (const attn_ctx *)arg;
    const int64_t h = job % a->heads, i = job / a->heads, d = a->d;
    const int64_t g = h / (a->heads / a->kv), width = (a->heads + 2 * a->kv) * d;
    const float *q = a->qkv + i * width + h * d;
    const float *K = a->kcache + g * a->capacity * d, *V = a->vcache + g * a->capacity * d;
    attend_row(a->ctx + i * a->heads * d + h * d, q, K, V, a->past + i + 1, d, a->scale);
}

EXPORT void nc_host_attention(float *ctx, const float *qkv, const float *kcache, const float *vcache, int64_t m,
                              int64_t heads, int64_t kv, int64_t d, int64_t past, int64_t capacity, float scale) {
    attn_ctx a = {ctx, qkv, kcache, vcache, m, heads, kv, d, past, capacity, scale};
    nc_pool_run(attention_task, &a, m * heads);
}

EXPORT void nc_host_softmax_causal(float *y, const float *s, int64_t heads, int64_t seq, int64_t past) {
    const int64_t total = past + seq;
    for (int64_t row = 0; row < heads * seq; ++row) {
        const int64_t T = past + row % seq + 1;
        float *out = y + row * total;
        for (int64_t t = 0; t < T; ++t) out[t] = s[row * total + t] + 0.0f;
        softmax_row(out, T);
        for (int64_t t = T; t < total; ++t) out[t] = 0.0f;
    }
}

EXPORT void nc_host_rope(float *y, const float *x, const float *inv_freq, int64_t heads, int64_t seq, int64_t d,
                         int64_t past) {
    const int64_t half = d / 2;
    for (int64_t row = 0; row < heads * seq; ++row) {
        const float fpos = (float)(past + row % seq);
        for (int64_t j = 0; j < half; ++j) {
            const float ang = fpos * inv_freq[j];
            rope_pair(x[row * d + j], x[row * d + j + half], nc_cosf(ang), nc_sinf(ang), &y[row * d + j],
                      &y[row * d + j + half]);
        }
    }
}

/* -- SwiGLU projection pair ------------------------------------------------ */

static float silu_mul(float g, float u) {
    const int p = 0.0f <= g;
    const float e = nc_expf(p ? -g : g);
    const float sig = (p ? 1.0f : e) / (e + 1.0f);
    return (g * sig) * u;
}

EXPORT void nc_host_silu_mul(float *y, const float *g, const float *u, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = silu_mul(g[i], u[i]);
}

EXPORT void nc_host_matmul_i8_token_swiglu(float *h, const int8_t *xq, const float *xs, const int8_t *qg,
                                           const float *sg, const int8_t *qu, const float *su, int64_t m,
                                           int64_t n, int64_t k) {
    float *g = (float *)malloc(sizeof(float) * (size_t)(m * n));
    float *u = (float *)malloc(sizeof(float) * (size_t)(m * n));
    nc_host_matmul_i8_token(g, xq, xs, qg, sg, NULL, NULL, m, n, k);
    nc_host_matmul_i8_token(u, xq, xs, qu, su, NULL, NULL, m, n, k);
    for (int64_t i = 0; i < m * n; ++i) h[i] = silu_mul(g[i], u[i]);
    free(g);
    free(u);
}

/* -- LM head and argmax ----------------------------------------------------- */

/* table8: blocks of 8 rows, [ceil(V/8)][H][8]; each row summed in k order. */
typedef struct { float *logits; const float *x; const float *table8; int64_t v, h, m; } lm_ctx;

#define LM_BLOCKS_PER_TASK 64

__attribute__((target("avx2"))) static void lm_block_avx2(float *out, const float *x, const float *t8, int64_t h) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t k = 0; k < h; ++k)
        acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_set1_ps(x[k]), _mm256_loadu_ps(t8 + k * 8)));
    _mm256_storeu_ps(out, acc);
}

static void lm_block_scalar(float *out, const float *x, const float *t8, int64_t h) {
    float acc[8] = {0};
    for (int64_t k = 0; k < h; ++k)
        for (int j = 0; j < 8; ++j) acc[j] = acc[j] + x[k] * t8[k * 8 + j];
    memcpy(out, acc, sizeof acc);
}

static int g_avx2 = -1;

static void lm_task(void *arg, int64_t task) {
    const lm_ctx *c = (const lm_ctx *)arg;
    const int64_t blocks = (c->v + 7) / 8;
    const int64_t b0 = task * LM_BLOCKS_PER_TASK;
    for (int64_t r = 0; r < c->m; ++r)
        for (int64_t b = b0; b < b0 + LM_BLOCKS_PER_TASK && b < blocks; ++b) {
            float out[8];
            if (g_avx2) lm_block_avx2(out, c->x + r * c->h, c->table8 + b * c->h * 8, c->h);
            else lm_block_scalar(out, c->x + r * c->h, c->table8 + b * c->h * 8, c->h);
            for (int j = 0; j < 8 && b * 8 + j < c->v; ++j) c->logits[r * c->v + b * 8 + j] = out[j];
        }
}

EXPORT void nc_host_lm_head(float *logits, const float *x, const float *table8, int64_t m, int64_t v, int64_t h) {
    if (g_avx2 < 0) {
        __builtin_cpu_init();
        g_avx2 = __builtin_cpu_supports("avx2");
    }
    lm_ctx c = {logits, x, table8, v, h, m};
    const int64_t blocks = (v + 7) / 8;
    nc_pool_run(lm_task, &c, (blocks + LM_BLOCKS_PER_TASK - 1) / LM_BLOCKS_PER_TASK);
}

static int64_t argmax_row(const float *x, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}

/* -- the whole model, int8 projections with per-token activations ------------ */

typedef struct {
    const float *gamma1, *gamma2;
    const int8_t *qkv_q;            /* [(heads + 2 kv) d, H]: q, k, v rows */
    const float *qkv_s, *qkv_b;
    const int8_t *o_q;              /* [H, heads d] */
    const float *o_s;
    const int8_t *g_q, *u_q;        /* [I, H] */
    const float *g_s, *u_s;
    const int8_t *d_q;              /* [H, I] */
    const float *d_s;
} layer_w;

typedef struct {
    int64_t vocab, hidden, inter, layers, heads, kv, d, capacity;
    float eps, scale;
    const float *embed;             /* [V, H] */
    const float *table8;            /* the LM head table in blocks of 8 rows */
    const float *norm;              /* final gamma [H] */
    const float *inv_freq;          /* [d / 2] */
    const layer_w *w;               /* [layers] */
    float *kcache, *vcache;         /* [layers, kv, capacity, d] */
} model_t;

/* One forward over m new tokens at positions past..past+m-1. Writes the last
 * row's logits (or every row's when all_rows) and returns the last row's
 * argmax, or -1 for a token id outside the vocabulary (the gather's Fail). */
EXPORT int64_t nc_host_qwen2_forward(const model_t *mdl, const int64_t *ids, int64_t m, int64_t past, float *logits,
                                     int all_rows) {
    const int64_t H = mdl->hidden, I = mdl->inter, Q = mdl->heads * mdl->d;
    const int64_t W = (mdl->heads + 2 * mdl->kv) * mdl->d;
    if (past + m > mdl->capacity) return -2;
    float *x = malloc(sizeof(float) * m * H), *qkv = malloc(sizeof(float) * m * W);
    float *ctx = malloc(sizeof(float) * m * Q), *h = malloc(sizeof(float) * m * I), *xs = malloc(sizeof(float) * m);
    int8_t *xq = malloc((size_t)(m * (I > H ? I : H)));
    for (int64_t i = 0; i < m; ++i) {
        if (ids[i] < 0 || ids[i] >= mdl->vocab) { m = -1; break; }
        memcpy(x + i * H, mdl->embed + ids[i] * H, sizeof(float) * H);
    }
    int64_t token = -1;
    if (m > 0) {
        const int64_t per_layer = mdl->kv * mdl->capacity * mdl->d;
        for (int64_t l = 0; l < mdl->layers; ++l) {
            const layer_w *w = &mdl->w[l];
            float *kc = mdl->kcache + l * per_layer, *vc = mdl->vcache + l * per_layer;
            nc_host_rms_norm_quant(NULL, xq, xs, x, w->gamma1, m, H, mdl->eps);
            nc_host_matmul_i8_token(qkv, xq, xs, w->qkv_q, w->qkv_s, w->qkv_b, NULL, m, W, H);
            nc_host_rope_append(qkv, kc, vc, mdl->inv_freq, m, mdl->heads, mdl->kv, mdl->d, past, mdl->capacity);
            nc_host_attention(ctx, qkv, kc, vc, m, mdl->heads, mdl->kv, mdl->d, past, mdl->capacity, mdl->scale);
            nc_host_quantize_token(xq, xs, ctx, m, Q);
            nc_host_matmul_i8_token(x, xq, xs, w->o_q, w->o_s, NULL, x, m, H, Q);
            nc_host_rms_norm_quant(NULL, xq, xs, x, w->gamma2, m, H, mdl->eps);
            nc_host_matmul_i8_token_swiglu(h, xq, xs, w->g_q, w->g_s, w->u_q, w->u_s, m, I, H);
            nc_host_quantize_token(xq, xs, h, m, I);
            nc_host_matmul_i8_token(x, xq, xs, w->d_q, w->d_s, NULL, x, m, H, I);
        }
        const int64_t first = all_rows ? 0 : m - 1, rows = all_rows ? m : 1;
        nc_host_rms_norm_quant(ctx, NULL, NULL, x + first * H, mdl->norm, rows, H, mdl->eps);
        nc_host_lm_head(logits, ctx, mdl->table8, rows, mdl->vocab, H);
        token = argmax_row(logits + (rows - 1) * mdl->vocab, mdl->vocab);
    }
    free(x); free(qkv); free(ctx); free(h); free(xs); free(xq);
    return token;
}

EXPORT int64_t nc_host_model_struct_size(void) { return (int64_t)sizeof(model_t); }
EXPORT int64_t nc_host_layer_struct_size(void) { return (int64_t)sizeof(layer_w); }
