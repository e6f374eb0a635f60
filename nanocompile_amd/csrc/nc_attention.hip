// Attention around the int8 projections: RoPE, the KV cache, and grouped-query
// attention with the causal mask, plus the standalone fused groups (softmax
// with the mask, RoPE) the reference emits as single row kernels.
//
// The arithmetic is the reference's (nn.py:57-106, models/qwen2.py:113-155),
// one IEEE float32 operation at a time, with these orders:
//  * RoPE: angle = f32(position) * inv_freq[j mod d/2] (inv_freq computed by
//    the host as the reference does, nn.py:69-75); y = x * cos + rot * sin
//    with rot = [-x[d/2:], x[:d/2]] (nn.py:97-106); cos and sin are
//    nc_cosf / nc_sinf (nc_math.h).
//  * softmax (nc_softmax_causal): m = max z (NaN-propagating, as
//    fusion.py:603-609); e_t = nc_expf(z_t - m); the sum of e_t in the row-sum
//    order of the row kernels (256 virtual threads, thread v adding
//    t = v, v + 256, ... in order; xor butterfly within each 64;
//    (w0 + w1) + (w2 + w3)); p_t = e_t / sum. Masked entries are 0.
//  * attention (nc_attention): scores s_t = sum over d of q[d] * k_t[d] in
//    order of d (the reference's matmul kernel, lower.py:255-269), times
//    scale, + 0 (the mask adds 0 where a key is visible; masked keys are
//    skipped); then the softmax and the context in 64-key chunks combined
//    after, the order nc_attend.h states (shared with the decode kernel).
// The host oracle (oracle/nc_model.c) replays exactly these orders.
#include "nc_common.h"
#include "nc_attend.h"
#include "nc_math.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxKeys = 16384;     // dynamic LDS: one float per visible key

__device__ __forceinline__ float nan_max(float a, float b) { return (a < b || b != b) ? b : a; }

// The row-sum order of every float sum over a row in this library, for a
// value per virtual thread already accumulated in `v` (thread tid holds
// virtual thread tid). Lanes: butterfly; waves: (w0 + w1) + (w2 + w3).
__device__ float row_sum(float v, float *scratch) {
    v = nc::wave_sum_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    const float r = __fadd_rn(__fadd_rn(scratch[0], scratch[1]), __fadd_rn(scratch[2], scratch[3]));
    __syncthreads();
    return r;
}

__device__ float row_max(float v, float *scratch) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    const float r = nan_max(nan_max(scratch[0], scratch[1]), nan_max(scratch[2], scratch[3]));
    __syncthreads();
    return r;
}

// Softmax over e[0..T) in LDS, in place: z -> p, in the stated order.
__device__ void softmax_lds(float *e, int T, float *scratch) {
    float m = -__builtin_inff();
    for (int t = threadIdx.x; t < T; t += kThreads) m = nan_max(m, e[t]);
    m = row_max(m, scratch);
    float partial = 0.0f;
    for (int t = threadIdx.x; t < T; t += kThreads) {
        const float v = nc_expf(__fsub_rn(e[t], m));
        e[t] = v;
        partial = __fadd_rn(partial, v);
    }
    const float sum = row_sum(partial, scratch);
    for (int t = threadIdx.x; t < T; t += kThreads) e[t] = nc::div_rn(e[t], sum);
    __syncthreads();
}

// A position read from the device (a captured decode step): past = *pos_ptr,
// which must leave room for the m new tokens. Every thread of every block
// reads the same word and takes the same branch.
__device__ __forceinline__ bool position_fits(const int64_t *pos_ptr, int m, int capacity, int32_t *error,
                                              int &past) {
    const int64_t p = *pos_ptr;
    if (p < 0 || p + m > capacity) {
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_CAPACITY);
        return false;
    }
    past = (int)p;
    return true;
}

__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float &y0, float &y1) {
    // y[j] = x[j] * c + (-x[j + h]) * s;  y[j + h] = x[j + h] * c + x[j] * s
    y0 = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
    y1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
}

// qkv[M, (H + 2 * KV * D)] rows: q heads rotated in place; k heads rotated and
// written with v into the cache at positions past + i.
__global__ __launch_bounds__(kThreads) void rope_append(float *__restrict__ qkv, float *__restrict__ kcache,
                                                        float *__restrict__ vcache,
                                                        const float *__restrict__ inv_freq, int heads, int kv_heads,
                                                        int D, int past, int capacity,
                                                        const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error) {
    if (pos_ptr && !position_fits(pos_ptr, (int)gridDim.x, capacity, error, past)) return;
    const int i = blockIdx.x;
    const int half = D / 2;
    const int width = (heads + 2 * kv_heads) * D;
    float *row = qkv + (size_t)i * width;
    const int pos = past + i;
    const float fpos = (float)pos;
    const int pairs = (heads + kv_heads) * half;
    for (int u = threadIdx.x; u < pairs; u += kThreads) {
        const int head = u / half, j = u - head * half;
        const float ang = __fmul_rn(fpos, inv_freq[j]);
        const float c = nc_cosf(ang), s = nc_sinf(ang);
        float *x = row + head * D;
        float y0, y1;
        rope_pair(x[j], x[j + half], c, s, y0, y1);
        if (head < heads) {
            x[j] = y0;
            x[j + half] = y1;
        } else {
            float *k = kcache + ((size_t)(head - heads) * capacity + pos) * D;
            k[j] = y0;
            k[j + half] = y1;
        }
    }
    const float *v = row + (heads + kv_heads) * D;
    for (int u = threadIdx.x; u < kv_heads * D; u += kThreads) {
        const int g = u / D, d = u - g * D;
        vcache[((size_t)g * capacity + pos) * D + d] = v[u];
    }
}

// One query row of one head: grid (heads, M). Query row i sits at position
// past + i and sees keys 0 .. past + i of its KV head (h / group). The four
// waves take the 64-key chunks in turn (nc_attend.h gives the order), leave
// their partials in LDS, and wave 0 combines them: the same bits as the
// decode kernel's split over workgroups.
template <int D>
__global__ __launch_bounds__(kThreads) void attention_rows(float *__restrict__ ctx, const float *__restrict__ qkv,
                                                           const float *__restrict__ kcache,
                                                           const float *__restrict__ vcache, int heads,
                                                           int kv_heads, int past, int capacity, float scale,
                                                           const int64_t *__restrict__ pos_ptr,
                                                           int32_t *__restrict__ error) {
    if (pos_ptr && !position_fits(pos_ptr, (int)gridDim.y, capacity, error, past)) return;
    extern __shared__ __align__(16) float lds[];  // [4 waves][chunk stage], then [J][D + 2]: m_j, l_j, o_j[D]
    float *stage = lds + (threadIdx.x >> 6) * nc::chunk_stage_floats<D>();
    float *part = lds + (kThreads / 64) * nc::chunk_stage_floats<D>();
    __shared__ __align__(16) float q[D];
    const int h = blockIdx.x, i = blockIdx.y;
    const int g = h / (heads / kv_heads);
    const int width = (heads + 2 * kv_heads) * D;
    const int T = past + i + 1, J = (T + nc::kChunk - 1) / nc::kChunk;
    if (threadIdx.x < D) q[threadIdx.x] = qkv[(size_t)i * width + h * D + threadIdx.x];
    __syncthreads();

    const float *K = kcache + (size_t)g * capacity * D;
    const float *V = vcache + (size_t)g * capacity * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int j = wave; j < J; j += kThreads / 64) {
        const int t0 = j * nc::kChunk;
        nc::Chunk<D, false> chunk(K, V, t0, min(nc::kChunk, T - t0), -1, capacity - 1);
        const nc::ChunkResult r = chunk.attend(q, nullptr, nullptr, scale, stage);
        float *pj = part + j * (D + 2);
        if (lane == 0) {
            pj[0] = r.m;
            pj[1] = r.l;
        }
        if (lane < D) pj[2 + lane] = r.o;
    }
    __syncthreads();
    if (wave == 0) {
        const float out = nc::combine_chunks(J, lane < D ? lane : 0,
                                             [&](int c, int k) { return part[c * (D + 2) + k]; });
        if (lane < D) ctx[(size_t)i * heads * D + h * D + lane] = out;
    }
}

// softmax(s + causal mask) over rows of s[heads, seq, past + seq]
// (models/qwen2.py:150-151, nn.py:57-66, 123-135): masked entries are 0.
__global__ __launch_bounds__(kThreads) void softmax_causal(float *__restrict__ y, const float *__restrict__ s,
                                                           int seq, int past) {
    extern __shared__ float e[];
    __shared__ float scratch[4];
    const int row = blockIdx.x;               // over heads * seq
    const int i = row % seq;
    const int total = past + seq, T = past + i + 1;
    const float *in = s + (size_t)row * total;
    for (int t = threadIdx.x; t < T; t += kThreads) e[t] = __fadd_rn(in[t], 0.0f);
    __syncthreads();
    softmax_lds(e, T, scratch);
    float *out = y + (size_t)row * total;
    for (int t = threadIdx.x; t < total; t += kThreads) out[t] = t < T ? e[t] : 0.0f;
}

// apply_rope on x[heads, seq, D] at positions past .. past + seq - 1.
__global__ __launch_bounds__(kThreads) void rope_rows(float *__restrict__ y, const float *__restrict__ x,
                                                      const float *__restrict__ inv_freq, int seq, int D, int past) {
    const int row = blockIdx.x;               // over heads * seq
    const int half = D / 2;
    const float fpos = (float)(past + row % seq);
    const float *in = x + (size_t)row * D;
    float *out = y + (size_t)row * D;
    for (int j = threadIdx.x; j < half; j += kThreads) {
        const float ang = __fmul_rn(fpos, inv_freq[j]);
        float y0, y1;
        rope_pair(in[j], in[j + half], nc_cosf(ang), nc_sinf(ang), y0, y1);
        out[j] = y0;
        out[j + half] = y1;
    }
}

float bits_to_float(int64_t bits) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)bits;
    return c.f;
}

}  // namespace

// p: [qkv f32[M, (H + 2*KV*D)] (q rotated in place), kcache f32[KV, C, D], vcache f32[KV, C, D],
//     inv_freq f32[D/2], pos i64[1] | NULL];  s: [M, heads, kv_heads, D, past, capacity]
// With pos, past is read from the device when the kernel runs (s[4] is ignored).
NC_EXPORT int32_t nc_rope_append(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3], "nc_rope_append: null operand");
    const int64_t M = s[0], heads = s[1], kv = s[2], D = s[3], past = s[4], cap = s[5];
    const int64_t *pos = (const int64_t *)p[4];
    NC_REQUIRE(M >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && D > 0 && D % 2 == 0 && D <= 64 &&
                   (pos || (past >= 0 && past + M <= cap)) && M <= cap && cap < (1 << 24) && M < (1 << 24),
               "nc_rope_append: bad shape or the cache is full");
    if (M == 0) return NC_OK;
    hipLaunchKernelGGL(rope_append, dim3((unsigned)M), dim3(kThreads), 0, nc::stream(), (float *)p[0],
                       (float *)p[1], (float *)p[2], (const float *)p[3], (int)heads, (int)kv, (int)D,
                       pos ? 0 : (int)past, (int)cap, pos, nc::error_word());
    return nc::launched("rope_append");
}

namespace {

template <int D>
int32_t launch_rows(void **p, int64_t M, int64_t heads, int64_t kv, int64_t past, int64_t cap, float scale,
                    const int64_t *pos) {
    // the waves' chunk stages (70 KB) and the partials of every chunk (up to
    // 256 chunks x 66 floats = 67.6 KB at 16384 keys): past the 64 KB a
    // launch gets without asking
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attention_rows<D>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024) != hipSuccess) {
            nc::set_message("nc_attention: could not raise the LDS limit");
            return NC_LAUNCH_FAILED;
        }
        raised = true;
    }
    const int64_t keys = pos ? cap : past + M;
    const size_t lds = ((size_t)(kThreads / 64) * nc::chunk_stage_floats<D>() +
                        (size_t)((keys + nc::kChunk - 1) / nc::kChunk) * (D + 2)) * sizeof(float);
    hipLaunchKernelGGL(attention_rows<D>, dim3((unsigned)heads, (unsigned)M), dim3(kThreads), lds, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const float *)p[2], (const float *)p[3], (int)heads,
                       (int)kv, pos ? 0 : (int)past, (int)cap, scale, pos, nc::error_word());
    return nc::launched("attention_rows");
}

}  // namespace

// p: [ctx f32[M, heads*D], qkv f32[M, (H + 2*KV*D)] (q rotated), kcache, vcache, pos i64[1] | NULL];
// s: [M, heads, kv_heads, D, past, capacity, scale as float32 bits]  (D 16, 32 or 64)
// With pos, past is read from the device when the kernel runs (s[4] is ignored).
NC_EXPORT int32_t nc_attention(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3], "nc_attention: null operand");
    const int64_t M = s[0], heads = s[1], kv = s[2], D = s[3], past = s[4], cap = s[5];
    const int64_t *pos = (const int64_t *)p[4];
    NC_REQUIRE(M >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && (D == 16 || D == 32 || D == 64) &&
                   (pos ? cap <= kMaxKeys : (past >= 0 && past + M <= cap && past + M <= kMaxKeys)) &&
                   M <= cap && M < 65536 && heads < 65536,
               "nc_attention: bad shape (head_dim 16, 32 or 64; at most 16384 keys)");
    if (M == 0) return NC_OK;
    const float scale = bits_to_float(s[6]);
    if (D == 64) return launch_rows<64>(p, M, heads, kv, past, cap, scale, pos);
    if (D == 32) return launch_rows<32>(p, M, heads, kv, past, cap, scale, pos);
    return launch_rows<16>(p, M, heads, kv, past, cap, scale, pos);
}


// p: [y f32[heads, seq, past+seq], s f32[heads, seq, past+seq]];  s: [heads, seq, past]
NC_EXPORT int32_t nc_softmax_causal(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1], "nc_softmax_causal: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] >= 0 && s[2] >= 0 && s[1] + s[2] <= kMaxKeys && s[0] * s[1] < (1 << 30),
               "nc_softmax_causal: bad shape");
    if (s[0] * s[1] == 0) return NC_OK;
    const size_t lds = (size_t)(s[1] + s[2]) * sizeof(float);
    hipLaunchKernelGGL(softmax_causal, dim3((unsigned)(s[0] * s[1])), dim3(kThreads), lds, nc::stream(),
                       (float *)p[0], (const float *)p[1], (int)s[1], (int)s[2]);
    return nc::launched("softmax_causal");
}

// p: [y f32[heads, seq, D], x f32[heads, seq, D], inv_freq f32[D/2]];  s: [heads, seq, D, past]
NC_EXPORT int32_t nc_rope(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_rope: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] >= 0 && s[2] > 0 && s[2] % 2 == 0 && s[3] >= 0 && s[3] + s[1] < (1 << 24) &&
                   s[0] * s[1] < (1 << 30),
               "nc_rope: bad shape");
    if (s[0] * s[1] == 0) return NC_OK;
    hipLaunchKernelGGL(rope_rows, dim3((unsigned)(s[0] * s[1])), dim3(kThreads), 0, nc::stream(), (float *)p[0],
                       (const float *)p[1], (const float *)p[2], (int)s[1], (int)s[2], (int)s[3]);
    return nc::launched("rope_rows");
}

namespace {
// cos and sin of f32(position) * inv_freq[i] for every position of a cache:
// RoPE's angles (nn.py:78-94, the reference's rope_tables) computed once with
// the same nc_cosf / nc_sinf the kernels use, so a table lookup gives the same
// bits as computing them in place.
__global__ __launch_bounds__(kThreads) void rope_table(float *__restrict__ table, const float *__restrict__ inv_freq,
                                                       int capacity, int half) {
    const int64_t n = (int64_t)capacity * half;
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= n) return;
    const int pos = (int)(u / half), i = (int)(u - (int64_t)pos * half);
    const float ang = __fmul_rn((float)pos, inv_freq[i]);
    table[u] = nc_cosf(ang);
    table[n + u] = nc_sinf(ang);
}
}  // namespace

// p: [table f32[2, C, D/2] (cos, then sin), inv_freq f32[D/2]];  s: [C, D]
NC_EXPORT int32_t nc_rope_table(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1], "nc_rope_table: null operand");
    NC_REQUIRE(s[0] > 0 && s[0] < (1 << 24) && s[1] > 0 && s[1] % 2 == 0 && s[1] <= 1024,
               "nc_rope_table: bad shape");
    const int64_t n = s[0] * (s[1] / 2);
    hipLaunchKernelGGL(rope_table, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (int)s[0], (int)(s[1] / 2));
    return nc::launched("rope_table");
}
