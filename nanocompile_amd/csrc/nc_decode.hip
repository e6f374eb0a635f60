// Decode-step kernels (one new token): each projection with its activation
// prologue fused in, and attention with RoPE and the cache append fused in.
//
// A decode step is latency-bound: each projection streams 0.1-4.4 MB, a few
// microseconds at HBM speed, so every separate small kernel (an rms_norm, a
// quantizer) costs as much as a projection. Here each workgroup of a
// projection recomputes its activation row itself (3.5 KB or 19 KB, read from
// L2) and quantizes it into LDS, then streams its 8 weight rows:
//
//   qkv:     rms_norm(x) -> int8 -> q,k,v rows + bias
//   o:       int8(ctx)          -> rows, residual x + y written in place
//   gate/up: rms_norm(x) -> int8 -> pairs of rows -> silu(gate) * up
//   down:    int8(h)            -> rows, residual x + y written in place
//
// The arithmetic and its order are exactly those of the unfused kernels
// (nc_quant.hip, nc_gemv.hip, nc_attention.hip): rms_norm's sum of squares in
// the 256-virtual-thread row-sum order, lane l of the one wave holding virtual
// threads l, l + 64, l + 128, l + 192; maxima exact; the same epilogues. So a
// fused step computes the same bits as the unfused one, and the host oracle
// covers both.
#include "nc_common.h"
#include "nc_epilogue.h"

namespace {

using nc::i8x16;
constexpr int kL = 8;                  // lanes per weight row: 8 x 16 B = one 128-byte line per load
constexpr int kRows = 64 / kL;         // weight rows per one-wave workgroup

enum Prologue { kNorm = 0, kQuant = 1 };
enum Epilogue { kBias = 0, kResidual = 1, kSwiglu = 2 };

// The activation row x[K] (f32) to int8 in LDS; returns its scale. NORM
// applies rms_norm first (rms_norm(x) * gamma, eps).
template <int K, int PRO>
__device__ float activation_prologue(int8_t *__restrict__ sxq, const float *__restrict__ x,
                                     const float *__restrict__ gamma, float eps) {
    constexpr int PER = (K + 63) / 64;
    const int lane = threadIdx.x;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int k = lane + 64 * i;
        v[i] = (K % 64 == 0 || k < K) ? x[k] : 0.0f;
    }
    if constexpr (PRO == kNorm) {
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};      // virtual threads lane + 64 g, g = 0..3
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = lane + 64 * i;
            if (K % 64 == 0 || k < K) s[i & 3] = __fadd_rn(s[i & 3], __fmul_rn(v[i], v[i]));
        }
        float w[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) w[g] = nc::wave_sum_f32(s[g]);
        const float ss = __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
        const float rcp = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = lane + 64 * i;
            if (K % 64 == 0 || k < K) v[i] = __fmul_rn(__fmul_rn(v[i], rcp), gamma[k]);
        }
    }
    float mag = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) mag = fmaxf(mag, fabsf(v[i]));
    const float scale = nc::token_scale(nc::wave_max_f32(mag));
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int k = lane + 64 * i;
        if (K % 64 == 0 || k < K) sxq[k] = nc::quantize_value(v[i], scale);
    }
    __syncthreads();
    return scale;
}

template <int K>
struct RowChunks {
    static constexpr int STEP = kL * 16;
    static constexpr int ITERS = K / STEP;
    static_assert(K % STEP == 0, "K must be a multiple of 128");
    i8x16 w[ITERS];

    // The lane's 16-byte chunks of its weight row, loads issued back to back.
    __device__ __forceinline__ void load(const int8_t *__restrict__ row, int sub) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) w[it] = nc::load16_stream(row + it * STEP + sub * 16);
    }

    __device__ __forceinline__ int32_t dot(const int8_t *__restrict__ sxq, int sub) const {
        int32_t acc = 0;
#pragma unroll
        for (int it = 0; it < ITERS; ++it)
            acc = nc::dot16(w[it], *reinterpret_cast<const i8x16 *>(sxq + it * STEP + sub * 16), acc);
        return acc;
    }
};

// One decode projection: workgroup = one wave = 8 rows (8 row pairs for SwiGLU).
// The weight loads are issued first, so they are in flight while the
// workgroup computes its activation prologue.
template <int K, int PRO, int EPI>
__global__ __launch_bounds__(64) void gemv_decode(float *__restrict__ out, const float *__restrict__ x,
                                                  const float *__restrict__ gamma, float eps,
                                                  const int8_t *__restrict__ q, const float *__restrict__ ws,
                                                  const float *__restrict__ bias, const int8_t *__restrict__ q2,
                                                  const float *__restrict__ ws2, int N) {
    __shared__ __align__(16) int8_t sxq[K];
    const int lane = threadIdx.x, sub = lane & (kL - 1);
    const int n = blockIdx.x * kRows + lane / kL;
    const bool valid = n < N;
    const int nr = valid ? n : 0;
    RowChunks<K> w1, w2;
    w1.load(q + (size_t)nr * K, sub);
    if constexpr (EPI == kSwiglu) w2.load(q2 + (size_t)nr * K, sub);
    const float xs = activation_prologue<K, PRO>(sxq, x, gamma, eps);
    int32_t acc = w1.dot(sxq, sub);
    int32_t acc2 = 0;
    if constexpr (EPI == kSwiglu) acc2 = w2.dot(sxq, sub);
    acc = nc::group_sum_i32<kL>(acc);
    if constexpr (EPI == kSwiglu) acc2 = nc::group_sum_i32<kL>(acc2);
    if (sub != 0 || !valid) return;
    const float y = __fmul_rn(__fmul_rn((float)acc, xs), ws[n]);
    if constexpr (EPI == kBias) {
        out[n] = __fadd_rn(y, bias[n]);
    } else if constexpr (EPI == kResidual) {
        out[n] = __fadd_rn(out[n], y);                     // out is the residual stream, updated in place
    } else {
        const float u = __fmul_rn(__fmul_rn((float)acc2, xs), ws2[n]);
        out[n] = nc::silu_mul(y, u);
    }
}

// -- attention for one new token, RoPE and the cache append fused in ---------------

constexpr int kT = 256;

__device__ __forceinline__ float nan_max(float a, float b) { return (a < b || b != b) ? b : a; }

__device__ float block_sum(float v, float *scratch) {
    v = nc::wave_sum_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    const float r = __fadd_rn(__fadd_rn(scratch[0], scratch[1]), __fadd_rn(scratch[2], scratch[3]));
    __syncthreads();
    return r;
}

__device__ float block_max(float v, float *scratch) {
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

// One key row held in registers: D/4 float4, dotted with q in order of d.
template <int D>
struct KeyRow {
    float4 v[D / 4];
    __device__ __forceinline__ void load(const float *__restrict__ row) {
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) v[d4] = reinterpret_cast<const float4 *>(row)[d4];
    }
    __device__ __forceinline__ void load_lds(const float *row) {
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) v[d4] = reinterpret_cast<const float4 *>(row)[d4];
    }
    __device__ __forceinline__ float score(const float *q, float scale) const {
        float acc = 0.0f;
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            acc = __fadd_rn(acc, __fmul_rn(q[4 * d4 + 0], v[d4].x));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * d4 + 1], v[d4].y));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * d4 + 2], v[d4].z));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * d4 + 3], v[d4].w));
        }
        return __fadd_rn(__fmul_rn(acc, scale), 0.0f);
    }
};

// Head h of the new token at position past (read from pos_ptr when given).
// q and the new k are rotated here (the same nc_cosf/nc_sinf of
// f32(past) * inv_freq[j] as nc_rope_append); the first query head of each KV
// group writes the new k and v into the cache; every head reads the new key
// and value from its own LDS copy, so no head waits on another's write.
template <int D>
__global__ __launch_bounds__(kT) void attention_decode(float *__restrict__ ctx, const float *__restrict__ qkv,
                                                       float *__restrict__ kcache, float *__restrict__ vcache,
                                                       const float *__restrict__ inv_freq, int heads, int kv_heads,
                                                       int past, int capacity, float scale,
                                                       const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error) {
    if (pos_ptr) {
        const int64_t p = *pos_ptr;
        if (p < 0 || p + 1 > capacity) {
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_CAPACITY);
            return;
        }
        past = (int)p;
    }
    extern __shared__ float e[];
    __shared__ __align__(16) float q[D];
    __shared__ __align__(16) float knew[D];
    __shared__ __align__(16) float vnew[D];
    __shared__ float part[4][D];
    __shared__ float scratch[4];
    constexpr int half = D / 2;
    const int h = blockIdx.x, group = heads / kv_heads, g = h / group;
    const int tid = threadIdx.x;
    const float *qrow = qkv + h * D;
    const float *krow = qkv + heads * D + g * D;
    const float *vrow = qkv + (heads + kv_heads) * D + g * D;
    const float fpos = (float)past;
    const int T = past + 1;
    const int lane = tid & 63, wave = tid >> 6;
    const int S = (T + 3) / 4;
    const int t0 = wave * S, t1 = min(T, t0 + S);
    float *K = kcache + (size_t)g * capacity * D;
    float *V = vcache + (size_t)g * capacity * D;

    // Cache reads go out first, all at once and without branches, so their
    // latency overlaps the RoPE and each other: the key rows this thread scores
    // (positions tid and tid + 256) and the first VP values of its wave's chunk
    // for P.V. Addresses are clamped into the cache and unused values replaced
    // by selection, never by guarding a load.
    constexpr int VP = 32;
    KeyRow<D> kreg;
    kreg.load(K + (size_t)(tid < past ? tid : 0) * D);
    const int dl = lane < D ? lane : 0;
    float vreg[VP];
#pragma unroll
    for (int j = 0; j < VP; ++j) {
        const int t = t0 + j;
        vreg[j] = V[(size_t)(t < past ? t : 0) * D + dl];
    }

    if (tid < half) {
        const float ang = __fmul_rn(fpos, inv_freq[tid]);
        const float c = nc_cosf(ang), s = nc_sinf(ang);
        const float x0 = qrow[tid], x1 = qrow[tid + half];
        q[tid] = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
        q[tid + half] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
    } else if (tid < 2 * half) {
        const int j = tid - half;
        const float ang = __fmul_rn(fpos, inv_freq[j]);
        const float c = nc_cosf(ang), s = nc_sinf(ang);
        const float x0 = krow[j], x1 = krow[j + half];
        knew[j] = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
        knew[j + half] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
    } else if (tid < 2 * D) {
        const int d = tid - D;
        vnew[d] = vrow[d];
    }
    __syncthreads();
    if (h % group == 0 && tid < D) {
        K[(size_t)past * D + tid] = knew[tid];
        V[(size_t)past * D + tid] = vnew[tid];
    }

    // scores: q . k in order of d; the new key (position past) from LDS
    if (tid == past) kreg.load_lds(knew);
    if (tid < T) e[tid] = kreg.score(q, scale);
    for (int t = tid + kT; t < T; t += kT) {              // contexts beyond 256 keys
        KeyRow<D> k;
        if (t == past) k.load_lds(knew);
        else k.load(K + (size_t)t * D);
        e[t] = k.score(q, scale);
    }
    __syncthreads();
    float m = -__builtin_inff();
    for (int t = tid; t < T; t += kT) m = nan_max(m, e[t]);
    m = block_max(m, scratch);
    float partial = 0.0f;
    for (int t = tid; t < T; t += kT) {
        const float v = nc_expf(__fsub_rn(e[t], m));
        e[t] = v;
        partial = __fadd_rn(partial, v);
    }
    const float sum = block_sum(partial, scratch);
    for (int t = tid; t < T; t += kT) e[t] = nc::div_rn(e[t], sum);
    __syncthreads();

    // P.V over the wave's chunk in position order. A position past the chunk
    // contributes 0 * 0 = +0, and the accumulator (from +0, adding products)
    // is never -0, so that addition is exact and changes nothing.
    const float vfresh = vnew[dl];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < VP; ++j) {
        const int t = t0 + j;
        const bool in = t < t1;
        const float p = in ? e[in ? t : 0] : 0.0f;
        const float v = in ? (t == past ? vfresh : vreg[j]) : 0.0f;
        acc = __fadd_rn(acc, __fmul_rn(p, v));
    }
    constexpr int TILE = 32;
    for (int t = t0 + VP; t < t1; t += TILE) {
        float vv[TILE];
#pragma unroll
        for (int j = 0; j < TILE; ++j) {
            const int tj = t + j;
            vv[j] = V[(size_t)(tj < past ? tj : 0) * D + dl];
        }
#pragma unroll
        for (int j = 0; j < TILE; ++j) {
            const int tj = t + j;
            const bool in = tj < t1;
            const float p = in ? e[in ? tj : 0] : 0.0f;
            const float v = in ? (tj == past ? vfresh : vv[j]) : 0.0f;
            acc = __fadd_rn(acc, __fmul_rn(p, v));
        }
    }
    if (lane < D) part[wave][lane] = acc;
    __syncthreads();
    if (tid < D) ctx[h * D + tid] = __fadd_rn(__fadd_rn(part[0][tid], part[1][tid]), __fadd_rn(part[2][tid], part[3][tid]));
}

float bits_to_float(int64_t bits) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)bits;
    return c.f;
}

template <int K, int PRO, int EPI>
int32_t launch_decode(void **p, int N, float eps) {
    hipLaunchKernelGGL((gemv_decode<K, PRO, EPI>), dim3((N + kRows - 1) / kRows), dim3(64), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const float *)p[2], eps, (const int8_t *)p[3],
                       (const float *)p[4], (const float *)p[5], (const int8_t *)p[6], (const float *)p[7], N);
    return nc::launched("gemv_decode");
}

}  // namespace

// One decode projection with its activation prologue (see the file header).
// p: [out f32[N] (in: the residual for kind 1), x f32[K], gamma f32[K] | NULL,
//     q i8[N,K], scales f32[N], bias f32[N] | NULL, q2 i8[N,K] | NULL, scales2 f32[N] | NULL];
// s: [N, K, kind, eps as float32 bits] with kind 0 = rms_norm prologue + bias (q, k, v),
//    1 = quantize prologue + residual (o, down), 2 = rms_norm prologue + SwiGLU pair (gate, up).
//    K is 896 or 4864 (the model's widths; any other K uses the unfused kernels).
NC_EXPORT int32_t nc_decode_projection(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[3] && p[4], "nc_decode_projection: null operand");
    const int64_t N = s[0], K = s[1], kind = s[2];
    const float eps = bits_to_float(s[3]);
    NC_REQUIRE(N > 0 && N < (1 << 24) && kind >= 0 && kind <= 2, "nc_decode_projection: bad shape");
    NC_REQUIRE(kind == 1 || p[2], "nc_decode_projection: rms_norm needs gamma");
    NC_REQUIRE(kind != 0 || p[5], "nc_decode_projection: q, k, v need their bias");
    NC_REQUIRE(kind != 2 || (p[6] && p[7]), "nc_decode_projection: SwiGLU needs the up projection");
    if (K == 896 && kind == 0) return launch_decode<896, kNorm, kBias>(p, (int)N, eps);
    if (K == 896 && kind == 1) return launch_decode<896, kQuant, kResidual>(p, (int)N, eps);
    if (K == 896 && kind == 2) return launch_decode<896, kNorm, kSwiglu>(p, (int)N, eps);
    if (K == 4864 && kind == 1) return launch_decode<4864, kQuant, kResidual>(p, (int)N, eps);
    // the test model's widths (hidden 128, MLP 256)
    if (K == 128 && kind == 0) return launch_decode<128, kNorm, kBias>(p, (int)N, eps);
    if (K == 128 && kind == 1) return launch_decode<128, kQuant, kResidual>(p, (int)N, eps);
    if (K == 128 && kind == 2) return launch_decode<128, kNorm, kSwiglu>(p, (int)N, eps);
    if (K == 256 && kind == 1) return launch_decode<256, kQuant, kResidual>(p, (int)N, eps);
    nc::set_message("nc_decode_projection: no fused kernel for this width and kind");
    return NC_BAD_ARGS;
}

// Attention of one new token with RoPE and the cache append fused in.
// p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated, with bias), kcache f32[kv,C,D],
//     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] | NULL];
// s: [heads, kv, D, past, C, scale as float32 bits]  (D = 64; past read from pos when given)
NC_EXPORT int32_t nc_attention_decode(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_attention_decode: null operand");
    const int64_t heads = s[0], kv = s[1], D = s[2], past = s[3], cap = s[4];
    const int64_t *pos = (const int64_t *)p[5];
    NC_REQUIRE(heads > 0 && kv > 0 && heads % kv == 0 && heads < 65536 && (D == 64 || D == 32) && cap > 0 &&
                   cap <= 16384 && (pos || (past >= 0 && past + 1 <= cap)),
               "nc_attention_decode: bad shape (head_dim 64 or 32, capacity at most 16384)");
    auto kernel = D == 64 ? attention_decode<64> : attention_decode<32>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)heads), dim3(kT), (size_t)cap * sizeof(float), nc::stream(),
                       (float *)p[0], (const float *)p[1], (float *)p[2], (float *)p[3], (const float *)p[4],
                       (int)heads, (int)kv, pos ? 0 : (int)past, (int)cap, bits_to_float(s[5]), pos,
                       nc::error_word());
    return nc::launched("attention_decode");
}
