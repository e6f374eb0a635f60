// Row kernels that produce int8: the per-row weight quantizer, the per-token
// activation quantizer, and rms_norm fused with the activation quantizer.
//
// One workgroup of 256 threads per row. Maxima are exact in any order. The
// one float sum here (rms_norm's sum of squares) has this order, which the
// host oracle replays bit for bit:
//   thread t: s_t = x[t]^2 + x[t+256]^2 + ... in index order, from 0;
//   wave w:   the butterfly of nc::wave_sum_f32 over its 64 threads;
//   block:    (w0 + w1) + (w2 + w3).
// The reference sums the row in index order (fusion.py:631-650); the two
// orders agree to float rounding, which the tests bound.
#include "nc_common.h"

namespace {

constexpr int kThreads = 256;

// The workgroup's maximum and sum through four LDS words. Each scratch array
// serves one reduction of a launch (every kernel here takes one row a
// workgroup), so no barrier is needed before it is written.
__device__ float block_max(float v, float *scratch) {
    v = nc::wave_max_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    return nc::nan_max(nc::nan_max(scratch[0], scratch[1]), nc::nan_max(scratch[2], scratch[3]));
}

__device__ float block_sum(float v, float *scratch) {
    v = nc::wave_sum_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    return __fadd_rn(__fadd_rn(scratch[0], scratch[1]), __fadd_rn(scratch[2], scratch[3]));
}

// quantize.py:55-70, operation for operation, in float32:
//   scale = max|row| / 127 (1 for an all-zero row); s = w / scale;
//   q = clip(sign(s) * floor(|s| + 0.5), -127, 127).
__global__ __launch_bounds__(kThreads) void quantize_rows(int8_t *__restrict__ q, float *__restrict__ scales,
                                                          const float *__restrict__ w, int K) {
    __shared__ float scratch[4];
    const float *row = w + (size_t)blockIdx.x * K;
    float mag = 0.0f;
    for (int k = threadIdx.x; k < K; k += kThreads) mag = nc::nan_max(mag, fabsf(row[k]));
    mag = block_max(mag, scratch);
    float scale = nc::div_rn(mag, 127.0f);
    if (scale == 0.0f) scale = 1.0f;
    int8_t *out = q + (size_t)blockIdx.x * K;
    for (int k = threadIdx.x; k < K; k += kThreads) {
        const float s = nc::div_rn(row[k], scale);
        const float r = floorf(__fadd_rn(fabsf(s), 0.5f));
        float v = s > 0.0f ? r : (s < 0.0f ? -r : 0.0f);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        out[k] = (int8_t)v;
    }
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

// Per-token quantization of one row per workgroup: the row read once into
// registers, PER_THREAD values a thread with every load in flight at once (a
// loop over a run-time K waits for each load before the next), its maximum,
// then the int8 values. Rows wider than 32 * kThreads take the loop.
template <int PER_THREAD>
__global__ __launch_bounds__(kThreads) void quantize_token(int8_t *__restrict__ xq, float *__restrict__ xs,
                                                           const float *__restrict__ x, int K) {
    __shared__ float scratch[4];
    const float *row = x + (size_t)blockIdx.x * K;
    int8_t *out = xq + (size_t)blockIdx.x * K;
    float mag = 0.0f;
    if constexpr (PER_THREAD > 0) {
        float v[PER_THREAD];
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int k = threadIdx.x + i * kThreads;
            v[i] = k < K ? row[k] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) mag = nc::nan_max(mag, fabsf(v[i]));
        const float scale = nc::token_scale(block_max(mag, scratch));
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int k = threadIdx.x + i * kThreads;
            if (k < K) out[k] = nc::quantize_value(v[i], scale);
        }
        if (threadIdx.x == 0) xs[blockIdx.x] = scale;
    } else {
        for (int k = threadIdx.x; k < K; k += kThreads) mag = nc::nan_max(mag, fabsf(row[k]));
        const float scale = nc::token_scale(block_max(mag, scratch));
        for (int k = threadIdx.x; k < K; k += kThreads) out[k] = nc::quantize_value(row[k], scale);
        if (threadIdx.x == 0) xs[blockIdx.x] = scale;
    }
}

// The same per row, 16 bytes of x a load and 4 bytes of xq a store, for rows
// of a multiple of 4 floats on 16-byte boundaries (the maximum of |x| does not
// depend on the order it is taken in, so the bits are quantize_token's).
template <int V4>
__global__ __launch_bounds__(kThreads) void quantize_token4(int8_t *__restrict__ xq, float *__restrict__ xs,
                                                            const float *__restrict__ x, int K) {
    __shared__ float scratch[4];
    const int K4 = K >> 2;
    const float4 *row = reinterpret_cast<const float4 *>(x + (size_t)blockIdx.x * K);
    char4 *out = reinterpret_cast<char4 *>(xq + (size_t)blockIdx.x * K);
    float4 v[V4];
#pragma unroll
    for (int i = 0; i < V4; ++i) {
        const int k = threadIdx.x + i * kThreads;
        v[i] = k < K4 ? row[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float mag = 0.0f;
#pragma unroll
    for (int i = 0; i < V4; ++i)
        mag = nc::nan_max(mag, nc::nan_max(nc::nan_max(fabsf(v[i].x), fabsf(v[i].y)),
                                           nc::nan_max(fabsf(v[i].z), fabsf(v[i].w))));
    const float scale = nc::token_scale(block_max(mag, scratch));
#pragma unroll
    for (int i = 0; i < V4; ++i) {
        const int k = threadIdx.x + i * kThreads;
        if (k < K4)
            out[k] = make_char4(nc::quantize_value(v[i].x, scale), nc::quantize_value(v[i].y, scale),
                                nc::quantize_value(v[i].z, scale), nc::quantize_value(v[i].w, scale));
    }
    if (threadIdx.x == 0) xs[blockIdx.x] = scale;
}

template <int V4>
int32_t launch_token4(void **p, int M, int K) {
    hipLaunchKernelGGL(quantize_token4<V4>, dim3((unsigned)M), dim3(kThreads), 0, nc::stream(), (int8_t *)p[0],
                       (float *)p[1], (const float *)p[2], K);
    return nc::launched("quantize_token4");
}

template <int PER_THREAD>
int32_t launch_token(void **p, int M, int K) {
    hipLaunchKernelGGL(quantize_token<PER_THREAD>, dim3((unsigned)M), dim3(kThreads), 0, nc::stream(),
                       (int8_t *)p[0], (float *)p[1], (const float *)p[2], K);
    return nc::launched("quantize_token");
}

// rms_norm (nn.py:34-38: (x * (1 / sqrt(sum(x*x) / K + eps))) * gamma) and
// then the per-token quantizer on the normed row, one pass over x. normed may
// be null when only the int8 row is wanted.
template <int PER_THREAD>
__global__ __launch_bounds__(kThreads) void rms_norm_quant(float *__restrict__ normed, int8_t *__restrict__ xq,
                                                           float *__restrict__ xs, const float *__restrict__ x,
                                                           const float *__restrict__ gamma, int K, float eps) {
    __shared__ float scratch[4], scratch_max[4];      // one array a reduction
    const float *row = x + (size_t)blockIdx.x * K;
    float v[PER_THREAD];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int k = threadIdx.x + i * kThreads;
        v[i] = k < K ? row[k] : 0.0f;
        if (k < K) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
    }
    ss = block_sum(ss, scratch);
    const float rcp = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
    float mag = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int k = threadIdx.x + i * kThreads;
        v[i] = k < K ? __fmul_rn(__fmul_rn(v[i], rcp), gamma[k]) : 0.0f;
        mag = nc::nan_max(mag, fabsf(v[i]));
    }
    const float scale = nc::token_scale(block_max(mag, scratch_max));
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int k = threadIdx.x + i * kThreads;
        if (k < K) {
            if (normed) normed[(size_t)blockIdx.x * K + k] = v[i];
            xq[(size_t)blockIdx.x * K + k] = nc::quantize_value(v[i], scale);
        }
    }
    if (threadIdx.x == 0) xs[blockIdx.x] = scale;
}

template <int PER_THREAD>
int32_t launch_rms(void **p, int M, int K, float eps) {
    hipLaunchKernelGGL((rms_norm_quant<PER_THREAD>), dim3(M), dim3(kThreads), 0, nc::stream(), (float *)p[0],
                       (int8_t *)p[1], (float *)p[2], (const float *)p[3], (const float *)p[4], K, eps);
    return nc::launched("rms_norm_quant");
}


}  // namespace

// p: [q i8[N,K], scales f32[N], w f32[N,K]];  s: [N, K]
NC_EXPORT int32_t nc_quantize_rows_i8(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_quantize_rows_i8: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] > 0 && s[0] < (1 << 26) && s[1] < (1 << 26), "nc_quantize_rows_i8: bad shape");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(quantize_rows, dim3((unsigned)s[0]), dim3(kThreads), 0, nc::stream(), (int8_t *)p[0],
                       (float *)p[1], (const float *)p[2], (int)s[1]);
    return nc::launched("quantize_rows");
}

namespace nc {
int32_t quantize_token_rows(int8_t *xq, float *xs, const float *x, int M, int K) {
    void *p[3] = {xq, xs, const_cast<float *>(x)};
    if (M == 0) return NC_OK;
    if (K % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(xq) % 4 == 0) {
        if (K <= 4 * kThreads) return launch_token4<1>(p, M, K);
        if (K <= 8 * kThreads) return launch_token4<2>(p, M, K);
        if (K <= 20 * kThreads) return launch_token4<5>(p, M, K);
        if (K <= 32 * kThreads) return launch_token4<8>(p, M, K);
    }
    if (K <= 4 * kThreads) return launch_token<4>(p, M, K);
    if (K <= 8 * kThreads) return launch_token<8>(p, M, K);
    if (K <= 20 * kThreads) return launch_token<20>(p, M, K);
    if (K <= 32 * kThreads) return launch_token<32>(p, M, K);
    return launch_token<0>(p, M, K);
}
}  // namespace nc

// p: [xq i8[M,K], xs f32[M], x f32[M,K]];  s: [M, K]
NC_EXPORT int32_t nc_quantize_token_i8(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_quantize_token_i8: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] > 0 && s[0] < (1 << 26) && s[1] < (1 << 26), "nc_quantize_token_i8: bad shape");
    return nc::quantize_token_rows((int8_t *)p[0], (float *)p[1], (const float *)p[2], (int)s[0], (int)s[1]);
}

// p: [normed f32[M,K] | NULL, xq i8[M,K], xs f32[M], x f32[M,K], gamma f32[K]];
// s: [M, K, eps as float32 bits]
NC_EXPORT int32_t nc_rms_norm_quant(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[1] && p[2] && p[3] && p[4], "nc_rms_norm_quant: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] > 0 && s[0] < (1 << 26) && s[1] <= 32 * kThreads, "nc_rms_norm_quant: bad shape");
    const int M = (int)s[0], K = (int)s[1];
    const float eps = nc::bits_to_float(s[2]);
    if (M == 0) return NC_OK;
    if (K <= 4 * kThreads) return launch_rms<4>(p, M, K, eps);
    if (K <= 8 * kThreads) return launch_rms<8>(p, M, K, eps);
    if (K <= 20 * kThreads) return launch_rms<20>(p, M, K, eps);
    return launch_rms<32>(p, M, K, eps);
}

namespace {
__global__ void fp32_ops(float *__restrict__ quotient, float *__restrict__ root, float *__restrict__ rounded,
                         const float *__restrict__ a, const float *__restrict__ b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        quotient[i] = nc::div_rn(a[i], b[i]);
        root[i] = nc::sqrt_rn(fabsf(a[i]));
        rounded[i] = nc::round_half_away(a[i]);
    }
}
}  // namespace

// The device's float32 division, square root and roundf, elementwise, so a
// test can hold them to IEEE correct rounding (the reference's C uses libm's
// correctly rounded sqrtf and '/', codegen_c.py:58, 141).
// p: [a / b f32[n], sqrt(|a|) f32[n], roundf(a) f32[n], a f32[n], b f32[n]];  s: [n]
NC_EXPORT int32_t nc_probe_fp32_ops(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_probe_fp32_ops: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < (1 << 28), "nc_probe_fp32_ops: bad size");
    if (s[0] == 0) return NC_OK;
    const int n = (int)s[0];
    hipLaunchKernelGGL(fp32_ops, dim3((n + 255) / 256), dim3(256), 0, nc::stream(), (float *)p[0], (float *)p[1],
                       (float *)p[2], (const float *)p[3], (const float *)p[4], n);
    return nc::launched("fp32_ops");
}
