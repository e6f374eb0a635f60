// The reference's two int8 matmul modes on the GPU, bit for bit.
//
// matmul_i8 (float activations, lower.py:294-356) and matmul_i8_vnni (int8
// activations in blocks, lower.py:359-397) carry their accumulation order in
// the reference's IR: 32 float accumulators, accumulator 8c + l fed by FMA
// with element 32*k0 + 8c + l (or, for vnni, the Dp4 of bytes
// 128*k0 + 32c + 4l .. +3 scaled by its block's scale), then one fixed tree.
// Here a group of 8 lanes owns a weight row and lane l owns the four chains
// 8c + l (c = 0..3), so every chain runs in its own order in one lane and the
// tree's first level, (acc[l] + acc[8+l]) + (acc[16+l] + acc[24+l]), is local;
// its last two levels are lane shuffles in the tree's order.
//
// Coalescing takes a repacked weight layout (the reference's pack idea,
// schedule.py:362-395), made once per weight on the host side of the library:
//   float mode: per row, per group of 4 blocks of 32, lane l's 16 bytes are
//     [block][c] = w[32*k0 + 8c + l], so the 8 lanes read 128 contiguous bytes;
//   vnni mode: per row, per block of 128, lane l's 16 bytes are the four
//     dwords w[128*k0 + 32c + 4l .. +3], c = 0..3: again 128 contiguous bytes.
// Elements past the last whole 32-block (or 128-block) are read from the
// plain row-major weights, in the reference's order.
#include "nc_common.h"

namespace {

using nc::i8x16;

__device__ __forceinline__ float tree_of_chains(float a0, float a1, float a2, float a3) {
    // h[l] = (acc[l] + acc[8+l]) + (acc[16+l] + acc[24+l]); u[j] = h[j] + h[j+4];
    // total = (u0 + u1) + (u2 + u3), lanes l = 0..7 of the row's group.
    const float h = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
    const float h4 = __shfl_down(h, 4, 8);
    const float u = __fadd_rn(h, h4);                 // valid in lanes 0..3
    const float u1 = __shfl_down(u, 1, 8), u2 = __shfl_down(u, 2, 8), u3 = __shfl_down(u, 3, 8);
    return __fadd_rn(__fadd_rn(u, u1), __fadd_rn(u2, u3));   // valid in lane 0
}

__device__ __forceinline__ int8_t byte_of(const i8x16 &v, int i) {
    return (int8_t)((v.w[i >> 2] >> (8 * (i & 3))) & 0xff);
}

// y[m, n] = tree(acc) (+ tail) * scales[n], float activations x[m, :] staged in LDS.
__global__ __launch_bounds__(64) void matmul_i8_f32(float *__restrict__ y, const float *__restrict__ x,
                                                    const int8_t *__restrict__ packed, const int8_t *__restrict__ q,
                                                    const float *__restrict__ scales, const float *__restrict__ bias,
                                                    const float *__restrict__ residual, int M, int N, int K) {
    extern __shared__ float sx[];
    const int m = blockIdx.y;
    for (int i = threadIdx.x; i < K; i += 64) sx[i] = x[(size_t)m * K + i];
    __syncthreads();
    const int lane = threadIdx.x, l = lane & 7;
    const int n = blockIdx.x * 8 + lane / 8;
    const bool valid = n < N;
    const int nr = valid ? n : 0;
    const int blocks = K / 32, quads = (blocks + 3) / 4;
    const int8_t *prow = packed + (size_t)nr * quads * 128 + l * 16;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < quads; ++j) {
        const i8x16 w = nc::load16(prow + (size_t)j * 128);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int k0 = 4 * j + kk;
            if (k0 < blocks) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    a[c] = __builtin_fmaf((float)byte_of(w, kk * 4 + c), sx[32 * k0 + 8 * c + l], a[c]);
            }
        }
    }
    const int wide = blocks * 32, groups = (K % 32) / 8, tail = wide + groups * 8;
    const int8_t *row = q + (size_t)nr * K;
    for (int k1 = 0; k1 < groups; ++k1) {
        const int at = wide + 8 * k1 + l;
        a[0] = __builtin_fmaf((float)row[at], sx[at], a[0]);
    }
    float sum = tree_of_chains(a[0], a[1], a[2], a[3]);
    if (l == 0 && valid) {
        for (int at = tail; at < K; ++at) sum = __fadd_rn(sum, __fmul_rn((float)row[at], sx[at]));
        float v = __fmul_rn(sum, scales[n]);
        const size_t o = (size_t)m * N + n;
        if (bias) v = __fadd_rn(v, bias[n]);
        if (residual) v = __fadd_rn(residual[o], v);
        y[o] = v;
    }
}

// Dp4 = sum_j (w_j + 128) * x_j = sdot4(w, x) + 128 * sum_j x_j, exact in int32.
__device__ __forceinline__ int32_t dp4_offset(int32_t w, int32_t x) {
    return nc::dot4(w, x, 0) + 128 * nc::dot4(x, 0x01010101, 0);
}

__global__ __launch_bounds__(64) void matmul_i8_vnni(float *__restrict__ y, const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xs, const float *__restrict__ offset,
                                                     const int8_t *__restrict__ packed, const int8_t *__restrict__ q,
                                                     const float *__restrict__ scales, const float *__restrict__ bias,
                                                     const float *__restrict__ residual, int M, int N, int K,
                                                     int block) {
    extern __shared__ __align__(16) int8_t smem[];
    int8_t *sxq = smem;                                          // K bytes
    float *sxs = reinterpret_cast<float *>(smem + ((K + 15) / 16) * 16);   // K / block floats
    const int m = blockIdx.y, nb = K / block;
    for (int i = threadIdx.x; i < K; i += 64) sxq[i] = xq[(size_t)m * K + i];
    for (int i = threadIdx.x; i < nb; i += 64) sxs[i] = xs[(size_t)m * nb + i];
    __syncthreads();
    const int lane = threadIdx.x, l = lane & 7;
    const int n = blockIdx.x * 8 + lane / 8;
    const bool valid = n < N;
    const int nr = valid ? n : 0;
    const int strides = K / 128;
    const int8_t *prow = packed + (size_t)nr * strides * 128 + l * 16;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < strides; ++k0) {
        const i8x16 w = nc::load16(prow + (size_t)k0 * 128);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int g = 128 * k0 + 32 * c;
            const int32_t xd = *reinterpret_cast<const int32_t *>(sxq + g + 4 * l);
            a[c] = __builtin_fmaf((float)dp4_offset(w.w[c], xd), sxs[g / block], a[c]);
        }
    }
    const int groups = (K % 128) / 32;
    const int8_t *row = q + (size_t)nr * K;
    for (int k1 = 0; k1 < groups; ++k1) {
        const int g = strides * 128 + 32 * k1;
        const int32_t wd = *reinterpret_cast<const int32_t *>(row + g + 4 * l);
        const int32_t xd = *reinterpret_cast<const int32_t *>(sxq + g + 4 * l);
        a[0] = __builtin_fmaf((float)dp4_offset(wd, xd), sxs[g / block], a[0]);
    }
    const float sum = tree_of_chains(a[0], a[1], a[2], a[3]);
    if (l == 0 && valid) {
        float v = __fmul_rn(__fsub_rn(sum, offset[m]), scales[n]);
        const size_t o = (size_t)m * N + n;
        if (bias) v = __fadd_rn(v, bias[n]);
        if (residual) v = __fadd_rn(residual[o], v);
        y[o] = v;
    }
}

// quantize.py:102-124: per block of `block` values, scale = max|x| / 127 (1 if
// zero), xq = clamp(round(x / scale)); offset = 128 * sum over blocks, in
// order, of f32(sum of the block's xq) * scale.
__global__ __launch_bounds__(256) void quantize_blocks(int8_t *__restrict__ xq, float *__restrict__ xs,
                                                       float *__restrict__ offset, const float *__restrict__ x, int K,
                                                       int block) {
    extern __shared__ float terms[];                              // one per block
    const int m = blockIdx.x, nb = K / block;
    const float *row = x + (size_t)m * K;
    for (int b = threadIdx.x; b < nb; b += 256) {
        const float *v = row + (size_t)b * block;
        float mag = 0.0f;
        for (int i = 0; i < block; ++i) mag = nc::nan_max(mag, fabsf(v[i]));
        const float scale = nc::token_scale(mag);
        int32_t sum = 0;
        for (int i = 0; i < block; ++i) {
            const int8_t qv = nc::quantize_value(v[i], scale);
            xq[(size_t)m * K + (size_t)b * block + i] = qv;
            sum += qv;
        }
        xs[(size_t)m * nb + b] = scale;
        terms[b] = __fmul_rn((float)sum, scale);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (int b = 0; b < nb; ++b) total = __fadd_rn(total, terms[b]);
        offset[m] = __fmul_rn(total, 128.0f);
    }
}

}  // namespace

// The reference's matmul_i8: y = x @ (q * scales).T in its 32-chain order, then
// + bias, then residual +.
// p: [y f32[M,N], x f32[M,K], packed i8 (nc_pack layout, float mode), q i8[N,K], scales f32[N],
//     bias f32[N] | NULL, residual f32[M,N] | NULL];  s: [M, N, K]
NC_EXPORT int32_t nc_matmul_i8(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_matmul_i8: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < 65536 && s[1] >= 0 && s[1] < (1 << 24) && s[2] > 0 && s[2] <= 16384,
               "nc_matmul_i8: bad shape (K at most 16384)");
    if (s[0] == 0 || s[1] == 0) return NC_OK;
    hipLaunchKernelGGL(matmul_i8_f32, dim3((unsigned)((s[1] + 7) / 8), (unsigned)s[0]), dim3(64),
                       (size_t)s[2] * sizeof(float), nc::stream(), (float *)p[0], (const float *)p[1],
                       (const int8_t *)p[2], (const int8_t *)p[3], (const float *)p[4], (const float *)p[5],
                       (const float *)p[6], (int)s[0], (int)s[1], (int)s[2]);
    return nc::launched("matmul_i8_f32");
}

// The reference's matmul_i8_vnni: y = (sum_b xs[b] * Dp4 sums - offset) * scales in its order.
// p: [y f32[M,N], xq i8[M,K], xs f32[M,K/block], offset f32[M], packed i8 (vnni layout), q i8[N,K],
//     scales f32[N], bias | NULL, residual | NULL];  s: [M, N, K, block]
NC_EXPORT int32_t nc_matmul_i8_vnni(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[5] && p[6], "nc_matmul_i8_vnni: null operand");
    const int64_t M = s[0], N = s[1], K = s[2], block = s[3];
    NC_REQUIRE(M >= 0 && M < 65536 && N >= 0 && N < (1 << 24) && K > 0 && K <= 16384 && block >= 32 &&
                   (block & (block - 1)) == 0 && K % block == 0,
               "nc_matmul_i8_vnni: bad shape (block a power of two >= 32 dividing K)");
    if (M == 0 || N == 0) return NC_OK;
    const size_t lds = (size_t)((K + 15) / 16) * 16 + (size_t)(K / block) * sizeof(float);
    hipLaunchKernelGGL(matmul_i8_vnni, dim3((unsigned)((N + 7) / 8), (unsigned)M), dim3(64), lds, nc::stream(),
                       (float *)p[0], (const int8_t *)p[1], (const float *)p[2], (const float *)p[3],
                       (const int8_t *)p[4], (const int8_t *)p[5], (const float *)p[6], (const float *)p[7],
                       (const float *)p[8], (int)M, (int)N, (int)K, (int)block);
    return nc::launched("matmul_i8_vnni");
}

// p: [xq i8[M,K], xs f32[M,K/block], offset f32[M], x f32[M,K]];  s: [M, K, block]
NC_EXPORT int32_t nc_quantize_blocks(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3], "nc_quantize_blocks: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < (1 << 30) && s[1] > 0 && s[2] > 0 && s[1] % s[2] == 0 && s[1] / s[2] <= 16384,
               "nc_quantize_blocks: bad shape (K a whole number of blocks)");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(quantize_blocks, dim3((unsigned)s[0]), dim3(256), (size_t)(s[1] / s[2]) * sizeof(float),
                       nc::stream(), (int8_t *)p[0], (float *)p[1], (float *)p[2], (const float *)p[3], (int)s[1],
                       (int)s[2]);
    return nc::launched("quantize_blocks");
}
