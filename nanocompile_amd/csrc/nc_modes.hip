// The reference's two int8 matmul modes on the GPU, bit for bit.
//
// matmul_i8 (float activations, lower.py:294-356) and matmul_i8_vnni (int8
// activations in blocks, lower.py:359-397) carry their accumulation order in
// the reference's IR: 32 float accumulators, accumulator 8c + l fed by FMA
// with element 32*k0 + 8c + l (or, for vnni, the Dp4 of bytes
// 128*k0 + 32c + 4l .. +3 scaled by its block's scale), then one fixed tree.
// At the model's widths (K = 896, 4864) 32 lanes own a weight row and lane
// 8c + l runs chain 8c + l alone, four waves a workgroup of 8 rows; at any
// other K a group of 8 lanes owns a row and lane l the four chains 8c + l
// (c = 0..3). Either way every chain runs in its own order in one lane and
// the tree, (acc[l] + acc[8+l]) + (acc[16+l] + acc[24+l]), then h[j] + h[j+4],
// then (u0 + u1) + (u2 + u3), is taken in its order through lane shuffles.
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
#include "nc_epilogue.h"
#include "nc_math.h"

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

// A serial chain over LDS (one thread's sum in index order) reads this many values ahead of its
// steps, so it waits on LDS once a batch rather than once a step.
constexpr int kChainBatch = 64;

// The model's widths (K = 128 QUADS) with a chain a lane: 32 lanes a row, lane 8c + l running
// accumulator 8c + l alone (elements 32 k0 + 8c + l, k0 in order), so a workgroup of 8 rows has
// four waves where the four-chains-a-lane form has one; lane 8c + l takes byte 4 kk + c of group
// l's 16-byte pieces (the four lanes of a group read the same piece). The tree's levels are
// shuffles in the tree's order: h[l] = (acc[l] + acc[8+l]) + (acc[16+l] + acc[24+l]),
// u[j] = h[j] + h[j+4], total = (u0 + u1) + (u2 + u3).
// gamma non-null: the row is first normalized as rms_norm_index_order does (every workgroup
// the same sum of squares in index order, so the same bits), the norm's launch saved.
template <int QUADS>
__global__ __launch_bounds__(256) void matmul_i8_lanes(float *__restrict__ y, const float *__restrict__ x,
                                                       const int8_t *__restrict__ packed,
                                                       const float *__restrict__ scales, const float *__restrict__ bias,
                                                       const float *__restrict__ residual, int N,
                                                       const float *__restrict__ gamma, float eps,
                                                       const float *__restrict__ gate) {
    constexpr int K = 128 * QUADS, PIECES = 32 * QUADS, PER = (PIECES + 255) / 256;
    constexpr int GPER = (K + 255) / 256;
    __shared__ __align__(16) float sx[K];
    const int m = blockIdx.y;
    {   // the row in 16-byte pieces, all in flight at once (rows of x start at multiples of 512 bytes)
        const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)m * K);
        float4 *s4 = reinterpret_cast<float4 *>(sx);
        float4 v[PER];                           // clamped reads: every load issued before any wait
#pragma unroll
        for (int u = 0; u < PER; ++u) v[u] = x4[min((int)threadIdx.x + 256 * u, PIECES - 1)];
#pragma unroll
        for (int u = 0; u < PER; ++u) s4[min((int)threadIdx.x + 256 * u, PIECES - 1)] = v[u];   // the last piece
                                                                  // written again with its own value
    }
    __syncthreads();
    if (gamma) {
        // rms_norm_index_order on the staged row: squares across the workgroup, the adds in
        // index order in thread 0, then (x * (1 / sqrt(ss / K + eps))) * gamma
        __shared__ __align__(16) float sq[K];
        __shared__ float rcp_shared;
        float gv[GPER];
#pragma unroll
        for (int j = 0; j < GPER; ++j) gv[j] = gamma[min((int)threadIdx.x + 256 * j, K - 1)];
#pragma unroll
        for (int j = 0; j < GPER; ++j) {
            const int k = min((int)threadIdx.x + 256 * j, K - 1);
            sq[k] = __fmul_rn(sx[k], sx[k]);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float ss = 0.0f;
            for (int k = 0; k < K; k += kChainBatch) {         // K is a multiple of the batch
                float t[kChainBatch];
#pragma unroll
                for (int u = 0; u < kChainBatch; ++u) t[u] = sq[k + u];
#pragma unroll
                for (int u = 0; u < kChainBatch; ++u) ss = __fadd_rn(ss, t[u]);
            }
            rcp_shared = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
        }
        __syncthreads();
        const float rcp = rcp_shared;
        float nv[GPER];
#pragma unroll
        for (int j = 0; j < GPER; ++j) {
            const int k = min((int)threadIdx.x + 256 * j, K - 1);
            nv[j] = __fmul_rn(__fmul_rn(sx[k], rcp), gv[j]);
        }
        __syncthreads();                                 // every read of the raw row before any write
#pragma unroll
        for (int j = 0; j < GPER; ++j) sx[min((int)threadIdx.x + 256 * j, K - 1)] = nv[j];
        __syncthreads();
    }
    const int lane = threadIdx.x & 31, c = lane >> 3, l = lane & 7;
    const int n = blockIdx.x * 8 + (int)(threadIdx.x >> 5);
    const bool valid = n < N;
    const int8_t *prow = packed + (size_t)(valid ? n : 0) * QUADS * 128 + l * 16;
    i8x16 w[QUADS];
#pragma unroll
    for (int j = 0; j < QUADS; ++j) w[j] = nc::load16(prow + (size_t)j * 128);
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < QUADS; ++j) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int8_t b = (int8_t)((w[j].w[kk] >> (8 * c)) & 0xff);
            a = __builtin_fmaf((float)b, sx[32 * (4 * j + kk) + lane], a);
        }
    }
    const float a8 = __shfl_down(a, 8, 32), a16 = __shfl_down(a, 16, 32), a24 = __shfl_down(a, 24, 32);
    const float h = __fadd_rn(__fadd_rn(a, a8), __fadd_rn(a16, a24));       // lanes 0..7
    const float u = __fadd_rn(h, __shfl_down(h, 4, 32));                     // lanes 0..3
    const float u1 = __shfl_down(u, 1, 32), u2 = __shfl_down(u, 2, 32), u3 = __shfl_down(u, 3, 32);
    const float sum = __fadd_rn(__fadd_rn(u, u1), __fadd_rn(u2, u3));        // lane 0
    if (lane == 0 && valid) {
        float v = __fmul_rn(sum, scales[n]);
        const size_t o = (size_t)m * N + n;
        if (bias) v = __fadd_rn(v, bias[n]);
        if (residual) v = __fadd_rn(residual[o], v);
        y[o] = gate ? nc::silu_mul(gate[o], v) : v;               // the up projection: silu(gate) * up
    }
}

// y[m, n] = tree(acc) (+ tail) * scales[n], float activations x[m, :] staged in LDS: any K (the
// model's widths take matmul_i8_lanes). The chains' order is the same either way.
__global__ __launch_bounds__(64) void matmul_i8_f32(float *__restrict__ y, const float *__restrict__ x,
                                                    const int8_t *__restrict__ packed, const int8_t *__restrict__ q,
                                                    const float *__restrict__ scales, const float *__restrict__ bias,
                                                    const float *__restrict__ residual, int M, int N, int K) {
    extern __shared__ __align__(16) float sx[];
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

// Any K (the model's widths take matmul_i8_vnni_lanes).
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

// The model's widths (K = 128 STRIDES) with a chain a lane, as matmul_i8_lanes: lane 8c + l runs
// accumulator 8c + l (the Dp4 of bytes 128 k0 + 32c + 4l .. +3, k0 in order), reading its own
// dword of each 128-byte packed piece, so a row's 32 lanes read the piece whole.
template <int STRIDES>
__global__ __launch_bounds__(256) void matmul_i8_vnni_lanes(float *__restrict__ y, const int8_t *__restrict__ xq,
                                                            const float *__restrict__ xs,
                                                            const float *__restrict__ offset,
                                                            const int8_t *__restrict__ packed,
                                                            const float *__restrict__ scales,
                                                            const float *__restrict__ bias,
                                                            const float *__restrict__ residual, int N, int shift,
                                                            const float *__restrict__ gate) {
    constexpr int K = 128 * STRIDES, PIECES = K / 16, PER = (PIECES + 255) / 256;
    const int block = 1 << shift;                                // a power of two: g / block = g >> shift
    __shared__ __align__(16) int8_t sxq[K];
    __shared__ float sxs[K / 32];
    const int m = blockIdx.y, nb = K / block;
    {   // the row's bytes in 16-byte pieces, all in flight at once, and its block scales
        const int4 *x16 = reinterpret_cast<const int4 *>(xq + (size_t)m * K);
        int4 *s16 = reinterpret_cast<int4 *>(sxq);
        int4 v[PER];                             // clamped reads: every load issued before any wait
#pragma unroll
        for (int u = 0; u < PER; ++u) v[u] = x16[min((int)threadIdx.x + 256 * u, PIECES - 1)];
        static_assert(K / 32 <= 256, "a block scale a thread");
        const float sv = xs[(size_t)m * nb + min((int)threadIdx.x, nb - 1)];   // nb <= K / 32
        sxs[min((int)threadIdx.x, nb - 1)] = sv;       // stores unconditional too (the last ones written
#pragma unroll                                          // again with their own values), so no load sinks
        for (int u = 0; u < PER; ++u) s16[min((int)threadIdx.x + 256 * u, PIECES - 1)] = v[u];
    }
    __syncthreads();
    const int lane = threadIdx.x & 31, c = lane >> 3, l = lane & 7;
    const int n = blockIdx.x * 8 + (int)(threadIdx.x >> 5);
    const bool valid = n < N;
    const int8_t *prow = packed + (size_t)(valid ? n : 0) * STRIDES * 128 + l * 16 + c * 4;
    int32_t w[STRIDES];
#pragma unroll
    for (int k0 = 0; k0 < STRIDES; ++k0) w[k0] = *reinterpret_cast<const int32_t *>(prow + (size_t)k0 * 128);
    float a = 0.0f;
#pragma unroll
    for (int k0 = 0; k0 < STRIDES; ++k0) {
        const int g = 128 * k0 + 32 * c;
        const int32_t xd = *reinterpret_cast<const int32_t *>(sxq + g + 4 * l);
        a = __builtin_fmaf((float)dp4_offset(w[k0], xd), sxs[g >> shift], a);
    }
    const float a8 = __shfl_down(a, 8, 32), a16 = __shfl_down(a, 16, 32), a24 = __shfl_down(a, 24, 32);
    const float h = __fadd_rn(__fadd_rn(a, a8), __fadd_rn(a16, a24));       // lanes 0..7
    const float u = __fadd_rn(h, __shfl_down(h, 4, 32));                     // lanes 0..3
    const float u1 = __shfl_down(u, 1, 32), u2 = __shfl_down(u, 2, 32), u3 = __shfl_down(u, 3, 32);
    const float sum = __fadd_rn(__fadd_rn(u, u1), __fadd_rn(u2, u3));        // lane 0
    if (lane == 0 && valid) {
        float v = __fmul_rn(__fsub_rn(sum, offset[m]), scales[n]);
        const size_t o = (size_t)m * N + n;
        if (bias) v = __fadd_rn(v, bias[n]);
        if (residual) v = __fadd_rn(residual[o], v);
        y[o] = gate ? nc::silu_mul(gate[o], v) : v;               // the up projection: silu(gate) * up
    }
}


// One block of 32 on the 32 lanes of a group, lane `lane` holding element `lane` (v): the
// block's maximum magnitude as an ordered tree of the chain's NaN-propagating step (see
// quantize_blocks), the lane's element quantized, the int32 sum of the block's values (exact in
// any order); lane 0 writes the scale and the block's term of the offset.
__device__ __forceinline__ void block32(float v, int lane, int8_t *q_out, float *scale_out, float *term_out) {
    float mag = fabsf(v);
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {
        const float other = __shfl_xor(mag, off, 32);
        const bool left = (lane & off) == 0;
        mag = nc::nan_max(left ? mag : other, left ? other : mag);
    }
    mag = nc::nan_max(0.0f, mag);
    const float scale = nc::token_scale(mag);
    const int8_t qv = nc::quantize_value(v, scale);
    q_out[lane] = qv;
    int32_t sum = qv;
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) sum += __shfl_xor(sum, off, 32);
    if (lane == 0) {
        *scale_out = scale;
        *term_out = __fmul_rn((float)sum, scale);
    }
}

// rms_norm_index_order of a row of K <= 1024 (a multiple of 64), then quantize_blocks of the
// normalized row with blocks of 32, in one workgroup: the norm's bits (the sum of squares in
// index order in thread 0, then (x * (1 / sqrt(ss / K + eps))) * gamma) and the quantizer's.
__global__ __launch_bounds__(256) void quantize_blocks_normed(int8_t *__restrict__ xq, float *__restrict__ xs,
                                                              float *__restrict__ offset, const float *__restrict__ x,
                                                              const float *__restrict__ gamma, int K, float eps) {
    extern __shared__ __align__(16) float nsmem[];           // the row's squares, then its normed values
    float *nrow = nsmem, *terms = nsmem + K;                 // and a term per block
    __shared__ float rcp_shared;
    const int m = blockIdx.x, nb = K / 32;
    const float *row = x + (size_t)m * K;
    float xv[4], gv[4];                                      // clamped reads: all issued before any wait
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = min((int)threadIdx.x + 256 * j, K - 1);
        xv[j] = row[k];
        gv[j] = gamma[k];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = threadIdx.x + 256 * j;
        if (k < K) nrow[k] = __fmul_rn(xv[j], xv[j]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int k = 0; k < K; k += kChainBatch) {
            float t[kChainBatch];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) t[u] = nrow[k + u];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) ss = __fadd_rn(ss, t[u]);
        }
        rcp_shared = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
    }
    __syncthreads();                                         // thread 0's reads of the squares are done
    const float rcp = rcp_shared;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = threadIdx.x + 256 * j;
        if (k < K) nrow[k] = __fmul_rn(__fmul_rn(xv[j], rcp), gv[j]);
    }
    __syncthreads();
    const int lane = threadIdx.x & 31, group = threadIdx.x >> 5;
    for (int b = group; b < nb; b += 8)
        block32(nrow[b * 32 + lane], lane, xq + (size_t)m * K + (size_t)b * 32, xs + (size_t)m * nb + b, terms + b);
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (int b = 0; b < nb; ++b) total = __fadd_rn(total, terms[b]);
        offset[m] = __fmul_rn(total, 128.0f);
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
    if (block == 32) {
        // a block of 32 on 32 lanes, an element a lane. The chain's maximum, mag = nan_max(mag,
        // |v_i|) from 0 in index order, as an ordered tree: its step is associative (a NaN on
        // the right wins, else one on the left, else the leftmost maximum), so lanes combined
        // by xor butterfly with the lower lanes' block on the left, then one step from 0, give
        // the chain's bits. Each lane quantizes its own element; the int32 sum is exact in any
        // order.
        const int lane = threadIdx.x & 31, group = threadIdx.x >> 5;
        auto one_block = [&](int b, float v) {
            block32(v, lane, xq + (size_t)m * K + (size_t)b * 32, xs + (size_t)m * nb + b, terms + b);
        };
        // a group's blocks b = group + 8 i: the first kHeldBlocks loaded before any is waited on
        // (K up to 5120 at once), the rest one after another
        constexpr int kHeldBlocks = 20;
        float held[kHeldBlocks];
#pragma unroll
        for (int i = 0; i < kHeldBlocks; ++i) {
            const int b = group + 8 * i;
            held[i] = row[(size_t)min(b, nb - 1) * 32 + lane];     // clamped: no load waits on another
        }
#pragma unroll
        for (int i = 0; i < kHeldBlocks; ++i) asm volatile("" : "+v"(held[i]));   // every value here before
#pragma unroll                                                                   // any block runs, so no
        for (int i = 0; i < kHeldBlocks; ++i) {                                  // load sinks into one
            const int b = group + 8 * i;
            if (b < nb) one_block(b, held[i]);
        }
        for (int b = group + 8 * kHeldBlocks; b < nb; b += 8) one_block(b, row[(size_t)b * 32 + lane]);
    } else {
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
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        int b = 0;
        for (; b + kChainBatch <= nb; b += kChainBatch) {
            float t[kChainBatch];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) t[u] = terms[b + u];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) total = __fadd_rn(total, t[u]);
        }
        for (; b < nb; ++b) total = __fadd_rn(total, terms[b]);
        offset[m] = __fmul_rn(total, 128.0f);
    }
}

// The reference's rms_norm row kernel in its own order (nn.py:34-38, fusion.py:631-650): the
// sum of squares in index order, one multiply and one add a step from 0, then
// (x * (1 / sqrt(ss / K + eps))) * gamma. The row and its squares are staged in
// LDS (every thread squaring its share: the same products), the one chain of adds
// runs in lane 0, and every thread then writes its share of the row.
__global__ __launch_bounds__(256) void rms_norm_index_order(float *__restrict__ normed, const float *__restrict__ x,
                                                            const float *__restrict__ gamma, int K, float eps) {
    extern __shared__ __align__(16) float sq[];  // the row's squares
    __shared__ float rcp_shared;
    constexpr int kHeld = 4;                     // values a thread holds in registers (the rest re-read)
    const float *row = x + (size_t)blockIdx.x * K;
    float xv[kHeld], gv[kHeld];                  // every load issued before the first is waited on
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
        const int k = threadIdx.x + j * blockDim.x;
        xv[j] = row[min(k, K - 1)];              // clamped reads: no load waits on another
        gv[j] = gamma[min(k, K - 1)];
    }
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
        const int k = threadIdx.x + j * blockDim.x;
        if (k < K) sq[k] = __fmul_rn(xv[j], xv[j]);   // every thread its squares; the chain only adds
    }
    for (int k = threadIdx.x + kHeld * blockDim.x; k < K; k += blockDim.x) sq[k] = __fmul_rn(row[k], row[k]);
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        int k = 0;
        for (; k + kChainBatch <= K; k += kChainBatch) {       // a batch's reads ahead of its steps
            float v[kChainBatch];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) v[u] = sq[k + u];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) ss = __fadd_rn(ss, v[u]);
        }
        for (; k < K; ++k) ss = __fadd_rn(ss, sq[k]);
        rcp_shared = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
    }
    __syncthreads();
    const float rcp = rcp_shared;
    float *out = normed + (size_t)blockIdx.x * K;
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
        const int k = threadIdx.x + j * blockDim.x;
        if (k < K) out[k] = __fmul_rn(__fmul_rn(xv[j], rcp), gv[j]);
    }
    for (int k = threadIdx.x + kHeld * blockDim.x; k < K; k += blockDim.x)
        out[k] = __fmul_rn(__fmul_rn(row[k], rcp), gamma[k]);
}

// The reference's attention for one query row and one head, in the order its graph states it
// (models/qwen2.py:143-147, nn.py:57-66, 109-135): each score a dot product over d in order,
// one multiply and one add a step from 0, times scale, plus the mask's 0; the row's maximum;
// e_t = exp(z_t - max); their sum in order of t from 0; p_t = e_t / sum; the context
// sum over t in order of p_t * v_t[d]. The key of row i at absolute position past + i sees
// positions 0 .. past + i; the masked positions after them would add exp(-inf) = 0 to the sum
// and 0 * v to each context sum, neither of which changes a float, so they are skipped.
// Keys and values come from the cache (RoPE'd keys; this call's rows already appended), the
// KV head of query head h being h / (heads / kv) (repeat_kv's consecutive groups).
// LDS: one float per visible position (the scores, then the exponentials, then p).
__global__ __launch_bounds__(256) void attention_index_order(float *__restrict__ ctx, const float *__restrict__ qkv,
                                                             const float *__restrict__ kcache,
                                                             const float *__restrict__ vcache,
                                                             const int64_t *__restrict__ pos, int heads, int kv,
                                                             int D, int past_arg, int M, int capacity, float scale,
                                                             int32_t *__restrict__ error) {
    extern __shared__ float sp[];
    __shared__ float sq[128];
    __shared__ float shared_max[4];
    __shared__ float shared_sum;
    const int i = blockIdx.x, h = blockIdx.y, g = h / (heads / kv);
    int past = past_arg;
    if (pos) {
        // a position read on the device (a captured decode step) must leave room for the M rows;
        // every thread reads the same word and takes the same branch
        const int64_t at = pos[0];
        if (at < 0 || at + M > capacity) {
            if (i == 0 && h == 0 && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_CAPACITY);
            return;
        }
        past = (int)at;
    }
    const int T = past + i + 1;
    const int W = (heads + 2 * kv) * D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) sq[d] = qkv[(size_t)i * W + (size_t)h * D + d];
    __syncthreads();
    const float *kh = kcache + (size_t)g * capacity * D;
    const float *vh = vcache + (size_t)g * capacity * D;
    float mx = -__builtin_inff();
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
        const float *kt = kh + (size_t)t * D;
        float acc = 0.0f;
        int d = 0;
        for (; d + 16 <= D; d += 16) {                        // the key's values ahead of the chain
            float kv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) kv[u] = kt[d + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) acc = __fadd_rn(acc, __fmul_rn(sq[d + u], kv[u]));
        }
        for (; d < D; ++d) acc = __fadd_rn(acc, __fmul_rn(sq[d], kt[d]));
        const float z = __fadd_rn(__fmul_rn(acc, scale), 0.0f);
        sp[t] = z;
        mx = nc::nan_max(mx, z);
    }
    // the maximum is exact in any order; NaN from any score wins, as the reference's does
    mx = nc::wave_max_f32(mx);
    if ((threadIdx.x & 63) == 0) shared_max[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = shared_max[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) mx = nc::nan_max(mx, shared_max[w]);
    for (int t = threadIdx.x; t < T; t += blockDim.x) sp[t] = nc_expf(__fsub_rn(sp[t], mx));
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        int t = 0;
        for (; t + kChainBatch <= T; t += kChainBatch) {
            float e[kChainBatch];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) e[u] = sp[t + u];
#pragma unroll
            for (int u = 0; u < kChainBatch; ++u) total = __fadd_rn(total, e[u]);
        }
        for (; t < T; ++t) total = __fadd_rn(total, sp[t]);
        shared_sum = total;
    }
    __syncthreads();
    const float total = shared_sum;
    for (int t = threadIdx.x; t < T; t += blockDim.x) sp[t] = nc::div_rn(sp[t], total);
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float acc = 0.0f;
        int t = 0;
        for (; t + 64 <= T; t += 64) {                        // 64 positions' p and v ahead of the chain
            float pv[64], vv[64];
#pragma unroll
            for (int u = 0; u < 64; ++u) {
                pv[u] = sp[t + u];
                vv[u] = vh[(size_t)(t + u) * D + d];
            }
#pragma unroll
            for (int u = 0; u < 64; ++u) acc = __fadd_rn(acc, __fmul_rn(pv[u], vv[u]));
        }
        for (; t + 16 <= T; t += 16) {
            float pv[16], vv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                pv[u] = sp[t + u];
                vv[u] = vh[(size_t)(t + u) * D + d];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) acc = __fadd_rn(acc, __fmul_rn(pv[u], vv[u]));
        }
        for (; t < T; ++t) acc = __fadd_rn(acc, __fmul_rn(sp[t], vh[(size_t)t * D + d]));
        ctx[(size_t)i * heads * D + (size_t)h * D + d] = acc;
    }
}

}  // namespace

// The reference's rms_norm in its index order (reference modes), normed rows only.
// p: [normed f32[M,K], x f32[M,K], gamma f32[K]];  s: [M, K, eps as float32 bits]
NC_EXPORT int32_t nc_rms_norm_index_order(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_rms_norm_index_order: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < (1 << 26) && s[1] > 0 && s[1] <= 16384, "nc_rms_norm_index_order: bad shape");
    if (s[0] == 0) return NC_OK;
    static bool raised = false;                  // the row's squares: up to 64 KB of LDS beside the static
    if (!raised) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&rms_norm_index_order),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 16384 * sizeof(float)) != hipSuccess) {
            nc::set_message("nc_rms_norm_index_order: could not raise the LDS limit");
            return NC_LAUNCH_FAILED;
        }
        raised = true;
    }
    hipLaunchKernelGGL(rms_norm_index_order, dim3((unsigned)s[0]), dim3(256), (size_t)s[1] * sizeof(float),
                       nc::stream(), (float *)p[0], (const float *)p[1], (const float *)p[2], (int)s[1],
                       nc::bits_to_float(s[2]));
    return nc::launched("rms_norm_index_order");
}

// The reference's attention in its own order (reference modes), after nc_rope_append.
// p: [ctx f32[M, heads*D], qkv f32[M, (heads+2kv)*D] (q rotated), kcache f32[kv, capacity, D],
//     vcache f32[kv, capacity, D] (rows 0 .. past+M-1 filled), pos i64[1] | NULL (past read on the device)];
// s: [M, heads, kv, D, past, capacity, scale as float32 bits]
NC_EXPORT int32_t nc_attention_index_order(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3], "nc_attention_index_order: null operand");
    const int64_t M = s[0], heads = s[1], kv = s[2], D = s[3], past = s[4], capacity = s[5];
    // one float of LDS per position the rows can see, beside 0.5 KB of the kernel's own: within 64 KB
    NC_REQUIRE(M >= 0 && M < 65536 && heads > 0 && heads < 65536 && kv > 0 && heads % kv == 0 && D > 0 &&
                   D <= 128 && past >= 0 && capacity > 0 && capacity <= 16000 && past + M <= capacity,
               "nc_attention_index_order: bad shape (head_dim at most 128, at most 16000 positions)");
    if (M == 0) return NC_OK;
    hipLaunchKernelGGL(attention_index_order, dim3((unsigned)M, (unsigned)heads), dim3(256),
                       (size_t)capacity * sizeof(float), nc::stream(), (float *)p[0], (const float *)p[1],
                       (const float *)p[2], (const float *)p[3], (const int64_t *)p[4], (int)heads, (int)kv, (int)D,
                       (int)past, (int)M, (int)capacity, nc::bits_to_float(s[6]), nc::error_word());
    return nc::launched("attention_index_order");
}

// The reference's matmul_i8: y = x @ (q * scales).T in its 32-chain order, then
// + bias, then residual +.
// p: [y f32[M,N], x f32[M,K], packed i8 (nc_pack layout, float mode), q i8[N,K], scales f32[N],
//     bias f32[N] | NULL, residual f32[M,N] | NULL];  s: [M, N, K]
NC_EXPORT int32_t nc_matmul_i8(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_matmul_i8: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < 65536 && s[1] >= 0 && s[1] < (1 << 24) && s[2] > 0 && s[2] <= 16384,
               "nc_matmul_i8: bad shape (K at most 16384)");
    if (s[0] == 0 || s[1] == 0) return NC_OK;
    // the model's widths, x 16-byte aligned: a chain a lane, the row staged in 16-byte pieces
    const bool whole = ((uintptr_t)p[1] & 15) == 0;
    if (whole && (s[2] == 896 || s[2] == 4864)) {
        const auto kernel = s[2] == 896 ? matmul_i8_lanes<7> : matmul_i8_lanes<38>;
        hipLaunchKernelGGL(kernel, dim3((unsigned)((s[1] + 7) / 8), (unsigned)s[0]), dim3(256), 0, nc::stream(),
                           (float *)p[0], (const float *)p[1], (const int8_t *)p[2], (const float *)p[4],
                           (const float *)p[5], (const float *)p[6], (int)s[1], (const float *)nullptr, 0.0f,
                           (const float *)nullptr);
        return nc::launched("matmul_i8_lanes");
    }
    hipLaunchKernelGGL(matmul_i8_f32, dim3((unsigned)((s[1] + 7) / 8), (unsigned)s[0]), dim3(64),
                       (size_t)s[2] * sizeof(float), nc::stream(), (float *)p[0], (const float *)p[1],
                       (const int8_t *)p[2], (const int8_t *)p[3], (const float *)p[4], (const float *)p[5],
                       (const float *)p[6], (int)s[0], (int)s[1], (int)s[2]);
    return nc::launched("matmul_i8_f32");
}

// rms_norm_index_order then matmul_i8 in one launch, at the model's widths (x 16-byte aligned).
// p: [y f32[M,N], x f32[M,K], packed i8, q i8[N,K], scales f32[N], bias | NULL, residual | NULL,
//     gamma f32[K]];  s: [M, N, K, eps as float32 bits]
NC_EXPORT int32_t nc_matmul_i8_normed(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[7], "nc_matmul_i8_normed: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < 65536 && s[1] >= 0 && s[1] < (1 << 24) && (s[2] == 896 || s[2] == 4864) &&
                   ((uintptr_t)p[1] & 15) == 0,
               "nc_matmul_i8_normed: bad shape (K 896 or 4864, x 16-byte aligned)");
    NC_REQUIRE(p[6] != p[1] && p[0] != p[1], "nc_matmul_i8_normed: y and the residual may not be x");
    if (s[0] == 0 || s[1] == 0) return NC_OK;
    const auto kernel = s[2] == 896 ? matmul_i8_lanes<7> : matmul_i8_lanes<38>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)((s[1] + 7) / 8), (unsigned)s[0]), dim3(256), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const int8_t *)p[2], (const float *)p[4],
                       (const float *)p[5], (const float *)p[6], (int)s[1], (const float *)p[7],
                       nc::bits_to_float(s[3]), (const float *)nullptr);
    return nc::launched("matmul_i8_lanes (normed)");
}

// matmul_i8 of the up projection with SwiGLU in its epilogue: h = silu(gate) * (x @ up.T),
// nc_silu_mul's operations on the projection's value (the model's widths, x 16-byte aligned).
// p: [h f32[M,N], x f32[M,K], packed i8, q i8[N,K], scales f32[N], gate f32[M,N]];  s: [M, N, K]
NC_EXPORT int32_t nc_matmul_i8_silu(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[5], "nc_matmul_i8_silu: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < 65536 && s[1] >= 0 && s[1] < (1 << 24) && (s[2] == 896 || s[2] == 4864) &&
                   ((uintptr_t)p[1] & 15) == 0 && p[0] != p[1],
               "nc_matmul_i8_silu: bad shape (K 896 or 4864, x 16-byte aligned, h not x)");
    if (s[0] == 0 || s[1] == 0) return NC_OK;
    const auto kernel = s[2] == 896 ? matmul_i8_lanes<7> : matmul_i8_lanes<38>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)((s[1] + 7) / 8), (unsigned)s[0]), dim3(256), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const int8_t *)p[2], (const float *)p[4],
                       (const float *)nullptr, (const float *)nullptr, (int)s[1], (const float *)nullptr, 0.0f,
                       (const float *)p[5]);
    return nc::launched("matmul_i8_lanes (silu)");
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
    // the model's widths, xq 16-byte aligned: a chain a lane, the row staged in 16-byte pieces
    if (((uintptr_t)p[1] & 15) == 0 && (K == 896 || K == 4864)) {
        const auto kernel = K == 896 ? matmul_i8_vnni_lanes<7> : matmul_i8_vnni_lanes<38>;
        hipLaunchKernelGGL(kernel, dim3((unsigned)((N + 7) / 8), (unsigned)M), dim3(256), 0, nc::stream(),
                           (float *)p[0], (const int8_t *)p[1], (const float *)p[2], (const float *)p[3],
                           (const int8_t *)p[4], (const float *)p[6], (const float *)p[7], (const float *)p[8],
                           (int)N, __builtin_ctzll((unsigned long long)block), (const float *)nullptr);
        return nc::launched("matmul_i8_vnni_lanes");
    }
    const size_t lds = (size_t)((K + 15) / 16) * 16 + (size_t)(K / block) * sizeof(float);
    hipLaunchKernelGGL(matmul_i8_vnni, dim3((unsigned)((N + 7) / 8), (unsigned)M), dim3(64), lds, nc::stream(),
                       (float *)p[0], (const int8_t *)p[1], (const float *)p[2], (const float *)p[3],
                       (const int8_t *)p[4], (const int8_t *)p[5], (const float *)p[6], (const float *)p[7],
                       (const float *)p[8], (int)M, (int)N, (int)K, (int)block);
    return nc::launched("matmul_i8_vnni");
}

// matmul_i8_vnni of the up projection with SwiGLU in its epilogue (as nc_matmul_i8_silu).
// p: [h f32[M,N], xq i8[M,K], xs f32[M,K/block], offset f32[M], packed i8, q i8[N,K], scales f32[N],
//     gate f32[M,N]];  s: [M, N, K, block] (K 896 or 4864, xq 16-byte aligned)
NC_EXPORT int32_t nc_matmul_i8_vnni_silu(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[5] && p[6] && p[7],
               "nc_matmul_i8_vnni_silu: null operand");
    const int64_t M = s[0], N = s[1], K = s[2], block = s[3];
    NC_REQUIRE(M >= 0 && M < 65536 && N >= 0 && N < (1 << 24) && (K == 896 || K == 4864) && block >= 32 &&
                   (block & (block - 1)) == 0 && K % block == 0 && ((uintptr_t)p[1] & 15) == 0,
               "nc_matmul_i8_vnni_silu: bad shape (K 896 or 4864, block a power of two >= 32 dividing K)");
    if (M == 0 || N == 0) return NC_OK;
    const auto kernel = K == 896 ? matmul_i8_vnni_lanes<7> : matmul_i8_vnni_lanes<38>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)((N + 7) / 8), (unsigned)M), dim3(256), 0, nc::stream(),
                       (float *)p[0], (const int8_t *)p[1], (const float *)p[2], (const float *)p[3],
                       (const int8_t *)p[4], (const float *)p[6], (const float *)nullptr, (const float *)nullptr,
                       (int)N, __builtin_ctzll((unsigned long long)block), (const float *)p[7]);
    return nc::launched("matmul_i8_vnni_lanes (silu)");
}

// p: [xq i8[M,K], xs f32[M,K/32], offset f32[M], x f32[M,K], gamma f32[K]];
// s: [M, K, eps as float32 bits] (K a multiple of 64, at most 1024; blocks of 32)
NC_EXPORT int32_t nc_quantize_blocks_normed(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_quantize_blocks_normed: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < (1 << 30) && s[1] > 0 && s[1] <= 1024 && s[1] % 64 == 0,
               "nc_quantize_blocks_normed: bad shape (K a multiple of 64, at most 1024)");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(quantize_blocks_normed, dim3((unsigned)s[0]), dim3(256),
                       (size_t)(s[1] + s[1] / 32) * sizeof(float), nc::stream(), (int8_t *)p[0], (float *)p[1],
                       (float *)p[2], (const float *)p[3], (const float *)p[4], (int)s[1], nc::bits_to_float(s[2]));
    return nc::launched("quantize_blocks_normed");
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
