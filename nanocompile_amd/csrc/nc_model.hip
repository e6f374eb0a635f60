// The model's ends: the embedding gather, the float32 LM head and the argmax.
//
// * Gather (lower.py:420-444, fusion.py:712-731): rows of the table by index;
//   an index outside 0..V-1 is the reference's Fail code 1, recorded in the
//   library's device error word (nc_sync returns it) and the row left zero.
// * LM head (models/qwen2.py:210-221, A15 in the reference's matmul kernel,
//   lower.py:255-269): logits[n] = sum over k of x[k] * E[n, k], one
//   accumulator, multiply then add, k in order. That is the reference's own
//   bit pattern. The table is read in a packed layout (the reference's pack,
//   schedule.py:362-395, runtime.py:157-164): blocks of 64 rows, and within a
//   block 4 consecutive k of each row together, so the 64 lanes of a wave read
//   1 KB contiguous per load while each lane still walks its own row in order.
// * Argmax: the first index of the largest logit (numpy.argmax), folded into
//   the LM head as a 64-bit atomic maximum of (ordered value bits, ~index), so
//   ties go to the smallest index whatever order the waves finish in.
#include "nc_common.h"

namespace {

__global__ __launch_bounds__(256) void embed_rows(float *__restrict__ x, const float *__restrict__ table,
                                                  const int64_t *__restrict__ ids, int H, int64_t V,
                                                  int32_t *__restrict__ error) {
    const int m = blockIdx.x;
    const int64_t id = ids[m];
    const bool bad = id < 0 || id >= V;
    if (bad && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_INDEX);
    const float *row = table + (bad ? 0 : id) * (int64_t)H;
    for (int k = threadIdx.x; k < H; k += 256) x[(size_t)m * H + k] = bad ? 0.0f : row[k];
}

// Packed index of (n, k): ((n / 64) * (H / 4) + k / 4) * 256 + (n % 64) * 4 + k % 4.
__global__ __launch_bounds__(256) void pack_rows64(float *__restrict__ packed, const float *__restrict__ table,
                                                   int64_t V, int H) {
    const int64_t blk = blockIdx.x;
    const int k4n = H / 4;
    for (int i = threadIdx.x; i < k4n * 64; i += 256) {
        const int k4 = i / 64, lane = i % 64;
        const int64_t n = blk * 64 + lane;
        float4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (n < V) v = *reinterpret_cast<const float4 *>(table + n * H + k4 * 4);
        reinterpret_cast<float4 *>(packed)[(blk * k4n + k4) * 64 + lane] = v;
    }
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int64_t n) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)n);
}

// Row m of x into LDS (sxh[0 .. H - 1]), rms-normed first (nn.py:34-38) when
// gamma is given, in the row kernels' order: virtual thread t of 256 sums
// x[t]^2, x[t+256]^2, ... in order; the butterfly over each group of 64
// virtual threads; (w0 + w1) + (w2 + w3). The workgroup is one wave: lane l
// holds virtual threads l, l + 64, l + 128 and l + 192.
__device__ void head_prologue(float *sxh, const float *__restrict__ x, int H, const float *__restrict__ gamma,
                              float eps) {
    const int lane = threadIdx.x;
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 0; base < H; base += 256) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int i = base + 64 * g + lane;
            if (i < H) {
                const float v = x[i];
                sxh[i] = v;
                s[g] = __fadd_rn(s[g], __fmul_rn(v, v));
            }
        }
    }
    if (gamma) {
        float w[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) w[g] = nc::wave_sum_f32(s[g]);
        const float total = __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
        const float rcp = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(total, (float)H), eps)));
        for (int i = lane; i < H; i += 64) sxh[i] = __fmul_rn(__fmul_rn(sxh[i], rcp), gamma[i]);
    }
    // (one wave: its own LDS writes land before its later reads)
}

// Row m's argmax key from this workgroup (one wave): the wave maximum, then
// either an atomic maximum into best[m] (slots == 0), or stored at
// best[m * slots + blockIdx.x] for the consumer to reduce (slots == gridDim.x:
// no atomics, whose same-address serialization costs 4-9 us over a head's
// workgroups, and nothing to clear beforehand).
__device__ __forceinline__ void publish_argmax(unsigned long long key, unsigned long long *best, int64_t m,
                                               int slots) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long other = __shfl_xor(key, off, 64);
        key = other > key ? other : key;
    }
    if (threadIdx.x != 0) return;
    if (slots == 0) {
        if (key != 0ull) atomicMax(best + m, key);
    } else {
        best[m * slots + blockIdx.x] = key;
    }
}

// logits[m, n] = acc, + bias[n] when given, and residual[m, n] + that when
// given (the reference's linear, nn.py:24-31, and its residual add): with a
// residual the output is usually the residual itself, updated in place.
__device__ __forceinline__ float head_epilogue(float acc, int64_t m, int64_t n, int64_t V,
                                               const float *__restrict__ bias, const float *residual) {
    if (bias) acc = __fadd_rn(acc, bias[n]);
    if (residual) acc = __fadd_rn(residual[(size_t)m * V + n], acc);
    return acc;
}

// One wave a workgroup, one block of 64 rows a wave: 2374 one-wave workgroups
// for the model's vocabulary spread over the 256 CUs at most 10 waves a CU,
// where workgroups of 4 waves left some CUs 12 (measured on MI355X: 91.1 us
// for V = 151936 with 4-wave workgroups, as long as V = 163840's 10 waves a
// CU, against 73.0 us for V = 131072's even 8).
__global__ __launch_bounds__(64) void lm_head(float *logits, unsigned long long *__restrict__ best,
                                              const float *__restrict__ x, const float4 *__restrict__ packed,
                                              int64_t V, int H, const float *__restrict__ gamma, float eps,
                                              const float *__restrict__ bias, const float *residual, int slots) {
    extern __shared__ float sxh[];
    const int m = blockIdx.y;
    head_prologue(sxh, x + (size_t)m * H, H, gamma, eps);
    const int lane = threadIdx.x;
    const int64_t blk = blockIdx.x;
    const int64_t n = blk * 64 + lane;
    const bool live = blk * 64 < V;
    const int k4n = H / 4;
    const float4 *e = packed + (live ? blk : 0) * k4n * 64 + lane;
    float acc = 0.0f;
#pragma unroll 16
    for (int k4 = 0; k4 < (live ? k4n : 0); ++k4) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(e + (size_t)k4 * 64));
        const float4 xv = *reinterpret_cast<const float4 *>(sxh + 4 * k4);
        acc = __fadd_rn(acc, __fmul_rn(xv.x, w.x));
        acc = __fadd_rn(acc, __fmul_rn(xv.y, w.y));
        acc = __fadd_rn(acc, __fmul_rn(xv.z, w.z));
        acc = __fadd_rn(acc, __fmul_rn(xv.w, w.w));
    }
    const bool valid = n < V;
    if (logits && valid) logits[(size_t)m * V + n] = head_epilogue(acc, m, n, V, bias, residual);
    if (best) publish_argmax(valid ? argmax_key(acc, n) : 0ull, best, m, slots);
}

// The same head for a width known at compile time, its loads kept in flight
// continuously: a ring of R 1-KB loads per wave, each refilled as soon as it is
// consumed (the loop is unrolled whole, so the compiler's waits count only the
// loads issued since), the first R issued before the x prologue. A loop that
// issues a batch of loads and then consumes it lets the batch drain to zero
// at every iteration, half its loads in flight on average.
template <int H, int R>
__global__ __launch_bounds__(64) void lm_head_ring(float *logits, unsigned long long *__restrict__ best,
                                                   const float *__restrict__ x, const float4 *__restrict__ packed,
                                                   int64_t V, const float *__restrict__ gamma, float eps,
                                                   const float *__restrict__ bias, const float *residual,
                                                   int slots) {
    static_assert(H % 4 == 0 && R <= H / 4, "ring of at most H / 4 loads");
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int K4 = H / 4;
    __shared__ __align__(16) float sxh[H];
    const int m = blockIdx.y;
    const int lane = threadIdx.x;
    const int64_t blk = blockIdx.x;
    const bool live = blk * 64 < V;
    const f32x4 *e = reinterpret_cast<const f32x4 *>(packed) + (live ? blk : 0) * K4 * 64 + lane;
    f32x4 ring[R];
#pragma unroll
    for (int i = 0; i < R; ++i) ring[i] = __builtin_nontemporal_load(e + (size_t)i * 64);
    head_prologue(sxh, x + (size_t)m * H, H, gamma, eps);
    float acc = 0.0f;
    if (live) {           // (a dead wave's ring read block 0: in bounds, unused)
#pragma unroll
        for (int k4 = 0; k4 < K4; ++k4) {
            const f32x4 w = ring[k4 % R];
            if (k4 + R < K4) ring[k4 % R] = __builtin_nontemporal_load(e + (size_t)(k4 + R) * 64);
            const float4 xv = *reinterpret_cast<const float4 *>(sxh + 4 * k4);
            acc = __fadd_rn(acc, __fmul_rn(xv.x, w.x));
            acc = __fadd_rn(acc, __fmul_rn(xv.y, w.y));
            acc = __fadd_rn(acc, __fmul_rn(xv.z, w.z));
            acc = __fadd_rn(acc, __fmul_rn(xv.w, w.w));
        }
    }
    const int64_t n = blk * 64 + lane;
    const bool valid = n < V;
    if (logits && valid) logits[(size_t)m * V + n] = head_epilogue(acc, m, n, V, bias, residual);
    if (best) publish_argmax(valid ? argmax_key(acc, n) : 0ull, best, m, slots);
}


__global__ void fill_u64(unsigned long long *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

__device__ __forceinline__ int64_t key_index(unsigned long long key) {
    return (int64_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

// The maximum of keys[0 .. slots - 1] in every thread of a 256-thread
// workgroup: each thread's share loaded 12 at a time, all in flight (one
// memory round trip for up to 3072 keys: the model's vocabulary leaves 2374).
__device__ unsigned long long reduce_keys(const unsigned long long *__restrict__ keys, int slots,
                                          unsigned long long *wkeys) {
    constexpr int kBatch = 12;
    unsigned long long k = 0ull;
    for (int base = 0; base < slots; base += kBatch * 256) {
        unsigned long long v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {       // (clamped, not guarded: a guarded load is a branch)
            const int i = base + threadIdx.x + 256 * u;
            const unsigned long long x = keys[min(i, slots - 1)];
            v[u] = i < slots ? x : 0ull;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) k = v[u] > k ? v[u] : k;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long other = __shfl_xor(k, off, 64);
        k = other > k ? other : k;
    }
    if ((threadIdx.x & 63) == 0) wkeys[threadIdx.x >> 6] = k;
    __syncthreads();
    k = wkeys[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) k = wkeys[i] > k ? wkeys[i] : k;
    return k;
}

__global__ void argmax_decode(int64_t *__restrict__ index, const unsigned long long *__restrict__ best, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) index[i] = key_index(best[i]);
}

// Row blockIdx.x's index from its per-workgroup keys.
__global__ __launch_bounds__(256) void argmax_reduce(int64_t *__restrict__ index,
                                                     const unsigned long long *__restrict__ best, int slots) {
    __shared__ unsigned long long wkeys[4];
    const unsigned long long k = reduce_keys(best + (size_t)blockIdx.x * slots, slots, wkeys);
    if (threadIdx.x == 0) index[blockIdx.x] = key_index(k);
}

}  // namespace

// p: [x f32[M,H], table f32[V,H], ids i64[M]];  s: [M, H, V]
NC_EXPORT int32_t nc_embed(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_embed: null operand");
    NC_REQUIRE(s[0] >= 0 && s[0] < (1 << 30) && s[1] > 0 && s[1] < (1 << 24) && s[2] > 0, "nc_embed: bad shape");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(embed_rows, dim3((unsigned)s[0]), dim3(256), 0, nc::stream(), (float *)p[0],
                       (const float *)p[1], (const int64_t *)p[2], (int)s[1], s[2], nc::error_word());
    return nc::launched("embed_rows");
}

// The LM head's packed table: p: [packed f32[ceil(V/64)*64, H], table f32[V,H]];  s: [V, H] (H % 4 == 0)
NC_EXPORT int32_t nc_pack_rows64(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1], "nc_pack_rows64: null operand");
    NC_REQUIRE(s[0] > 0 && s[1] > 0 && s[1] % 4 == 0 && s[1] < (1 << 20) && s[0] < (1LL << 31),
               "nc_pack_rows64: bad shape (H must be a multiple of 4)");
    hipLaunchKernelGGL(pack_rows64, dim3((unsigned)((s[0] + 63) / 64)), dim3(256), 0, nc::stream(), (float *)p[0],
                       (const float *)p[1], s[0], (int)s[1]);
    return nc::launched("pack_rows64");
}

// logits[m, n] = sum_k x[m, k] * table[n, k] in k order, and best[m] the
// argmax key of row m (atomic maximum: clear it first with nc_argmax_clear).
// With gamma (p[4]), x is rms-normed first with eps = s[3] (as float32 bits).
// With bias (p[5]) the sum is followed by + bias[n]; with residual (p[6]),
// logits = residual + that (the reference's float32 linear and residual add;
// the argmax, when asked for, is of the plain sums). With s[4] = 1 the argmax
// is left as one key per workgroup, best u64[M, G] with G = ceil(V / 64),
// for nc_argmax_index / nc_decode_advance to reduce (no atomics, no clear);
// with s[4] = 0, best u64[M] gets atomic maxima (clear it first).
// p: [logits f32[M,V] | NULL, best | NULL, x f32[M,H], packed table, gamma f32[H] | NULL,
//     bias f32[V] | NULL, residual f32[M,V] | NULL (may be logits itself)];
// s: [M, V, H, eps bits, key per workgroup 0 | 1]
NC_EXPORT int32_t nc_lm_head(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[2] && p[3] && (p[0] || p[1]), "nc_lm_head: null operand");
    NC_REQUIRE(p[0] || (!p[5] && !p[6]), "nc_lm_head: a bias or residual needs the logits output");
    const float *bias = (const float *)p[5], *residual = (const float *)p[6];
    NC_REQUIRE(s[0] >= 0 && s[0] < 65536 && s[1] > 0 && s[1] < (1LL << 31) && s[2] > 0 && s[2] % 4 == 0 &&
                   s[2] <= 16384,
               "nc_lm_head: bad shape (H a multiple of 4, at most 16384)");
    if (s[0] == 0) return NC_OK;
    NC_REQUIRE(s[4] == 0 || s[4] == 1, "nc_lm_head: s[4] must be 0 (one key per row) or 1 (a key per workgroup)");
    const int64_t blocks = (s[1] + 63) / 64;
    const dim3 grid((unsigned)blocks, (unsigned)s[0]);
    const int slots = s[4] ? (int)grid.x : 0;
    if (s[2] == 896) {       // the model's width: the ring kernel, 24 loads (24 KB) in flight per wave
        hipLaunchKernelGGL((lm_head_ring<896, 24>), grid, dim3(64), 0, nc::stream(), (float *)p[0],
                           (unsigned long long *)p[1], (const float *)p[2], (const float4 *)p[3], s[1],
                           (const float *)p[4], nc::bits_to_float(s[3]), bias, residual, slots);
        return nc::launched("lm_head_ring");
    }
    hipLaunchKernelGGL(lm_head, grid, dim3(64), (size_t)s[2] * sizeof(float), nc::stream(), (float *)p[0],
                       (unsigned long long *)p[1], (const float *)p[2], (const float4 *)p[3], s[1], (int)s[2],
                       (const float *)p[4], nc::bits_to_float(s[3]), bias, residual, slots);
    return nc::launched("lm_head");
}

// p: [best u64[n]];  s: [n]
NC_EXPORT int32_t nc_argmax_clear(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && s[0] >= 0 && s[0] < (1 << 24), "nc_argmax_clear: bad operand");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(fill_u64, dim3((unsigned)((s[0] + 255) / 256)), dim3(256), 0, nc::stream(),
                       (unsigned long long *)p[0], (int)s[0]);
    return nc::launched("fill_u64");
}

// p: [index i64[n], best u64[n] or u64[n, G]];  s: [n, G] (G = 0: one key per row; else the
// per-workgroup keys nc_lm_head leaves with s[4] = 1)
NC_EXPORT int32_t nc_argmax_index(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && s[0] >= 0 && s[0] < (1 << 24) && s[1] >= 0 && s[1] < (1 << 24),
               "nc_argmax_index: bad operand");
    if (s[0] == 0) return NC_OK;
    if (s[1] > 0) {
        hipLaunchKernelGGL(argmax_reduce, dim3((unsigned)s[0]), dim3(256), 0, nc::stream(), (int64_t *)p[0],
                           (const unsigned long long *)p[1], (int)s[1]);
        return nc::launched("argmax_reduce");
    }
    hipLaunchKernelGGL(argmax_decode, dim3((unsigned)((s[0] + 255) / 256)), dim3(256), 0, nc::stream(),
                       (int64_t *)p[0], (const unsigned long long *)p[1], (int)s[0]);
    return nc::launched("argmax_decode");
}

namespace {
// One greedy step's bookkeeping on the device: the argmax of the step just run
// becomes the next input token and is appended to the history at position
// pos + 1; pos advances; a single argmax key is cleared for the next step
// (per-workgroup keys, slots > 0, are reduced here and need no clearing). With
// x, the token's embedding row is gathered into x too (the next step's input,
// as nc_embed would: an id outside 0..V-1 records Fail code 1 and leaves x zero).
__global__ __launch_bounds__(256) void decode_advance(int64_t *__restrict__ ids, int64_t *__restrict__ tokens,
                                                      unsigned long long *__restrict__ best, int slots,
                                                      int64_t *__restrict__ pos, int64_t capacity,
                                                      float *__restrict__ x, const float *__restrict__ table, int H,
                                                      int64_t V, int32_t *__restrict__ error) {
    __shared__ unsigned long long wkeys[4];
    const int64_t p = *pos;
    if (p < -1 || p + 1 >= capacity) {
        if (threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_CAPACITY);
        return;
    }
    const int64_t token = key_index(slots > 0 ? reduce_keys(best, slots, wkeys) : best[0]);
    if (x) {
        const bool bad = token < 0 || token >= V;
        if (bad && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_INDEX);
        const float *row = table + (bad ? 0 : token) * (int64_t)H;
        for (int k = threadIdx.x; k < H; k += 256) x[k] = bad ? 0.0f : row[k];
    }
    __syncthreads();                              // every thread has read best before it is cleared
    if (threadIdx.x != 0) return;
    tokens[p + 1] = token;
    ids[0] = token;
    *pos = p + 1;
    if (slots == 0) best[0] = 0ull;
}
}  // namespace

// The greedy loop's step on the device (models/qwen2.py:362-367 does it on
// the host: argmax, append, feed back), so a captured decode step needs no
// host round trip.
// p: [ids i64[1], tokens i64[capacity], best u64[1] or u64[G], pos i64[1], x f32[H] | NULL,
//     table f32[V,H] | NULL];
// s: [capacity, H, V, G] (H and V read only with x; G = 0: one argmax key, else nc_lm_head's
//    per-workgroup keys)
NC_EXPORT int32_t nc_decode_advance(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && s[0] > 0 && s[3] >= 0 && s[3] < (1 << 24),
               "nc_decode_advance: bad operand");
    NC_REQUIRE(!p[4] || (p[5] && s[1] > 0 && s[1] < (1 << 24) && s[2] > 0), "nc_decode_advance: x needs the table");
    hipLaunchKernelGGL(decode_advance, dim3(1), dim3(256), 0, nc::stream(), (int64_t *)p[0], (int64_t *)p[1],
                       (unsigned long long *)p[2], (int)s[3], (int64_t *)p[3], s[0], (float *)p[4],
                       (const float *)p[5], p[4] ? (int)s[1] : 0, p[4] ? s[2] : 0, nc::error_word());
    return nc::launched("decode_advance");
}
