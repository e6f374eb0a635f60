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
#include "nc_attend.h"
#include "nc_epilogue.h"

namespace {

using nc::i8x16;
constexpr int kL = 8;                  // lanes per weight row: 8 x 16 B = one 128-byte line per load

enum Prologue { kNorm = 0, kQuant = 1 };
enum Epilogue { kBias = 0, kResidual = 1, kSwiglu = 2 };

// The activation row x[K] (f32) to int8 in LDS; returns its scale. NORM
// applies rms_norm first (rms_norm(x) * gamma, eps). The workgroup's W waves
// share the work: thread t of 64 W holds elements t, t + 64 W, ... With W = 4
// the threads are the row-sum order's 256 virtual threads themselves; with
// W = 1 lane l holds virtual threads l, l + 64, l + 128, l + 192. Either way
// the sum of squares is the row kernels' (nc_quant.hip) bit for bit.
template <int K, int PRO, int W>
__device__ float activation_prologue(int8_t *__restrict__ sxq, const float *__restrict__ x,
                                     const float *__restrict__ gamma, float eps, float *scratch) {
    static_assert(W == 1 || W == 4, "one wave, or the row order's 256 threads");
    constexpr int T = 64 * W;
    constexpr int PER = (K + T - 1) / T;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int k = tid + T * i;
        v[i] = (K % T == 0 || k < K) ? x[k] : 0.0f;
    }
    if constexpr (PRO == kNorm) {
        float ss;
        if constexpr (W == 1) {
            float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};      // virtual threads lane + 64 g, g = 0..3
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int k = lane + 64 * i;
                if (K % 64 == 0 || k < K) s[i & 3] = __fadd_rn(s[i & 3], __fmul_rn(v[i], v[i]));
            }
            float w[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) w[g] = nc::wave_sum_f32(s[g]);
            ss = __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
        } else {
            float s = 0.0f;                             // virtual thread tid
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int k = tid + T * i;
                if (K % T == 0 || k < K) s = __fadd_rn(s, __fmul_rn(v[i], v[i]));
            }
            s = nc::wave_sum_f32(s);
            if (lane == 0) scratch[wave] = s;
            __syncthreads();
            ss = __fadd_rn(__fadd_rn(scratch[0], scratch[1]), __fadd_rn(scratch[2], scratch[3]));
            __syncthreads();
        }
        const float rcp = nc::div_rn(1.0f, nc::sqrt_rn(__fadd_rn(nc::div_rn(ss, (float)K), eps)));
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = tid + T * i;
            if (K % T == 0 || k < K) v[i] = __fmul_rn(__fmul_rn(v[i], rcp), gamma[k]);
        }
    }
    float mag = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) mag = fmaxf(mag, fabsf(v[i]));
    mag = nc::wave_max_f32(mag);
    if constexpr (W > 1) {
        if (lane == 0) scratch[4 + wave] = mag;
        __syncthreads();
        mag = fmaxf(fmaxf(scratch[4], scratch[5]), fmaxf(scratch[6], scratch[7]));
    }
    const float scale = nc::token_scale(mag);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int k = tid + T * i;
        if (K % T == 0 || k < K) sxq[k] = nc::quantize_value(v[i], scale);
    }
    __syncthreads();
    return scale;
}

template <int K, int L>
struct RowChunks {
    static constexpr int STEP = L * 16;
    static constexpr int ITERS = K / STEP;
    static_assert(K % STEP == 0, "K must be a multiple of 16 L");
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

// One decode projection: W waves a workgroup, 64 / L rows a wave (row pairs
// for SwiGLU), L lanes per row. The weight loads are issued first, so they
// are in flight while the workgroup computes its activation prologue, which
// its W waves share.
template <int K, int PRO, int EPI, int L, int W>
__global__ __launch_bounds__(64 * W) void gemv_decode(float *__restrict__ out, const float *__restrict__ x,
                                                      const float *__restrict__ gamma, float eps,
                                                      const int8_t *__restrict__ q, const float *__restrict__ ws,
                                                      const float *__restrict__ bias, const int8_t *__restrict__ q2,
                                                      const float *__restrict__ ws2, int N) {
    __shared__ __align__(16) int8_t sxq[K];
    __shared__ float scratch[8];
    const int lane = threadIdx.x & 63, sub = lane & (L - 1);
    const int n = blockIdx.x * (W * 64 / L) + (threadIdx.x >> 6) * (64 / L) + lane / L;
    const bool valid = n < N;
    const int nr = valid ? n : 0;
    RowChunks<K, L> w1, w2;
    w1.load(q + (size_t)nr * K, sub);
    if constexpr (EPI == kSwiglu) w2.load(q2 + (size_t)nr * K, sub);
    const float xs = activation_prologue<K, PRO, W>(sxq, x, gamma, eps, scratch);
    int32_t acc = w1.dot(sxq, sub);
    int32_t acc2 = 0;
    if constexpr (EPI == kSwiglu) acc2 = w2.dot(sxq, sub);
    acc = nc::group_sum_i32<L>(acc);
    if constexpr (EPI == kSwiglu) acc2 = nc::group_sum_i32<L>(acc2);
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
//
// One workgroup per query head, kWaves wavefronts: wave w attends the head to
// the 64-key chunks w, w + kWaves, ... (nc_attend.h gives the order), leaves
// each chunk's partial result in LDS, and wave 0 combines them. Up to
// 64 * kWaves keys every chunk is in flight at once; the chunk loads go out
// before RoPE, which overlaps their latency. The same order as
// nc_attention's prefill kernel, so a decode step and a prefill agree bit for
// bit. (Splitting a head over several workgroups instead costs device-scope
// fences or a second launch to combine, more than the keys take to read at
// these lengths.)
constexpr int kWaves = 4;

template <int D, bool TABLE>
__global__ __launch_bounds__(64 * kWaves) void attention_decode(
    float *__restrict__ ctx, const float *__restrict__ qkv, float *__restrict__ kcache, float *__restrict__ vcache,
    const float *__restrict__ inv_freq, int heads, int kv_heads, int past, int capacity, float scale,
    const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error, const float *__restrict__ table) {
    if (pos_ptr) {
        const int64_t p = *pos_ptr;
        if (p < 0 || p + 1 > capacity) {
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicCAS(error, 0, NC_FAIL_CAPACITY);
            return;
        }
        past = (int)p;
    }
    extern __shared__ __align__(16) float lds[];  // [kWaves][chunk stage], then [J][D + 2]: m_j, l_j, o_j[D]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *stage = lds + wave * nc::chunk_stage_floats<D>();
    float *part = lds + kWaves * nc::chunk_stage_floats<D>();
    __shared__ __align__(16) float rotated[kWaves][3 * D];     // per wave: q, the new key, the new value
    float *q = rotated[wave], *knew = q + D, *vnew = q + 2 * D;
    constexpr int half = D / 2;
    const int h = blockIdx.x, group = heads / kv_heads, g = h / group;
    const int T = past + 1, J = (T + nc::kChunk - 1) / nc::kChunk;
    float *K = kcache + (size_t)g * capacity * D;
    float *V = vcache + (size_t)g * capacity * D;

    // every wave's first chunk (clamped to the last for waves past J) loads now
    const int j0 = min(wave, J - 1), t0 = j0 * nc::kChunk;
    nc::Chunk<D, true> chunk(K, V, t0, min(nc::kChunk, T - t0), past, capacity - 1);

    // Each wave rotates its own copy of q (lanes 0 .. half - 1) and of the new
    // key (lanes half .. D - 1), so no workgroup barrier separates the loads
    // above from their use: cos and sin of f32(past) * inv_freq[i] from the
    // cache's table (nc_rope_table) when given, else computed here, the same
    // nc_cosf / nc_sinf either way. A wave's LDS writes complete before its
    // own later reads.
    if (lane < D) {
        const float *qrow = qkv + h * D;
        const float *krow = qkv + heads * D + g * D;
        const float *vrow = qkv + (heads + kv_heads) * D + g * D;
        const int i = lane < half ? lane : lane - half;
        const float *x = lane < half ? qrow : krow;
        float *y = lane < half ? q : knew;
        float c, s;
        if constexpr (TABLE) {
            c = table[(size_t)past * half + i];
            s = table[((size_t)capacity + past) * half + i];
        } else {
            const float ang = __fmul_rn((float)past, inv_freq[i]);
            c = nc_cosf(ang);
            s = nc_sinf(ang);
        }
        const float x0 = x[i], x1 = x[i + half];
        y[i] = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
        y[i + half] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
        vnew[lane] = vrow[lane];
    }
    auto keep = [&](int j, const nc::ChunkResult &r) {
        float *pj = part + j * (D + 2);
        if (lane == 0) {
            pj[0] = r.m;
            pj[1] = r.l;
        }
        if (lane < D) pj[2 + lane] = r.o;
    };
    if (wave < J) keep(wave, chunk.attend(q, knew, vnew, scale, stage));
    for (int j = wave + kWaves; j < J; j += kWaves) {      // contexts past 64 * kWaves keys
        const int tj = j * nc::kChunk;
        nc::Chunk<D, true> more(K, V, tj, min(nc::kChunk, T - tj), past, capacity - 1);
        keep(j, more.attend(q, knew, vnew, scale, stage));
    }
    // The cache row of the new key, written after the chunks are read: no
    // workgroup reads it (the chunk holding it takes knew / vnew), and a
    // store through the cache pointer before the reads would make the
    // compiler keep the chunk's registers in scratch (a generic pointer may
    // alias them).
    if (wave == 0 && h % group == 0 && lane < D) {
        K[(size_t)past * D + lane] = knew[lane];
        V[(size_t)past * D + lane] = vnew[lane];
    }
    __syncthreads();
    if (wave == 0) {
        const float out = nc::combine_chunks(J, lane < D ? lane : 0,
                                             [&](int c, int k) { return part[c * (D + 2) + k]; });
        if (lane < D) ctx[h * D + lane] = out;
    }
}

float bits_to_float(int64_t bits) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)bits;
    return c.f;
}

// Lanes per row: 8 (one 128-byte line per load), or 16 for the long down
// projection (half the loads each). Waves per workgroup: 1, or 4 for the long
// down projection, whose 4864-wide prologue would otherwise cost each lane 76
// correctly rounded divisions (measured on MI355X: 7.3 us with one wave,
// 5.4 us with four; the 896-wide projections are faster with one).
template <int K, int PRO, int EPI, int L = (K >= 4096 ? 16 : kL), int W = (K >= 4096 ? 4 : 1)>
int32_t launch_decode(void **p, int N, float eps) {
    constexpr int ROWS = W * 64 / L;
    hipLaunchKernelGGL((gemv_decode<K, PRO, EPI, L, W>), dim3((N + ROWS - 1) / ROWS), dim3(64 * W), 0, nc::stream(),
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

namespace {

template <int D, bool TABLE>
int32_t launch_attention_decode(void **p, const int64_t *s, const int64_t *pos) {
    static bool raised = false;          // chunk stages (70 KB) + partials of 256 chunks (67.6 KB)
    if (!raised) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attention_decode<D, TABLE>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024) != hipSuccess) {
            nc::set_message("nc_attention_decode: could not raise the LDS limit");
            return NC_LAUNCH_FAILED;
        }
        raised = true;
    }
    const int64_t cap = s[4];
    const size_t lds = ((size_t)kWaves * nc::chunk_stage_floats<D>() +
                        (size_t)((cap + nc::kChunk - 1) / nc::kChunk) * (D + 2)) * sizeof(float);
    hipLaunchKernelGGL((attention_decode<D, TABLE>), dim3((unsigned)s[0]), dim3(64 * kWaves), lds, nc::stream(),
                       (float *)p[0], (const float *)p[1], (float *)p[2], (float *)p[3], (const float *)p[4],
                       (int)s[0], (int)s[1], pos ? 0 : (int)s[3], (int)cap, bits_to_float(s[5]), pos,
                       nc::error_word(), (const float *)p[6]);
    return nc::launched("attention_decode");
}

}  // namespace

// Attention of one new token with RoPE and the cache append fused in.
// p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated, with bias), kcache f32[kv,C,D],
//     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] | NULL, rope table f32[2,C,D/2] | NULL];
// s: [heads, kv, D, past, C, scale as float32 bits]  (D 64 or 32, C <= 16384; past read from pos when given)
NC_EXPORT int32_t nc_attention_decode(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_attention_decode: null operand");
    const int64_t heads = s[0], kv = s[1], D = s[2], past = s[3], cap = s[4];
    const int64_t *pos = (const int64_t *)p[5];
    NC_REQUIRE(heads > 0 && kv > 0 && heads % kv == 0 && heads < 65536 && (D == 64 || D == 32) && cap > 0 &&
                   cap <= 16384 && (pos || (past >= 0 && past + 1 <= cap)),
               "nc_attention_decode: bad shape (head_dim 64 or 32, capacity at most 16384)");
    if (p[6]) return D == 64 ? launch_attention_decode<64, true>(p, s, pos) : launch_attention_decode<32, true>(p, s, pos);
    return D == 64 ? launch_attention_decode<64, false>(p, s, pos) : launch_attention_decode<32, false>(p, s, pos);
}


