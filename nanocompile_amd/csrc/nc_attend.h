// Attention of one query over a chunk of at most 64 keys, by one wavefront:
// the unit that both the decode kernel and the prefill kernel are built from
// (a workgroup stages a chunk's keys and values in LDS once, and its waves
// attend every query head of the KV group, and every query row it holds, to
// it), so both compute the same bits, and the host oracle replays the same
// order.
//
// The order (models/qwen2.py:113-155 computes softmax(q K^T * scale) V; this
// is the split form of that softmax, each chunk normalised by its own max and
// the chunks combined after):
//
//   per chunk j of keys t = 64 j .. 64 j + n_j - 1:
//     s_t  = (a = 0; a = fma(q[d], k_t[d], a) in order of d) * scale + 0
//     m_j  = max_t s_t                       (NaN propagates)
//     p_t  = exp(s_t - m_j)
//     l_j  = sum_t p_t                       (wavefront butterfly, xor 32 .. 1, over 64 lanes, 0 past n_j)
//     o_j  = (o = 0; o = fma(p_t, v_t, o) in order of t)
//   over the chunks j = 0 .. J - 1, in order:
//     m    = max_j m_j
//     w_j  = exp(m_j - m)
//     L    = sum_j l_j * w_j,   O = sum_j o_j * w_j   (in order of j, from +0)
//     out  = O / L
//
// Each fma rounds once, every other multiply and add rounds once
// (-ffp-contract=off forms no other fused operation); exp is nc_expf.
// The chunk results (m_j, l_j, o_j) of a query travel between the two
// kernels as D + 2 floats: m_j, l_j, o_j[0 .. D - 1].
#pragma once

#include "nc_common.h"
#include "nc_math.h"

namespace nc {

constexpr int kChunk = 64;    // keys per chunk: one per lane of a wavefront

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// A chunk staged in LDS: key rows padded to D + 4 floats (so 16-byte reads of
// consecutive rows hit distinct banks), then value rows of D floats.
template <int D>
struct Staged {
    static constexpr int kKeyStride = D + 4;
    static constexpr int kFloats = kChunk * (D + 4) + kChunk * D;
    float *keys, *values;
    __device__ __forceinline__ explicit Staged(float *lds) : keys(lds), values(lds + kChunk * (D + 4)) {}
};

// Keys and values t0 .. t0 + 63 of one KV head (rows clamped to last_row),
// loaded by the workgroup's NT threads, coalesced, 16 bytes a thread a load.
// issue() starts the loads, so a caller can overlap them with other work;
// store() writes them to LDS, rows from `valid` on as zeros (the rows past the
// context: whatever the cache holds there must not reach a product) and row
// `skip` (-1: none) left for the caller.
template <int D, int NT>
struct ChunkLoad {
    static constexpr int kRow4 = D / 4;                     // float4 per row
    static constexpr int kTotal = kChunk * kRow4;
    static constexpr int kIters = (kTotal + NT - 1) / NT;
    float4 k[kIters], v[kIters];

    __device__ __forceinline__ void issue(const float *__restrict__ K, const float *__restrict__ V, int t0,
                                          int last_row) {
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int u = threadIdx.x + it * NT;
            const int row = u / kRow4, col = (u % kRow4) * 4;
            const size_t at = (size_t)min(t0 + row, last_row) * D + col;
            if (kTotal % NT == 0 || u < kTotal) {
                k[it] = *reinterpret_cast<const float4 *>(K + at);
                v[it] = *reinterpret_cast<const float4 *>(V + at);
            }
        }
    }

    // (selects per component: a float4-wide select is lowered through scratch)
    static __device__ __forceinline__ float4 keep_if(bool in, const float4 &x) {
        return make_float4(in ? x.x : 0.0f, in ? x.y : 0.0f, in ? x.z : 0.0f, in ? x.w : 0.0f);
    }

    __device__ __forceinline__ void store(const Staged<D> &st, int skip, int valid) const {
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int u = threadIdx.x + it * NT;
            const int row = u / kRow4, col = (u % kRow4) * 4;
            if ((kTotal % NT == 0 || u < kTotal) && row != skip) {
                const bool in = row < valid;
                *reinterpret_cast<float4 *>(st.keys + row * Staged<D>::kKeyStride + col) = keep_if(in, k[it]);
                *reinterpret_cast<float4 *>(st.values + row * D + col) = keep_if(in, v[it]);
            }
        }
    }
};

// The maximum of a chunk's scores over the wavefront, as a butterfly of
// nan_max would give it: scores are never -0 (s * scale + 0 is +0 for any
// zero), so plain compares give the maximum of the finite and infinite ones,
// and a NaN in any lane (one ballot) makes the result NaN.
__device__ __forceinline__ float scores_max(float s) {
    float m = butterfly<64>(s, [](float a, float b) { return a < b ? b : a; });
    m = lane_value(m, 0);
    return __ballot(s != s) ? __builtin_nanf("") : m;
}

struct ChunkResult {
    float m, l, o;    // the chunk's max and sum (every lane), and o[d] in lane d
};

// The two halves of attending one query to the first n keys of a staged
// chunk whose rows past the context are zeros. The whole wavefront must call
// each together; the chunk must be staged (and a barrier passed) before.
//
// chunk_scores: s_t, m, p_t = exp(s_t - m) and l from q (D floats in LDS,
// read by every lane); p_t goes to p[t] (64 floats of LDS owned by the wave,
// which may be q itself: every read of q comes before the write).
template <int D>
__device__ __forceinline__ void chunk_scores(const float *q, const Staged<D> &st, int n, float scale, float *p,
                                             float &m_out, float &l_out) {
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    const float *krow = st.keys + lane * Staged<D>::kKeyStride;
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
        const float4 k = *reinterpret_cast<const float4 *>(krow + 4 * i);
        const float4 qi = *reinterpret_cast<const float4 *>(q + 4 * i);
        acc = __builtin_fmaf(qi.x, k.x, acc);
        acc = __builtin_fmaf(qi.y, k.y, acc);
        acc = __builtin_fmaf(qi.z, k.z, acc);
        acc = __builtin_fmaf(qi.w, k.w, acc);
    }
    const float s = lane < n ? __fadd_rn(__fmul_rn(acc, scale), 0.0f) : -__builtin_inff();
    const float m = scores_max(s);
    const float pt = nc_expf(__fsub_rn(s, m));       // exp(-inf) = 0 for lanes past the chunk
    l_out = wave_sum_f32(pt);
    m_out = m;
    p[lane] = pt;
}

// chunk_values: o[d] in key order from the p_t that chunk_scores left in LDS
// (the wave's own write lands before its reads), four at a time. A key past n
// has p = 0, and fma(0, v, o) = o + (+-0) = o exactly (v a real key, masked,
// or a zero row; o starts at +0 and is never -0).
template <int D>
__device__ __forceinline__ float chunk_values(const float *p, const Staged<D> &st) {
    const int lane = threadIdx.x & 63;
    const int dl = lane < D ? lane : 0;
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kChunk / 4; ++i) {
        const float4 pi = *reinterpret_cast<const float4 *>(p + 4 * i);
        o = __builtin_fmaf(pi.x, st.values[(4 * i + 0) * D + dl], o);
        o = __builtin_fmaf(pi.y, st.values[(4 * i + 1) * D + dl], o);
        o = __builtin_fmaf(pi.z, st.values[(4 * i + 2) * D + dl], o);
        o = __builtin_fmaf(pi.w, st.values[(4 * i + 3) * D + dl], o);
    }
    return o;
}

// Both halves for one query, with `pbuf` (64 floats of LDS owned by the
// calling wave) holding the p_t between them.
template <int D>
__device__ __forceinline__ ChunkResult attend_staged(const float *q, const Staged<D> &st, int n, float scale,
                                                     float *pbuf) {
    ChunkResult r;
    chunk_scores<D>(q, st, n, scale, pbuf, r.m, r.l);
    r.o = chunk_values<D>(pbuf, st);
    return r;
}

// The same two halves for H queries at once, each in the order above: the
// products run d (or key) outermost and query innermost, so each key or value
// element is read from LDS once for the H chains and neither the key row nor
// the value column stays in registers. qp[u] holds query u (D floats) and
// receives its p_t.
template <int D, int H>
__device__ __forceinline__ void chunk_scores_n(float (*qp)[kChunk], const Staged<D> &st, int n, float scale,
                                               float (&m)[H], float (&l)[H]) {
    const int lane = threadIdx.x & 63;
    float acc[H];
#pragma unroll
    for (int u = 0; u < H; ++u) acc[u] = 0.0f;
    const float *krow = st.keys + lane * Staged<D>::kKeyStride;
#pragma unroll 2
    for (int i = 0; i < D / 4; ++i) {
        const float4 k = *reinterpret_cast<const float4 *>(krow + 4 * i);
#pragma unroll
        for (int u = 0; u < H; ++u) {
            const float4 qi = *reinterpret_cast<const float4 *>(qp[u] + 4 * i);
            acc[u] = __builtin_fmaf(qi.x, k.x, acc[u]);
            acc[u] = __builtin_fmaf(qi.y, k.y, acc[u]);
            acc[u] = __builtin_fmaf(qi.z, k.z, acc[u]);
            acc[u] = __builtin_fmaf(qi.w, k.w, acc[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < H; ++u) {
        const float s = lane < n ? __fadd_rn(__fmul_rn(acc[u], scale), 0.0f) : -__builtin_inff();
        const float mu = scores_max(s);
        const float pt = nc_expf(__fsub_rn(s, mu));
        l[u] = wave_sum_f32(pt);
        m[u] = mu;
        qp[u][lane] = pt;
    }
}

// chunk_scores_n with the queries read from global memory at a wave-uniform
// address, query u at q + u D (q wave-uniform, the memory unchanged while the
// kernel runs): scalar loads bring them to SGPRs, so each product reads one
// operand from LDS (the key, once for the H chains) instead of also a 16-byte
// broadcast of the query per head. The same chains in the same order; the
// probabilities go to p[u].
template <int D, int H>
__device__ __forceinline__ void chunk_scores_sq(const float *__restrict__ q, float (*p)[kChunk], const Staged<D> &st,
                                                int n, float scale, float (&m)[H], float (&l)[H]) {
    const int lane = threadIdx.x & 63;
    float acc[H];
#pragma unroll
    for (int u = 0; u < H; ++u) acc[u] = 0.0f;
    const float *krow = st.keys + lane * Staged<D>::kKeyStride;
#pragma unroll 2
    for (int i = 0; i < D / 4; ++i) {
        const float4 k = *reinterpret_cast<const float4 *>(krow + 4 * i);
#pragma unroll
        for (int u = 0; u < H; ++u) {
            const float4 qi = *reinterpret_cast<const float4 *>(q + u * D + 4 * i);
            acc[u] = __builtin_fmaf(qi.x, k.x, acc[u]);
            acc[u] = __builtin_fmaf(qi.y, k.y, acc[u]);
            acc[u] = __builtin_fmaf(qi.z, k.z, acc[u]);
            acc[u] = __builtin_fmaf(qi.w, k.w, acc[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < H; ++u) {
        const float s = lane < n ? __fadd_rn(__fmul_rn(acc[u], scale), 0.0f) : -__builtin_inff();
        const float mu = scores_max(s);
        const float pt = nc_expf(__fsub_rn(s, mu));
        l[u] = wave_sum_f32(pt);
        m[u] = mu;
        p[u][lane] = pt;
    }
}

// (keys from n on have p = 0 and leave the accumulators unchanged, so the key
// loop stops at the first group of four that holds none of the n keys)
template <int D, int H>
__device__ __forceinline__ void chunk_values_n(float (*qp)[kChunk], const Staged<D> &st, int n, float (&o)[H]) {
    const int lane = threadIdx.x & 63;
    const int dl = lane < D ? lane : 0;
#pragma unroll
    for (int u = 0; u < H; ++u) o[u] = 0.0f;
    const int groups = (n + 3) >> 2;
#pragma unroll 2
    for (int i = 0; i < groups; ++i) {
        const float v0 = st.values[(4 * i + 0) * D + dl], v1 = st.values[(4 * i + 1) * D + dl];
        const float v2 = st.values[(4 * i + 2) * D + dl], v3 = st.values[(4 * i + 3) * D + dl];
#pragma unroll
        for (int u = 0; u < H; ++u) {
            const float4 pi = *reinterpret_cast<const float4 *>(qp[u] + 4 * i);
            o[u] = __builtin_fmaf(pi.x, v0, o[u]);
            o[u] = __builtin_fmaf(pi.y, v1, o[u]);
            o[u] = __builtin_fmaf(pi.z, v2, o[u]);
            o[u] = __builtin_fmaf(pi.w, v3, o[u]);
        }
    }
}

// Store a chunk result at part[0 .. D + 1] (m_j, l_j, o_j).
template <int D>
__device__ __forceinline__ void keep_result(float *part, const ChunkResult &r) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) {
        part[0] = r.m;
        part[1] = r.l;
    }
    if (lane < D) part[2 + lane] = r.o;
}

// The combine over chunks 0 .. J - 1 for lane d: partial j is m_j = at(j, 0),
// l_j = at(j, 1), o_j[d] = at(j, 2 + d). The weights w_j are computed 64 at a
// time, one per lane, then the sums run in order of j. The whole wavefront
// must call this together.
template <typename At>
__device__ __forceinline__ float combine_chunks(int J, int dl, At at) {
    const int lane = threadIdx.x & 63;
    float m = -__builtin_inff();
    for (int j = 0; j < J; ++j) m = nan_max(m, at(j, 0));
    float L = 0.0f, O = 0.0f;
    for (int j0 = 0; j0 < J; j0 += 64) {
        const float w = j0 + lane < J ? nc_expf(__fsub_rn(at(j0 + lane, 0), m)) : 0.0f;
        const int end = min(64, J - j0);
        for (int j = 0; j < end; ++j) {
            const float wj = lane_value(w, j);
            L = __fadd_rn(L, __fmul_rn(at(j0 + j, 1), wj));
            O = __fadd_rn(O, __fmul_rn(at(j0 + j, 2 + dl), wj));
        }
    }
    return div_rn(O, L);
}

}  // namespace nc
