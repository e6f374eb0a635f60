// Attention of one query over a chunk of at most 64 keys, by one wavefront:
// the unit that both the decode kernel (one workgroup per chunk, so a long
// context spreads over many CUs) and the prefill kernel (a workgroup's four
// waves taking turns through the chunks) are built from, so both compute the
// same bits, and the host oracle replays the same order.
//
// The order (models/qwen2.py:113-155 computes softmax(q K^T * scale) V; this
// is the split form of that softmax, each chunk normalised by its own max and
// the chunks combined after):
//
//   per chunk j of keys t = 64 j .. 64 j + n_j - 1:
//     s_t  = (sum_d q[d] * k_t[d], in order of d) * scale + 0
//     m_j  = max_t s_t                       (NaN propagates)
//     p_t  = exp(s_t - m_j)
//     l_j  = sum_t p_t                       (wavefront butterfly, xor 32 .. 1, over 64 lanes, 0 past n_j)
//     o_j  = sum_t p_t * v_t                 (in order of t, from +0)
//   over the chunks j = 0 .. J - 1, in order:
//     m    = max_j m_j
//     w_j  = exp(m_j - m)
//     L    = sum_j l_j * w_j,   O = sum_j o_j * w_j   (in order of j, from +0)
//     out  = O / L
//
// Every multiply and add rounds once (-ffp-contract=off); exp is nc_expf.
#pragma once

#include "nc_common.h"
#include "nc_math.h"

namespace nc {

constexpr int kChunk = 64;    // keys per chunk: one per lane of a wavefront

__device__ __forceinline__ float nan_max(float a, float b) { return (a < b || b != b) ? b : a; }

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

struct ChunkResult {
    float m, l, o;    // the chunk's max and sum (every lane), and o[d] in lane d
};

// One chunk's keys and values in registers: lane l holds key row t0 + l and,
// for each of the chunk's keys i, value v[t0 + i][d] for its d = l. Loads
// are issued in the constructor, from addresses clamped into the chunk (rows
// past it, and the row `fresh`, are read at t0 and never used), so a caller
// can start them early and overlap their latency with other work. With
// FRESH, key `fresh` (when in the chunk) is taken from knew / vnew instead of
// the cache: the decode kernel's new key, whose cache row another workgroup
// may be writing.
template <int D, bool FRESH>
struct Chunk {
    static_assert(D % 4 == 0 && D <= 64, "head_dim");
    float4 k[D / 4];
    float v[kChunk];
    int t0, n, fresh;

    __device__ __forceinline__ Chunk(const float *__restrict__ K, const float *__restrict__ V, int t0_, int n_,
                                     int fresh_)
        : t0(t0_), n(n_), fresh(FRESH ? fresh_ : -1) {
        const int lane = threadIdx.x & 63;
        const int dl = lane < D ? lane : 0;
        const int t = t0 + lane;
        const float *krow = K + (size_t)(lane < n && t != fresh ? t : t0) * D;
#pragma unroll
        for (int i = 0; i < D / 4; ++i) k[i] = reinterpret_cast<const float4 *>(krow)[i];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int ti = t0 + i;
            v[i] = V[(size_t)(i < n && ti != fresh ? ti : t0) * D + dl];
        }
    }

    // Attend q (rotated, D floats readable by every lane, e.g. in LDS). The
    // whole wavefront must call this together.
    __device__ __forceinline__ ChunkResult attend(const float *q, const float *knew, const float *vnew,
                                                  float scale) const {
        const int lane = threadIdx.x & 63;
        const int dl = lane < D ? lane : 0;
        const bool mine = t0 + lane == fresh;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 4; ++i) {
            float4 kk = k[i];
            if constexpr (FRESH) {      // per component: a select of whole float4s goes through scratch
                const float4 f = reinterpret_cast<const float4 *>(knew)[i];
                kk.x = mine ? f.x : kk.x;
                kk.y = mine ? f.y : kk.y;
                kk.z = mine ? f.z : kk.z;
                kk.w = mine ? f.w : kk.w;
            }
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 0], kk.x));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 1], kk.y));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 2], kk.z));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 3], kk.w));
        }
        const float s = lane < n ? __fadd_rn(__fmul_rn(acc, scale), 0.0f) : -__builtin_inff();
        float m = s;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = nan_max(m, __shfl_xor(m, off, 64));
        m = lane_value(m, 0);
        const float p = nc_expf(__fsub_rn(s, m));        // exp(-inf) = 0 for lanes past the chunk
        const float l = wave_sum_f32(p);

        // o[d] in key order. A key past the chunk adds 0 * 0 = +0 to an
        // accumulator that starts at +0 and is never -0: exact, no change.
        float vf = 0.0f;
        if constexpr (FRESH) vf = vnew[dl];
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const bool in = i < n;
            const float pi = lane_value(p, i);
            float vi = v[i];
            if constexpr (FRESH) vi = t0 + i == fresh ? vf : vi;
            o = __fadd_rn(o, __fmul_rn(in ? pi : 0.0f, in ? vi : 0.0f));
        }
        return {m, l, o};
    }
};

// The combine over chunks 0 .. J - 1 for lane d: partial j is m_j = at(j, 0),
// l_j = at(j, 1), o_j[d] = at(j, 2 + d).
template <typename At>
__device__ __forceinline__ float combine_chunks(int J, int dl, At at) {
    float m = -__builtin_inff();
    for (int j = 0; j < J; ++j) m = nan_max(m, at(j, 0));
    float L = 0.0f, O = 0.0f;
    for (int j = 0; j < J; ++j) {
        const float w = nc_expf(__fsub_rn(at(j, 0), m));
        L = __fadd_rn(L, __fmul_rn(at(j, 1), w));
        O = __fadd_rn(O, __fmul_rn(at(j, 2 + dl), w));
    }
    return div_rn(O, L);
}

}  // namespace nc
