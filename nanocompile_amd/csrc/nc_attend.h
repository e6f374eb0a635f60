// Attention of one query over a chunk of at most 64 keys, by one wavefront:
// the unit that both the decode kernel (a workgroup's waves taking a head's
// chunks) and the prefill kernel (the same, per query row) are built from, so
// both compute the same bits, and the host oracle replays the same order.
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

// LDS floats one wave needs to turn its chunk's key rows around (rows padded
// by 4 floats, so 16-byte reads of consecutive rows hit distinct banks).
template <int D>
constexpr int chunk_stage_floats() { return kChunk * (D + 4); }

struct ChunkResult {
    float m, l, o;    // the chunk's max and sum (every lane), and o[d] in lane d
};

// One chunk's keys and values: the key rows loaded coalesced (D / 4 lanes
// per row, 16 bytes each) and turned around through LDS so lane l holds key
// row t0 + l; for each key i, value v[t0 + i][d] for the lane's d = l. Loads
// are issued in the constructor, rows clamped to the cache's last row (rows
// past the chunk are never used), so a caller can start them early. With
// FRESH, key `fresh` (the last key of the context, when in this chunk) comes
// from knew / vnew instead of the cache: the decode kernel's new key, whose
// cache row another workgroup may be writing.
template <int D, bool FRESH>
struct Chunk {
    static_assert(D % 4 == 0 && D <= 64 && 256 % D == 0, "head_dim");
    static constexpr int kLanesPerRow = D / 4;
    static constexpr int kRowsPerLoad = 64 / kLanesPerRow;
    float4 kc[D / 4];          // coalesced: load r holds row r * kRowsPerLoad + lane / kLanesPerRow
    float v[kChunk];
    int t0, n, fresh;

    __device__ __forceinline__ Chunk(const float *__restrict__ K, const float *__restrict__ V, int t0_, int n_,
                                     int fresh_, int last_row)
        : t0(t0_), n(n_), fresh(FRESH ? fresh_ : -1) {
        const int lane = threadIdx.x & 63;
        const int dl = lane < D ? lane : 0;
        const int col = (lane % kLanesPerRow) * 4;
#pragma unroll
        for (int r = 0; r < D / 4; ++r) {
            const int row = min(t0 + r * kRowsPerLoad + lane / kLanesPerRow, last_row);
            kc[r] = *reinterpret_cast<const float4 *>(K + (size_t)row * D + col);
        }
#pragma unroll
        for (int i = 0; i < kChunk; ++i) v[i] = V[(size_t)min(t0 + i, last_row) * D + dl];
    }

    // Attend q (rotated, D floats readable by every lane, e.g. in LDS), using
    // `stage` (chunk_stage_floats<D>() floats of LDS owned by this wave). The
    // whole wavefront must call this together.
    __device__ __forceinline__ ChunkResult attend(const float *q, const float *knew, const float *vnew, float scale,
                                                  float *stage) const {
        const int lane = threadIdx.x & 63;
        const int dl = lane < D ? lane : 0;
        constexpr int P = D + 4;
#pragma unroll
        for (int r = 0; r < D / 4; ++r) {
            const int row = r * kRowsPerLoad + lane / kLanesPerRow;
            *reinterpret_cast<float4 *>(stage + row * P + (lane % kLanesPerRow) * 4) = kc[r];
        }
        // (the wave's own LDS writes complete before its reads: in order, no barrier)
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 4; ++i) {
            const float4 k = *reinterpret_cast<const float4 *>(stage + lane * P + 4 * i);
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 0], k.x));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 1], k.y));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 2], k.z));
            acc = __fadd_rn(acc, __fmul_rn(q[4 * i + 3], k.w));
        }
        const bool has_fresh = FRESH && fresh >= t0 && fresh < t0 + n;   // uniform; then fresh = t0 + n - 1
        if (has_fresh) {
            float f = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) f = __fadd_rn(f, __fmul_rn(q[d], knew[d]));
            acc = lane == fresh - t0 ? f : acc;
        }
        const float s = lane < n ? __fadd_rn(__fmul_rn(acc, scale), 0.0f) : -__builtin_inff();
        float m = s;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = nan_max(m, __shfl_xor(m, off, 64));
        m = lane_value(m, 0);
        const float p = nc_expf(__fsub_rn(s, m));        // exp(-inf) = 0 for lanes past the chunk
        const float l = wave_sum_f32(p);

        // o[d] in key order, the new key (the chunk's last) added last. A key
        // past the loop's range adds 0 * 0 = +0 to an accumulator that starts
        // at +0 and is never -0: exact, no change.
        const int looped = has_fresh ? n - 1 : n;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const bool in = i < looped;
            const float pi = lane_value(p, i);
            o = __fadd_rn(o, __fmul_rn(in ? pi : 0.0f, in ? v[i] : 0.0f));
        }
        if (has_fresh) o = __fadd_rn(o, __fmul_rn(lane_value(p, n - 1), vnew[dl]));
        return {m, l, o};
    }
};

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
