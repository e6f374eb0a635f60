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
#include <algorithm>

#include "nc_common.h"
#include "nc_attend.h"
#include "nc_epilogue.h"
#include "nc_math.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxKeys = 16384;     // dynamic LDS: one float per visible key


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
    v = nc::butterfly<64>(v, [](float a, float b) { return nc::nan_max(a, b); });
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    const float r = nc::nan_max(nc::nan_max(scratch[0], scratch[1]), nc::nan_max(scratch[2], scratch[3]));
    __syncthreads();
    return r;
}

// Softmax over e[0..T) in LDS, in place: z -> p, in the stated order.
__device__ void softmax_lds(float *e, int T, float *scratch) {
    float m = -__builtin_inff();
    for (int t = threadIdx.x; t < T; t += kThreads) m = nc::nan_max(m, e[t]);
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

using nc::rope_pair;

// qkv[M, (H + 2 * KV * D)] rows: q heads rotated in place; k heads rotated and
// written with v into the cache at positions past + i. cos and sin come from
// the cache's table (nc_rope_table: the same nc_cosf / nc_sinf bits) when
// given, else are computed here.
__global__ __launch_bounds__(kThreads) void rope_append(float *__restrict__ qkv, float *__restrict__ kcache,
                                                        float *__restrict__ vcache,
                                                        const float *__restrict__ inv_freq, int heads, int kv_heads,
                                                        int D, int past, int capacity,
                                                        const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error,
                                                        const float *__restrict__ table) {
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
        float c, s;
        if (table) {
            c = table[(size_t)pos * half + j];
            s = table[((size_t)capacity + pos) * half + j];
        } else {
            const float ang = __fmul_rn(fpos, inv_freq[j]);
            c = nc_cosf(ang);
            s = nc_sinf(ang);
        }
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

// -- attention over a chunked context --------------------------------------------
//
// Two kernels a call. The first takes a grid of (64-key chunk, KV head[, block
// of query rows]): each workgroup stages its chunk's keys and values in LDS
// once and attends every query of the block to it, one wave per query row,
// for every query head of the KV group (h / group), writing each query's
// chunk result (m_j, l_j, o_j) to a workspace. The second combines a query's
// chunk results in order of j. The order is nc_attend.h's, shared by the
// prefill and the decode kernels and the host oracle, so a prompt's rows and a
// decode step at the same position agree bit for bit. Splitting at a kernel
// boundary (rather than combining inside one workgroup per head) puts one
// workgroup on every chunk: at 384 keys a decode step uses 12 workgroups that
// each read 32 KB instead of 14 that each read 196 KB.
//
// Workspace layout, floats: part[((h * rows + r) * jstride + j) * (D + 2) + e],
// e = 0 (m_j), 1 (l_j), 2 + d (o_j[d]); jstride = the chunks of the longest
// context of the call.
constexpr int kWaves = 8;              // decode: waves of a chunk workgroup, one query head each
// Prefill: 4 query rows per workgroup, one per wave. A wave attends its row's
// heads of the group together, up to 7 at a time (nc_attend.h's
// chunk_scores_sq and chunk_values_n: every key or value element read from LDS
// once for all the heads' chains, the row's queries read with scalar loads
// into SGPRs (29.7 -> 29.3 us with the combine at 512 rows, where they were
// 16-byte LDS broadcasts), the d and key loops unrolled by two): 109 VGPRs,
// and 40 KB of LDS a workgroup (the staged chunk and 7 query/probability rows
// a wave), so a CU holds four workgroups, four waves a SIMD. Measured on
// MI355X at 512 rows, chunks + combine: 46 us; 49 us with 8-head batches
// (42 KB: three workgroups a CU), also with 8-row workgroups; 58 us when each
// head was attended alone with the key row and value column held in
// registers across the heads (~220 VGPRs, two waves a SIMD). Earlier variants
// of that one-head kernel, all slower: 8, 2 or 1 rows a workgroup (62, 63, 99
// us), registers capped at three waves a SIMD (spills: 168 us), each head's
// query read with scalar loads (69-73 us).
constexpr int kRowsPerBlock = 4;         // prefill: query rows (waves) a chunk workgroup, the library's choice
// The prefill schedules a tuner may choose: schedule s (1..4) stages each
// chunk for kScheduleRows[s - 1] rows; schedule 0 is kRowsPerBlock. Every
// choice computes the same bits: a row's arithmetic does not depend on which
// workgroup holds it.
constexpr int kScheduleRows[4] = {2, 4, 8, 16};
constexpr int kHeadBatch = 7;          // prefill: query heads of a row held in LDS at once (a group, in Qwen2)

// The chunk a prefill workgroup takes: blockIdx.x rotated by the row block.
// Workgroup i of a launch runs on XCD i mod 8, and blockIdx.x is the fastest
// index, so with the chunk as blockIdx.x every workgroup of chunk 0 (which
// every row sees) would share XCD 0 and those of the last chunk (which only
// the last rows see) XCD 7: a causal 512-token prompt would give one XCD
// 8/36 of the work. Rotated, each XCD takes every chunk in turn (measured on
// MI355X at 512 rows, chunks + combine: 35.4 -> 29.7 us; same bits).
__device__ __forceinline__ int chunk_of_block() {
    return (int)((blockIdx.x + blockIdx.z) % gridDim.x);
}

template <typename F>
__device__ __forceinline__ F *chunk_result(F *part, int h, int rows, int r, int jstride, int j, int D) {
    return part + (((size_t)h * rows + r) * jstride + j) * (D + 2);
}

// H heads of one query row attended to a staged chunk (nc_attend.h's two
// halves for H queries), their chunk results stored head_stride floats apart.
// The queries are read at q (wave-uniform, in global memory) into SGPRs; qp
// holds the probabilities between the halves.
template <int D, int H>
__device__ __forceinline__ void attend_heads(const float *__restrict__ q, float (*qp)[nc::kChunk],
                                             const nc::Staged<D> &st, int n, float scale, float *dst,
                                             size_t head_stride) {
    float m[H], l[H], o[H];
    nc::chunk_scores_sq<D, H>(q, qp, st, n, scale, m, l);
    nc::chunk_values_n<D, H>(qp, st, n, o);
#pragma unroll
    for (int u = 0; u < H; ++u) nc::keep_result<D>(dst + u * head_stride, nc::ChunkResult{m[u], l[u], o[u]});
}

// attend_heads<D, hn> for a run-time hn in 1 .. H.
template <int D, int H>
__device__ __forceinline__ void attend_heads_upto(int hn, const float *__restrict__ q, float (*qp)[nc::kChunk],
                                                  const nc::Staged<D> &st, int n, float scale, float *dst,
                                                  size_t head_stride) {
    if constexpr (H > 1) {
        if (hn < H) return attend_heads_upto<D, H - 1>(hn, q, qp, st, n, scale, dst, head_stride);
    }
    attend_heads<D, H>(q, qp, st, n, scale, dst, head_stride);
}

// Prefill: grid (chunks, kv_heads, ceil(rows / ROWS)) over the slab of query
// rows i0 .. i0 + rows - 1 of a call of M rows; row i sits at position past + i
// and sees keys 0 .. past + i (the cache already holds them, nc_rope_append).
// A wave takes its row's heads in batches of up to 8 in two phases: the
// scores, softmax and sums of every head of the batch (each head's
// probabilities written over its query in LDS), then every head's P V.
template <int D, int ROWS>
__global__ __launch_bounds__(64 * ROWS) void attention_rows_chunks(
    float *__restrict__ part, const float *__restrict__ qkv, const float *__restrict__ kcache,
    const float *__restrict__ vcache, int heads, int kv_heads, int past, int capacity, float scale, int i0, int rows,
    int M, int jstride, const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error) {
    if (pos_ptr && !position_fits(pos_ptr, M, capacity, error, past)) return;
    const int j = chunk_of_block(), g = blockIdx.y, t0 = j * nc::kChunk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r_last = min((int)blockIdx.z * ROWS + ROWS, rows) - 1;
    if (past + i0 + r_last + 1 <= t0) return;             // no row of the block sees this chunk
    __shared__ __align__(16) float lds[nc::Staged<D>::kFloats];
    __shared__ __align__(16) float qp[ROWS][kHeadBatch][nc::kChunk];   // per wave: its heads' p
    const nc::Staged<D> st(lds);
    const int group = heads / kv_heads, width = (heads + 2 * kv_heads) * D;
    nc::ChunkLoad<D, 64 * ROWS> load;
    load.issue(kcache + (size_t)g * capacity * D, vcache + (size_t)g * capacity * D, t0, capacity - 1);
    // the wave's row, wave-uniform (readfirstlane), so its queries' address is too
    const int r = blockIdx.z * ROWS + __builtin_amdgcn_readfirstlane(wave), i = i0 + r;
    const bool valid = r < rows && past + i + 1 > t0;
    const float *qrow = qkv + (size_t)(valid ? i : 0) * width + (size_t)g * group * D;
    load.store(st, -1, past + M - t0);                    // keys past + M and on: not yet in the cache
    __syncthreads();
    if (!valid) return;
    (void)lane;
    const int n = min(nc::kChunk, past + i + 1 - t0);
    for (int h0 = 0; h0 < group; h0 += kHeadBatch) {
        const int hn = min(kHeadBatch, group - h0);
        float *dst = chunk_result(part, g * group + h0, rows, r, jstride, j, D);
        const size_t head_stride = (size_t)rows * jstride * (D + 2);
        attend_heads_upto<D, kHeadBatch>(hn, qrow + h0 * D, qp[wave], st, n, scale, dst, head_stride);
    }
}

// The combine of one query's chunk results: grid (heads, rows), one wave.
// Row r of the slab is query row i0 + r at position past + i0 + r. The first
// 64 * BATCH floats of the row's results (BATCH = 8: up to 7 chunks, 448 keys,
// at D = 64; 16: up to 15 chunks, 960 keys) are loaded before the position is
// read, all in flight at once.
template <int D, int BATCH>
__global__ __launch_bounds__(64) void attention_combine(float *__restrict__ ctx, const float *__restrict__ part,
                                                        int heads, int past, int capacity, int i0, int rows, int M,
                                                        int jstride, const int64_t *__restrict__ pos_ptr) {
    extern __shared__ __align__(16) float results[];     // [J][D + 2]
    constexpr int kBatch = BATCH;                        // independent loads a lane keeps in flight
    const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const float *src = chunk_result(part, h, rows, r, jstride, 0, D);
    const int all = jstride * (D + 2);
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
        const int at = lane + 64 * u;
        v[u] = at < all ? src[at] : 0.0f;
    }
    if (pos_ptr) {
        const int64_t p = *pos_ptr;
        if (p < 0 || p + M > capacity) return;            // the chunk kernel reported it
        past = (int)p;
    }
    const int J = (past + i0 + r + 1 + nc::kChunk - 1) / nc::kChunk;
    const int total = J * (D + 2);
    for (int base = 0; base < total; base += 64 * kBatch) {
        if (base > 0) {
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int at = base + lane + 64 * u;
                v[u] = at < total ? src[at] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int at = base + lane + 64 * u;
            if (at < total) results[at] = v[u];
        }
    }
    // (a wave's LDS writes complete before its own later reads: no barrier)
    const float out = nc::combine_chunks(J, lane < D ? lane : 0,
                                         [&](int c, int k) { return results[c * (D + 2) + k]; });
    if (lane < D) ctx[(size_t)(i0 + r) * heads * D + h * D + lane] = out;
}

// The combine of a whole query row, one wave per head (grid rows, heads x 64
// threads), then the row's per-token int8 quantization (nc_quant.hip's
// quantize_token: the maximum of |ctx| over the row, its scale, each value
// quantized) in the same launch: ctx, xq and xs with the bits of a combine
// followed by nc_quantize_token_i8.
template <int D, int BATCH>
__global__ __launch_bounds__(1024) void attention_combine_quant(float *__restrict__ ctx, int8_t *__restrict__ xq,
                                                                float *__restrict__ xs, const float *__restrict__ part,
                                                                int heads, int past, int capacity, int i0, int rows,
                                                                int M, int jstride, const int64_t *__restrict__ pos_ptr) {
    if (pos_ptr) {
        const int64_t p = *pos_ptr;
        if (p < 0 || p + M > capacity) return;            // the chunk kernel reported it
        past = (int)p;
    }
    extern __shared__ __align__(16) float results_all[];   // [heads][jstride][D + 2]
    __shared__ float maxima[16];
    const int r = blockIdx.x, lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int J = (past + i0 + r + 1 + nc::kChunk - 1) / nc::kChunk;
    float *results = results_all + (size_t)h * jstride * (D + 2);
    const float *src = chunk_result(part, h, rows, r, jstride, 0, D);
    const int total = J * (D + 2);
    constexpr int kBatch = BATCH;                        // loads a lane keeps in flight
    for (int base = 0; base < total; base += 64 * kBatch) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int at = base + lane + 64 * u;
            v[u] = at < total ? src[at] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int at = base + lane + 64 * u;
            if (at < total) results[at] = v[u];
        }
    }
    const float out = nc::combine_chunks(J, lane < D ? lane : 0,
                                         [&](int c, int k) { return results[c * (D + 2) + k]; });
    const size_t at = (size_t)(i0 + r) * heads * D + h * D + lane;
    if (lane < D) ctx[at] = out;
    const float mag = nc::wave_max_f32(lane < D ? fabsf(out) : 0.0f);
    if (lane == 0) maxima[h] = mag;
    __syncthreads();
    float row_max = maxima[0];
    for (int i = 1; i < heads; ++i) row_max = nc::nan_max(row_max, maxima[i]);
    const float scale = nc::token_scale(row_max);
    if (lane < D) xq[at] = nc::quantize_value(out, scale);
    if (threadIdx.x == 0) xs[i0 + r] = scale;
}

// Decode: one new token at position past. Grid (chunks, kv_heads). Wave w
// attends query head g * group + w (then + 8, ... for larger groups), each
// wave rotating its own head's query; wave 0 of the chunk holding the new key
// rotates it, puts it and the new value in the staged chunk, and appends both
// to the cache (no workgroup loads that row: the others' chunks end before
// it). cos and sin of f32(past) * inv_freq[i] come from the cache's table
// (nc_rope_table) when given, else are computed here, the same nc_cosf /
// nc_sinf either way. The loads that do not depend on the position (the
// first kEarlyChunks chunks' keys and values, the q, k, v rows) go out before
// the position is read, so the two memory round trips overlap.
constexpr int kEarlyChunks = 16;

template <int D, bool TABLE>
__global__ __launch_bounds__(64 * kWaves) void attention_decode_chunks(
    float *__restrict__ part, const float *__restrict__ qkv, float *__restrict__ kcache, float *__restrict__ vcache,
    const float *__restrict__ inv_freq, const float *__restrict__ table, int heads, int kv_heads, int past,
    int capacity, float scale, int jstride, const int64_t *__restrict__ pos_ptr, int32_t *__restrict__ error) {
    const int j = blockIdx.x, g = blockIdx.y, t0 = j * nc::kChunk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int group = heads / kv_heads;
    constexpr int half = D / 2;
    float *K = kcache + (size_t)g * capacity * D;
    float *V = vcache + (size_t)g * capacity * D;
    nc::ChunkLoad<D, 64 * kWaves> load;
    const bool early = j < kEarlyChunks;
    if (early) load.issue(K, V, t0, capacity - 1);

    // RoPE operands: lane i < half of wave w, pair i of its head's query;
    // lanes half .. D - 1 of wave 0, pair lane - half of the new key.
    const int pi = lane < half ? lane : lane - half;
    const bool holds = lane < D && (lane < half ? wave < group : wave == 0);
    float x0 = 0.0f, x1 = 0.0f;
    if (holds) {
        const float *x = qkv + (size_t)(lane < half ? g * group + wave : heads + g) * D;
        x0 = x[pi];
        x1 = x[pi + half];
    }
    const float vnew = (wave == 0 && lane < D) ? qkv[(size_t)(heads + kv_heads + g) * D + lane] : 0.0f;

    if (pos_ptr && !position_fits(pos_ptr, 1, capacity, error, past)) return;
    const int T = past + 1, J = (T + nc::kChunk - 1) / nc::kChunk;
    if (j >= J) return;
    if (!early) load.issue(K, V, t0, capacity - 1);
    __shared__ __align__(16) float lds[nc::Staged<D>::kFloats];
    __shared__ __align__(16) float qs[kWaves][D];
    __shared__ __align__(16) float pbuf[kWaves][nc::kChunk];
    const nc::Staged<D> st(lds);
    const int n = min(nc::kChunk, T - t0);
    const bool fresh = j == J - 1;                       // the new key is row past - t0 of this chunk
    const bool rotates = holds && (lane < half || fresh);
    float c = 0.0f, s = 0.0f;
    if (holds) {
        if constexpr (TABLE) {
            c = table[(size_t)past * half + pi];
            s = table[((size_t)capacity + past) * half + pi];
        } else {
            const float ang = __fmul_rn((float)past, inv_freq[pi]);
            c = nc_cosf(ang);
            s = nc_sinf(ang);
        }
    }
    load.store(st, fresh ? past - t0 : -1, n);
    if (rotates) {
        float y0, y1;
        rope_pair(x0, x1, c, s, y0, y1);
        float *y = lane < half ? qs[wave] : st.keys + (past - t0) * nc::Staged<D>::kKeyStride;
        y[pi] = y0;
        y[pi + half] = y1;
        if (lane >= half) {
            K[(size_t)past * D + pi] = y0;
            K[(size_t)past * D + pi + half] = y1;
        }
    }
    if (fresh && wave == 0 && lane < D) {
        st.values[(past - t0) * D + lane] = vnew;
        V[(size_t)past * D + lane] = vnew;
    }
    __syncthreads();
    for (int hh = wave; hh < group; hh += kWaves) {
        if (hh != wave && lane < half) {                  // groups of more than 8 heads (wave-local)
            const float *x = qkv + (size_t)(g * group + hh) * D;
            float y0, y1;
            rope_pair(x[pi], x[pi + half], c, s, y0, y1);
            qs[wave][pi] = y0;
            qs[wave][pi + half] = y1;
        }
        const nc::ChunkResult res = nc::attend_staged<D>(qs[wave], st, n, scale, pbuf[wave]);
        nc::keep_result<D>(chunk_result(part, g * group + hh, 1, 0, jstride, j, D), res);
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


}  // namespace

// p: [qkv f32[M, (H + 2*KV*D)] (q rotated in place), kcache f32[KV, C, D], vcache f32[KV, C, D],
//     inv_freq f32[D/2], pos i64[1] | NULL, rope table f32[2, C, D/2] | NULL];
// s: [M, heads, kv_heads, D, past, capacity]
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
                       pos ? 0 : (int)past, (int)cap, pos, nc::error_word(), (const float *)p[5]);
    return nc::launched("rope_append");
}

namespace {

// LDS of a combine: J chunk results of D + 2 floats, 67.6 KB at 16384 keys and
// D = 64, past the 64 KB a launch gets without asking.
template <int D, int BATCH>
int32_t launch_combine_batch(float *ctx, const float *part, int64_t heads, int64_t past, int64_t cap, int64_t i0,
                             int64_t rows, int64_t M, int64_t jstride, const int64_t *pos) {
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attention_combine<D, BATCH>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024) != hipSuccess) {
            nc::set_message("attention: could not raise the LDS limit of the combine");
            return NC_LAUNCH_FAILED;
        }
        raised = true;
    }
    const size_t lds = (size_t)jstride * (D + 2) * sizeof(float);
    hipLaunchKernelGGL((attention_combine<D, BATCH>), dim3((unsigned)heads, (unsigned)rows), dim3(64), lds,
                       nc::stream(), ctx, part, (int)heads, (int)past, (int)cap, (int)i0, (int)rows, (int)M,
                       (int)jstride, pos);
    return nc::launched("attention_combine");
}

// The first batch of loads sized to the chunk results a row can have.
template <int D>
int32_t launch_combine(float *ctx, const float *part, int64_t heads, int64_t past, int64_t cap, int64_t i0,
                       int64_t rows, int64_t M, int64_t jstride, const int64_t *pos) {
    if (jstride * (D + 2) <= 64 * 8)
        return launch_combine_batch<D, 8>(ctx, part, heads, past, cap, i0, rows, M, jstride, pos);
    return launch_combine_batch<D, 16>(ctx, part, heads, past, cap, i0, rows, M, jstride, pos);
}

// A head's chunk results in one batch of loads up to 9 chunks at D = 64 (576
// floats: a 512-token prompt's 8 chunks in one memory round trip), else in
// batches of 16 loads a lane.
template <int D>
int32_t launch_combine_quant(void **p, const float *part, int64_t heads, int64_t past, int64_t cap, int64_t i0,
                             int64_t rows, int64_t M, int64_t jstride, const int64_t *pos) {
    const size_t lds = (size_t)heads * jstride * (D + 2) * sizeof(float);
    auto kernel = jstride * (D + 2) <= 64 * 9 ? attention_combine_quant<D, 9> : attention_combine_quant<D, 16>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)rows), dim3((unsigned)(64 * heads)), lds, nc::stream(), (float *)p[0],
                       (int8_t *)p[6], (float *)p[7], part, (int)heads, (int)past, (int)cap, (int)i0, (int)rows,
                       (int)M, (int)jstride, pos);
    return nc::launched("attention_combine_quant");
}

// Query rows in slabs whose chunk results fit the workspace; each slab is a
// chunk launch and a combine launch.
template <int D, int ROWS>
int32_t launch_prefill(void **p, int64_t M, int64_t heads, int64_t kv, int64_t past, int64_t cap, float scale,
                       const int64_t *pos, float *work, int64_t work_bytes) {
    const int64_t jstride = ((pos ? cap : past + M) + nc::kChunk - 1) / nc::kChunk;
    const int64_t row_bytes = heads * jstride * (D + 2) * (int64_t)sizeof(float);
    int64_t slab = std::min<int64_t>(M, work_bytes / row_bytes);
    NC_REQUIRE(slab >= 1, "nc_attention: the workspace is smaller than one query row's chunk results "
                          "(heads * ceil(keys / 64) * (head_dim + 2) floats)");
    // with xq and xs, the per-token int8 of ctx too: in the combine's own launch
    // while a row's chunk results fit its workgroup's LDS, else after
    const bool quantize = p[6] && p[7];
    const bool fused = quantize && heads <= 16 && heads * jstride * (D + 2) * (int64_t)sizeof(float) <= 64 * 1024;
    if (slab < M && slab >= ROWS) slab -= slab % ROWS;
    const int64_t host_past = pos ? 0 : past;
    for (int64_t i0 = 0; i0 < M; i0 += slab) {
        const int64_t rows = std::min(slab, M - i0);
        const int64_t chunks = pos ? jstride : (past + i0 + rows + nc::kChunk - 1) / nc::kChunk;
        hipLaunchKernelGGL((attention_rows_chunks<D, ROWS>),
                           dim3((unsigned)chunks, (unsigned)kv, (unsigned)((rows + ROWS - 1) / ROWS)),
                           dim3(64 * ROWS), 0, nc::stream(), work, (const float *)p[1], (const float *)p[2],
                           (const float *)p[3], (int)heads, (int)kv, (int)host_past, (int)cap, scale, (int)i0,
                           (int)rows, (int)M, (int)jstride, pos, nc::error_word());
        int32_t rc = nc::launched("attention_rows_chunks");
        if (rc == NC_OK && fused)
            rc = launch_combine_quant<D>(p, work, heads, host_past, cap, i0, rows, M, jstride, pos);
        else if (rc == NC_OK)
            rc = launch_combine<D>((float *)p[0], work, heads, host_past, cap, i0, rows, M, jstride, pos);
        if (rc != NC_OK) return rc;
    }
    if (quantize && !fused)        // ctx whole first: the per-token scale spans every head of a row
        return nc::quantize_token_rows((int8_t *)p[6], (float *)p[7], (const float *)p[0], (int)M, (int)(heads * D));
    return NC_OK;
}

template <int D, bool TABLE>
int32_t launch_decode(void **p, const int64_t *s, const int64_t *pos, float *work, int64_t work_bytes) {
    const int64_t heads = s[0], kv = s[1], past = s[3], cap = s[4];
    const int64_t jstride = ((pos ? cap : past + 1) + nc::kChunk - 1) / nc::kChunk;
    NC_REQUIRE(heads * jstride * (D + 2) * (int64_t)sizeof(float) <= work_bytes,
               "nc_attention_decode: the workspace is smaller than heads * ceil(keys / 64) * (head_dim + 2) floats");
    const int64_t host_past = pos ? 0 : past;
    hipLaunchKernelGGL((attention_decode_chunks<D, TABLE>), dim3((unsigned)jstride, (unsigned)kv), dim3(64 * kWaves), 0,
                       nc::stream(), work, (const float *)p[1], (float *)p[2], (float *)p[3], (const float *)p[4],
                       (const float *)p[6], (int)heads, (int)kv, (int)host_past, (int)cap, nc::bits_to_float(s[5]),
                       (int)jstride, pos, nc::error_word());
    const int32_t rc = nc::launched("attention_decode_chunks");
    if (rc != NC_OK) return rc;
    return launch_combine<D>((float *)p[0], work, heads, host_past, cap, 0, 1, 1, jstride, pos);
}

}  // namespace

// p: [ctx f32[M, heads*D], qkv f32[M, (H + 2*KV*D)] (q rotated), kcache, vcache, pos i64[1] | NULL,
//     work f32[...], xq i8[M, heads*D] | NULL, xs f32[M] | NULL (with both: ctx's per-token int8 too)];
// s: [M, heads, kv_heads, D, past, capacity, scale as float32 bits, work bytes, schedule]
//    (D 16, 32 or 64; schedule 0 the library's rows a workgroup, 1..4 the tuner's choices:
//    nc_attention_schedule_info)
// With pos, past is read from the device when the kernels run (s[4] is ignored). The workspace
// holds the chunk results; one query row needs heads * ceil(keys / 64) * (D + 2) floats, keys =
// past + M (capacity with pos), and a smaller workspace than M rows' takes the rows in slabs.
NC_EXPORT int32_t nc_attention(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[5], "nc_attention: null operand");
    const int64_t M = s[0], heads = s[1], kv = s[2], D = s[3], past = s[4], cap = s[5], work_bytes = s[7];
    const int64_t *pos = (const int64_t *)p[4];
    NC_REQUIRE(M >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && (D == 16 || D == 32 || D == 64) &&
                   (pos ? cap <= kMaxKeys : (past >= 0 && past + M <= cap && past + M <= kMaxKeys)) &&
                   M <= cap && M < 65536 && heads < 65536 && work_bytes >= 0,
               "nc_attention: bad shape (head_dim 16, 32 or 64; at most 16384 keys)");
    const int64_t schedule = s[8];
    NC_REQUIRE(schedule >= 0 && schedule <= 4, "nc_attention: no such schedule (0..4)");
    if (M == 0) return NC_OK;
    const float scale = nc::bits_to_float(s[6]);
    float *work = (float *)p[5];
    const int rows = schedule == 0 ? kRowsPerBlock : kScheduleRows[schedule - 1];
#define NC_PREFILL(R)                                                                             \
    if (rows == R) {                                                                              \
        if (D == 64) return launch_prefill<64, R>(p, M, heads, kv, past, cap, scale, pos, work, work_bytes); \
        if (D == 32) return launch_prefill<32, R>(p, M, heads, kv, past, cap, scale, pos, work, work_bytes); \
        return launch_prefill<16, R>(p, M, heads, kv, past, cap, scale, pos, work, work_bytes);    \
    }
    NC_PREFILL(2)
    NC_PREFILL(4)
    NC_PREFILL(8)
    NC_PREFILL(16)
#undef NC_PREFILL
    return NC_BAD_ARGS;
}

// A prefill attention schedule's launch shape, for the tuner (no device call):
// out = [query rows a chunk workgroup (its waves)]; NC_BAD_ARGS past the table.
NC_EXPORT int32_t nc_attention_schedule_info(int64_t schedule, int64_t *out) {
    if (!out || schedule < 1 || schedule > 4) return NC_BAD_ARGS;
    out[0] = kScheduleRows[schedule - 1];
    return NC_OK;
}

// Attention of one new token with RoPE and the cache append fused in.
// p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated, with bias), kcache f32[kv,C,D],
//     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] | NULL, rope table f32[2,C,D/2] | NULL,
//     work f32[heads * ceil(keys / 64) * (D + 2)]];
// s: [heads, kv, D, past, C, scale as float32 bits, work bytes]  (D 16, 32 or 64, C <= 16384; past
//    read from pos when given, and then keys = C, else past + 1)
NC_EXPORT int32_t nc_attention_decode(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[7], "nc_attention_decode: null operand");
    const int64_t heads = s[0], kv = s[1], D = s[2], past = s[3], cap = s[4];
    const int64_t *pos = (const int64_t *)p[5];
    NC_REQUIRE(heads > 0 && kv > 0 && heads % kv == 0 && heads < 65536 && (D == 64 || D == 32 || D == 16) &&
                   cap > 0 && cap <= kMaxKeys && (pos || (past >= 0 && past + 1 <= cap)),
               "nc_attention_decode: bad shape (head_dim 16, 32 or 64, capacity at most 16384)");
    float *work = (float *)p[7];
    const bool table = p[6] != nullptr;
    if (D == 64) return table ? launch_decode<64, true>(p, s, pos, work, s[6]) : launch_decode<64, false>(p, s, pos, work, s[6]);
    if (D == 32) return table ? launch_decode<32, true>(p, s, pos, work, s[6]) : launch_decode<32, false>(p, s, pos, work, s[6]);
    return table ? launch_decode<16, true>(p, s, pos, work, s[6]) : launch_decode<16, false>(p, s, pos, work, s[6]);
}


// -- decode attention with no allocation ---------------------------------------
//
// nc_attention_decode_static is nc_attention_decode (the same kernels, the same
// bits) with its chunk-result workspace in a device array the library holds
// for the life of the process, for callers that cannot allocate (code under
// graph capture, serving loops, harnesses that forbid hipMalloc). Each GPU has
// its own copy, at its own address, looked up once per device by nc_init (the
// array's name in host code is a host-side stand-in, not a device address).
// Every call on a GPU shares that GPU's copy, so calls that overlap on one GPU
// (two streams, two threads) race. Nothing in it needs clearing between calls:
// a call's chunk kernel writes every chunk result its combine then reads.
namespace {
constexpr int64_t kScratchBytes = 1 << 20;     // 14 heads x 256 chunks (16384 keys) x 66 floats fit
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
float *g_scratch[kMaxDevices] = {};            // each device's address of `scratch`
}  // namespace

int32_t nc::attention_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) {
        set_message("nc_init: device index beyond the library's table of workspace addresses");
        return NC_BAD_ARGS;
    }
    if (g_scratch[device]) return NC_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
        set_message("nc_init: hipGetSymbolAddress of the attention workspace failed");
        return NC_LAUNCH_FAILED;
    }
    g_scratch[device] = static_cast<float *>(ptr);
    return NC_OK;
}

// p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated, with bias), kcache f32[kv,C,D],
//     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] | NULL, rope table f32[2,C,D/2] | NULL];
// s: [heads, kv, D, past, C, scale as float32 bits]; heads * ceil(keys / 64) * (D + 2) floats
//    (keys = C with pos, else past + 1) must fit the 1 MiB workspace.
NC_EXPORT int32_t nc_attention_decode_static(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_attention_decode_static: null operand");
    const int64_t heads = s[0], kv = s[1], D = s[2], past = s[3], cap = s[4];
    const int64_t *pos = (const int64_t *)p[5];
    NC_REQUIRE(heads > 0 && kv > 0 && heads % kv == 0 && heads < 65536 && (D == 64 || D == 32 || D == 16) &&
                   cap > 0 && cap <= kMaxKeys && (pos || (past >= 0 && past + 1 <= cap)),
               "nc_attention_decode_static: bad shape (head_dim 16, 32 or 64, capacity at most 16384)");
    const int dev = nc::device();
    NC_REQUIRE(dev >= 0 && dev < kMaxDevices && g_scratch[dev], "nc_attention_decode_static: call nc_init first");
    const int64_t keys = pos ? cap : past + 1;
    NC_REQUIRE(heads * ((keys + nc::kChunk - 1) / nc::kChunk) * (D + 2) * (int64_t)sizeof(float) <= kScratchBytes,
               "nc_attention_decode_static: heads * ceil(keys / 64) * (head_dim + 2) floats exceed the "
               "library's 1 MiB workspace; use nc_attention_decode with a workspace of that size");
    float *work = g_scratch[dev];
    const bool table = p[6] != nullptr;
    if (D == 64) return table ? launch_decode<64, true>(p, s, pos, work, kScratchBytes)
                              : launch_decode<64, false>(p, s, pos, work, kScratchBytes);
    if (D == 32) return table ? launch_decode<32, true>(p, s, pos, work, kScratchBytes)
                              : launch_decode<32, false>(p, s, pos, work, kScratchBytes);
    return table ? launch_decode<16, true>(p, s, pos, work, kScratchBytes)
                 : launch_decode<16, false>(p, s, pos, work, kScratchBytes);
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
