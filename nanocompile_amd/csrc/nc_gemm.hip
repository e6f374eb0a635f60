// The per-token int8 projection, prefill shape, on the i8 matrix cores:
//
//   acc[m, n] = sum_k xq[m, k] * q[n, k]          exact, int32 (any order)
//   y[m, n]   = (f32(acc) * xs[m]) * scales[n]     then + bias[n], then residual[m, n] + y
//
// (the epilogue of nc_gemv.hip, from nc_epilogue.h, so prefill and decode
// produce the same bits). The reference's int8 matmuls are a k loop per
// output (lower.py:294-417); a GEMM has nothing of that order to keep,
// because integer accumulation is exact in any order.
//
// Tiling for gfx950 (CDNA4):
//  * v_mfma_i32_16x16x64_i8: a 16 x 16 int32 tile from 16 rows of q (first
//    operand) and 16 rows of xq (second), 64 bytes of k each. Lane l supplies
//    row l % 16, bytes 16 * (l / 16) .. + 15 of the 64 for both operands (the
//    same k set for both, which is all an exact sum needs), and receives
//    acc[n = 4 * (l / 16) + r][m = l % 16], r = 0..3: four consecutive
//    outputs of one token row, stored with one 16-byte write.
//  * A workgroup of WAVES = (BM / WM) * (BN / WN) waves owns a BM x BN output
//    tile; wave w computes a WM x WN sub-tile as (WM / 16) x (WN / 16) MFMAs.
//  * Each k stage moves BM x BK bytes of xq and BN x BK bytes of q (twice for
//    the SwiGLU pair) from HBM/L2 into registers with 16-byte loads, 8 or 4
//    lanes per 128- or 64-byte row segment, then into unpadded LDS rows whose
//    16-byte chunks are permuted (chunk c of row r at c ^ ((r / 2) mod the
//    chunks a row)), so neither the stores nor the 16-byte MFMA operand reads
//    of 16 consecutive rows meet a bank conflict (rocprofv3
//    SQ_LDS_BANK_CONFLICT: 0 cycles for 128- and 64-byte rows, against about
//    2.6 an LDS instruction with rows padded by 16 bytes, and 3 permuting by
//    r mod the chunks a row at 64 bytes; 11.5 against 12.4 us on (896,4864)
//    at M = 512).
//    A ring of NS register stages keeps the loads of stages
//    t + 1 .. t + NS - 1 in flight while stage t is multiplied out of one of
//    two LDS buffers; one barrier per stage.
//  * Tiles are handed to the 8 XCDs (workgroup i runs on XCD i % 8) so that
//    each XCD takes a contiguous range of tiles, m fastest: the workgroups
//    sharing a band of weight rows share one XCD's L2, and each weight byte
//    comes from HBM once.
//  * Edges: rows past M or N are clamped to the last valid row for loading and
//    not stored; k chunks past K (K a multiple of 16) load as zero.
#include "nc_common.h"
#include "nc_epilogue.h"

namespace {

using nc::i8x16;
typedef int32_t v4i __attribute__((ext_vector_type(4)));

enum Epilogue { kDequant = 0, kAccOut = 1, kSwiglu = 2, kRope = 3 };

// The qkv projection's RoPE and cache append, as nc_rope_append does them
// after it (nc_attention.hip): with tiles exactly one head wide (BN = D).
struct RopeArgs {
    float *kcache, *vcache;            // [kv, capacity, D]
    const float *table;                // cos, sin [2, capacity, D / 2] (nc_rope_table)
    const int64_t *pos;                // the position of row 0, or NULL: past
    int32_t *error;
    int heads, kv, past, capacity;
    int head_dim;                      // the tile's n must equal it: the epilogue takes a tile as one head
};

struct GemmArgs {
    void *out;
    const int8_t *xq;
    const float *xs;
    const int8_t *q;
    const float *ws;
    const float *bias;
    const float *residual;
    const int8_t *q2;        // SwiGLU: the up projection
    const float *ws2;
    int M, N, K;
    RopeArgs rope;
};

__device__ __forceinline__ int tile_of(int id, int total) {
    const int full = total & ~7;
    return id < full ? (id & 7) * (total >> 3) + (id >> 3) : id;
}

template <int BM, int BN, int BK, int WM, int WN, int NS, int EPI, bool FULLK>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_i8_mfma(GemmArgs a) {
    constexpr int WAVES = (BM / WM) * (BN / WN);
    constexpr int THREADS = WAVES * 64;
    constexpr int NB = EPI == kSwiglu ? 2 : 1;        // weight matrices per tile
    constexpr int CPR = BK / 16;                      // 16-byte chunks per row per stage
    constexpr int STRIDE = BK;                        // LDS row, unpadded
    static_assert(BK == 64 || BK == 128, "LDS chunk permutation measured for 64- and 128-byte rows");
    // The byte offset in an LDS buffer of 16-byte chunk c of row r: the chunks
    // of a row permuted by (r / 2) mod CPR, so the 16-byte fragment reads of
    // 16 consecutive rows at one k, and the stores of a row's consecutive
    // chunks, meet no bank conflict (measured, both row lengths).
    auto lds_at = [](int r, int c) { return r * STRIDE + ((c ^ ((r >> 1) & (CPR - 1))) << 4); };
    constexpr int A_PER = BM * CPR / THREADS;
    constexpr int B_PER = NB * BN * CPR / THREADS;
    constexpr int MI = WM / 16, NI = WN / 16;
    static_assert(BM * CPR % THREADS == 0 && NB * BN * CPR % THREADS == 0, "tile and workgroup mismatch");
    static_assert(BK % 64 == 0 && WM % 16 == 0 && WN % 16 == 0, "MFMA tile shape");
    static_assert(NS >= 2 && NS % 2 == 0, "the register ring alternates the two LDS buffers");

    __shared__ __align__(16) int8_t sA[2][BM * STRIDE];
    __shared__ __align__(16) int8_t sB[2][NB * BN * STRIDE];

    const int M = a.M, N = a.N, K = a.K;
    const int mtiles = (M + BM - 1) / BM;
    const int t = tile_of(blockIdx.x, gridDim.x);
    const int m0 = (t % mtiles) * BM, n0 = (t / mtiles) * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave / (BN / WN)) * WM, wn = (wave % (BN / WN)) * WN;

    // This thread's share of a stage: fixed rows (clamped into range) and chunk
    // columns, k advancing.
    const int8_t *srcA[A_PER];
    int dstA[A_PER], colA[A_PER];
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
        const int id = tid + i * THREADS, r = id / CPR, c = id % CPR;
        srcA[i] = a.xq + (size_t)min(m0 + r, M - 1) * K;
        dstA[i] = lds_at(r, c);
        colA[i] = c * 16;
    }
    const int8_t *srcB[B_PER];
    int dstB[B_PER], colB[B_PER];
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
        const int id = tid + i * THREADS, r = id / CPR, c = id % CPR;   // r < NB * BN
        const int8_t *base = (NB == 2 && r >= BN) ? a.q2 : a.q;
        srcB[i] = base + (size_t)min(n0 + r % BN, N - 1) * K;
        dstB[i] = lds_at(r, c);
        colB[i] = c * 16;
    }

    // The register ring: slot j holds stage s's chunks for s % NS == j, loaded
    // NS - 1 stages before they are written to LDS.
    i8x16 ra[NS][A_PER], rb[NS][B_PER];
    auto load_stage = [&](int k0, i8x16 (&xa)[A_PER], i8x16 (&xb)[B_PER]) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            if constexpr (FULLK) {
                xa[i] = nc::load16(srcA[i] + k0 + colA[i]);
            } else {
                const bool in = k0 + colA[i] < K;    // else a row's first chunk, always in bounds
                const i8x16 v = nc::load16(srcA[i] + (in ? k0 + colA[i] : 0));
                xa[i] = in ? v : i8x16{};
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            if constexpr (FULLK) {
                xb[i] = nc::load16(srcB[i] + k0 + colB[i]);
            } else {
                const bool in = k0 + colB[i] < K;
                const i8x16 v = nc::load16(srcB[i] + (in ? k0 + colB[i] : 0));
                xb[i] = in ? v : i8x16{};
            }
        }
    };
    auto store_stage = [&](int buf, const i8x16 (&xa)[A_PER], const i8x16 (&xb)[B_PER]) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) *reinterpret_cast<i8x16 *>(&sA[buf][dstA[i]]) = xa[i];
#pragma unroll
        for (int i = 0; i < B_PER; ++i) *reinterpret_cast<i8x16 *>(&sB[buf][dstB[i]]) = xb[i];
    };

    v4i acc[NB][MI][NI];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[b][i][j] = v4i{0, 0, 0, 0};

    // The weight fragment goes first, so the accumulator tile is [n][m] and a
    // lane ends with 4 consecutive n of one m: one 16-byte store per tile.
    const int row16 = lane & 15, kq = (lane >> 4) * 16;
    auto multiply = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 64) {
            v4i fa[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                fa[i] = *reinterpret_cast<const v4i *>(&sA[buf][lds_at(wm + i * 16 + row16, (kk + kq) >> 4)]);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const v4i fb =
                        *reinterpret_cast<const v4i *>(&sB[buf][lds_at(b * BN + wn + j * 16 + row16, (kk + kq) >> 4)]);
#pragma unroll
                    for (int i = 0; i < MI; ++i)
                        acc[b][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb, fa[i], acc[b][i][j], 0, 0, 0);
                }
            }
        }
    };

    // The epilogue's per-row and per-column operands, fetched now so their
    // latency hides under the k loop (indices clamped; unused past the edges).
    const int nq = (lane >> 4) * 4;
    float xs_r[MI], w1_r[NI][4], w2_r[NI][4], b_r[NI][4];
    if constexpr (EPI != kAccOut) {
#pragma unroll
        for (int i = 0; i < MI; ++i) xs_r[i] = a.xs[min(m0 + wm + i * 16 + row16, M - 1)];
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = min(n0 + wn + j * 16 + nq + r, N - 1);
                w1_r[j][r] = a.ws[n];
                if constexpr (EPI == kSwiglu) w2_r[j][r] = a.ws2[n];
                if constexpr (EPI == kDequant || EPI == kRope) b_r[j][r] = a.bias ? a.bias[n] : 0.0f;
            }
    }
    // RoPE: the tile's rows' positions and this thread's pairs' cos and sin,
    // also fetched before the k loop (pair u of the thread: idx = tid + u THREADS).
    constexpr int HALF = BN / 2;
    constexpr int PAIRS = EPI == kRope ? BM * HALF / THREADS : 1;
    static_assert(EPI != kRope || BM * HALF % THREADS == 0, "whole pairs per thread");
    float rc[PAIRS], rs[PAIRS];
    int rope_past = 0;
    bool rotate = true;
    if constexpr (EPI == kRope) {
        const RopeArgs &ro = a.rope;
        rope_past = ro.past;
        if (ro.pos) {
            const int64_t p = *ro.pos;
            if (p < 0 || p + M > ro.capacity) {
                if (blockIdx.x == 0 && threadIdx.x == 0) atomicCAS(ro.error, 0, NC_FAIL_CAPACITY);
                rotate = false;                      // as nc_rope_append: qkv as projected, nothing appended
            } else {
                rope_past = (int)p;
            }
        }
#pragma unroll
        for (int u = 0; u < PAIRS; ++u) {
            const int idx = tid + u * THREADS, mm = idx / HALF, jj = idx - mm * HALF;
            const int position = rotate ? rope_past + min(m0 + mm, M - 1) : 0;
            rc[u] = ro.table[(size_t)position * HALF + jj];
            rs[u] = ro.table[((size_t)ro.capacity + position) * HALF + jj];
        }
    }

    // Step s: refill slot s % NS with stage s + NS, multiply stage s from LDS
    // buffer s & 1, write stage s + 1 (slot (s + 1) % NS) into the other
    // buffer, barrier. NS is even, so slot and buffer are fixed per unrolled j.
    // The main loop runs whole groups of NS steps with no branch, so the
    // compiler's waits for slot (s + 1) % NS count only the loads issued
    // after it; loads past the last stage repeat the last stage (never
    // multiplied). The last stages % NS steps have nothing left to load.
    const int stages = (K + BK - 1) / BK;
    const int last = (stages - 1) * BK;
#pragma unroll
    for (int j = 0; j < NS; ++j) load_stage(min(j * BK, last), ra[j], rb[j]);
    store_stage(0, ra[0], rb[0]);
    __syncthreads();
    int s0 = 0;
    for (; s0 + NS <= stages; s0 += NS) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            load_stage(min((s0 + j + NS) * BK, last), ra[j], rb[j]);
            multiply(j & 1);
            store_stage((j + 1) & 1, ra[(j + 1) % NS], rb[(j + 1) % NS]);
            __syncthreads();
        }
    }
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
        if (s0 + j < stages) {
            multiply(j & 1);
            store_stage((j + 1) & 1, ra[(j + 1) % NS], rb[(j + 1) % NS]);
            __syncthreads();
        }
    }

    if constexpr (EPI == kRope) {
        // The tile is one head, [BM rows][BN = D columns]: dequantized (+ bias)
        // into LDS, then each pair (j, j + D/2) of a row rotated at the row's
        // position (q heads, written back in place; k heads, into the cache)
        // or copied (v heads, into the cache). The qkv rows of k and v keep
        // their unrotated values, as after nc_rope_append.
        static_assert(BM * BN * sizeof(float) <= sizeof(sA), "the tile must fit the staging LDS");
        const RopeArgs &ro = a.rope;
        __syncthreads();                             // every wave is done with the staging buffers
        float *tile = reinterpret_cast<float *>(&sA[0][0]);
        // Element (row, col) of the tile: the row's 4-float granules permuted by
        // a bijection of the row index (consecutive rows taking opposite halves),
        // so the 16-byte stores of 16 rows at one column, and the reads of two
        // consecutive rows, meet no bank conflict.
        constexpr int G = BN / 4;
        auto tile_at = [](int row, int col) {
            const int f = (row ^ ((row & 1) * (G / 2))) & (G - 1);
            return row * BN + ((((col >> 2) ^ f)) << 2) + (col & 3);
        };
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                float *t = tile + tile_at(wm + i * 16 + row16, wn + j * 16 + nq);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = nc::dequant(acc[0][i][j][r], xs_r[i], w1_r[j][r]);
                    if (a.bias) v = __fadd_rn(v, b_r[j][r]);
                    t[r] = v;
                }
            }
        }
        __syncthreads();
        const int head = n0 / BN;
#pragma unroll
        for (int u = 0; u < PAIRS; ++u) {
            const int idx = tid + u * THREADS, mm = idx / HALF, jj = idx - mm * HALF, m = m0 + mm;
            if (m >= M) continue;
            const float x0 = tile[tile_at(mm, jj)], x1 = tile[tile_at(mm, jj + HALF)];
            float *y = static_cast<float *>(a.out) + (size_t)m * N + n0;
            const int position = rope_past + m;
            float y0 = x0, y1 = x1;
            if (rotate && head < ro.heads + ro.kv) nc::rope_pair(x0, x1, rc[u], rs[u], y0, y1);
            if (head < ro.heads && rotate) {
                y[jj] = y0;
                y[jj + HALF] = y1;
            } else {
                y[jj] = x0;
                y[jj + HALF] = x1;
            }
            if (rotate && head >= ro.heads) {
                const bool is_k = head < ro.heads + ro.kv;
                const int g = head - ro.heads - (is_k ? 0 : ro.kv);
                float *c = (is_k ? ro.kcache : ro.vcache) + ((size_t)g * ro.capacity + position) * BN;
                c[jj] = is_k ? y0 : x0;
                c[jj + HALF] = is_k ? y1 : x1;
            }
        }
        return;
    }

    // Epilogue: lane holds n = 4 * (lane / 16) + r, r = 0..3, of each 16 x 16
    // tile, for m = lane % 16. With N a multiple of 4 a lane's 4 outputs are one
    // aligned 16-byte store (and residual load).
    const bool vec = (N & 3) == 0;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int m = m0 + wm + i * 16 + row16;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int nb = n0 + wn + j * 16 + nq;
            if (nb >= N) continue;
            const size_t at = (size_t)m * N + nb;
            float v[4];
            if constexpr (EPI == kAccOut) {
                if (vec) {
                    *reinterpret_cast<v4i *>(static_cast<int32_t *>(a.out) + at) = acc[0][i][j];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (nb + r < N) static_cast<int32_t *>(a.out)[at + r] = acc[0][i][j][r];
                }
                continue;
            } else if constexpr (EPI == kDequant) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    v[r] = nc::dequant(acc[0][i][j][r], xs_r[i], w1_r[j][r]);
                    if (a.bias) v[r] = __fadd_rn(v[r], b_r[j][r]);
                }
                if (a.residual) {
                    if (vec) {
                        const float4 res = *reinterpret_cast<const float4 *>(a.residual + at);
                        v[0] = __fadd_rn(res.x, v[0]);
                        v[1] = __fadd_rn(res.y, v[1]);
                        v[2] = __fadd_rn(res.z, v[2]);
                        v[3] = __fadd_rn(res.w, v[3]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (nb + r < N) v[r] = __fadd_rn(a.residual[at + r], v[r]);
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float g = nc::dequant(acc[0][i][j][r], xs_r[i], w1_r[j][r]);
                    const float u = nc::dequant(acc[NB - 1][i][j][r], xs_r[i], w2_r[j][r]);
                    v[r] = nc::silu_mul(g, u);
                }
            }
            float *y = static_cast<float *>(a.out) + at;
            if (vec) {
                *reinterpret_cast<float4 *>(y) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (nb + r < N) y[r] = v[r];
            }
        }
    }
}

template <int BM, int BN, int BK, int WM, int WN, int NS, int EPI>
int32_t launch_tile(const GemmArgs &a) {
    const unsigned tiles = (unsigned)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    constexpr int THREADS = (BM / WM) * (BN / WN) * 64;
    if (a.K % BK == 0)
        hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, BK, WM, WN, NS, EPI, true>), dim3(tiles), dim3(THREADS), 0,
                           nc::stream(), a);
    else
        hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, BK, WM, WN, NS, EPI, false>), dim3(tiles), dim3(THREADS), 0,
                           nc::stream(), a);
    return nc::launched("gemm_i8_mfma");
}

}  // namespace

// The MFMA tile table, one row per tile index: (index, BM, BN, BK, WM, WN, NS).
// Shared with nc_gemv.hip's schedule dispatch (indices kGemmFirst..) and
// reported by nc_schedule_info, so the tuner reads the same table it runs.
#define NC_GEMM_TILES(X)            \
    X(0, 64, 64, 128, 32, 32, 4)    \
    X(1, 32, 64, 128, 32, 16, 4)    \
    X(2, 32, 32, 128, 16, 16, 4)    \
    X(3, 32, 32, 128, 16, 16, 8)    \
    X(4, 32, 64, 128, 32, 16, 8)    \
    X(5, 64, 64, 128, 32, 32, 2)    \
    X(6, 64, 128, 128, 32, 32, 4)   \
    X(7, 128, 128, 64, 32, 64, 4)   \
    X(8, 128, 64, 128, 32, 32, 4)

namespace nc {

int32_t gemm_i8_token(int tile, int epi, void *out, const int8_t *xq, const float *xs, const int8_t *q,
                      const float *ws, const float *bias, const float *residual, const int8_t *q2,
                      const float *ws2, int M, int N, int K) {
    const GemmArgs a{out, xq, xs, q, ws, bias, residual, q2, ws2, M, N, K};
    if (M == 0 || N == 0) return NC_OK;
#define NC_TILE_CASE(I, BM, BN, BK, WM, WN, NS)                                     \
    case I:                                                                         \
        if (epi == kAccOut) return launch_tile<BM, BN, BK, WM, WN, NS, kAccOut>(a); \
        if (epi == kSwiglu) return launch_tile<BM, BN, BK, WM, WN, NS, kSwiglu>(a); \
        return launch_tile<BM, BN, BK, WM, WN, NS, kDequant>(a);
    switch (tile) {
        NC_GEMM_TILES(NC_TILE_CASE)
        default: set_message("gemm_i8_token: no such tile"); return NC_BAD_ARGS;
    }
#undef NC_TILE_CASE
}

// The qkv projection with RoPE and the cache append in its epilogue: tiles one
// head wide (BN = head_dim) only.
template <int BM, int BN, int BK, int WM, int WN, int NS>
int32_t launch_rope_tile(const GemmArgs &a) {
    if constexpr (BN == 32 || BN == 64) {
        if (a.rope.head_dim != BN) {        // the epilogue's head index is n / BN: BN must be the head
            set_message("nc_matmul_i8_token_rope: the tile is not one head wide");
            return NC_BAD_ARGS;
        }
        return launch_tile<BM, BN, BK, WM, WN, NS, kRope>(a);
    } else {
        set_message("nc_matmul_i8_token_rope: the tile is not one head wide");
        return NC_BAD_ARGS;
    }
}

int32_t gemm_i8_token_rope(int tile, const GemmArgs &a) {
#define NC_ROPE_CASE(I, BM, BN, BK, WM, WN, NS) \
    case I: return launch_rope_tile<BM, BN, BK, WM, WN, NS>(a);
    switch (tile) {
        NC_GEMM_TILES(NC_ROPE_CASE)
        default: set_message("nc_matmul_i8_token_rope: no such tile"); return NC_BAD_ARGS;
    }
#undef NC_ROPE_CASE
}

// out: [BM, BN, BK, WM, WN, NS, workgroup threads, LDS bytes with one weight matrix,
//       LDS bytes with the SwiGLU pair's two]: the kernel's two unpadded buffers of
//       BM activation rows and NB * BN weight rows of BK bytes.
int32_t gemm_tile_info(int tile, int64_t *out) {
#define NC_TILE_INFO(I, BM, BN, BK, WM, WN, NS)                                          \
    case I: {                                                                            \
        const int64_t v[9] = {BM, BN, BK, WM, WN, NS, (BM / WM) * (BN / WN) * 64,        \
                              2 * (BM + BN) * BK, 2 * (BM + 2 * BN) * BK};               \
        for (int i = 0; i < 9; ++i) out[i] = v[i];                                       \
        return NC_OK;                                                                    \
    }
    switch (tile) {
        NC_GEMM_TILES(NC_TILE_INFO)
        default: return NC_BAD_ARGS;
    }
#undef NC_TILE_INFO
}

}  // namespace nc

// The schedule numbers of the MFMA tiles (nc_gemv.hip's space: 16 + tile index).
constexpr int64_t kGemmFirstSchedule = 16, kGemmTileCount = 9;

// The qkv projection of a prompt with RoPE and the KV-cache append fused into
// its epilogue: the bits of nc_matmul_i8_token (bias, no residual) followed by
// nc_rope_append with the cache's table (q rotated in place; k rotated and v
// copied into the cache at positions past + i; k and v left in qkv as
// projected), in one launch. The tile is one head wide: 64 x 64 when that
// gives 576 tiles or more, else 32 x 64 (head_dim 64); 32 x 32 (head_dim 32).
// (Measured on MI355X, Qwen2.5-0.5B's qkv, 32 x 64 against 64 x 64: M = 128
// 5.00 / 6.73 us, 512 6.53 / 7.13, 1024 8.37 / 8.66, 2048 11.78 / 11.40.)
// p: [qkv f32[M,W] (out), xq i8[M,K], xs f32[M], q i8[W,K], scales f32[W], bias f32[W] | NULL,
//     kcache f32[kv,C,D], vcache f32[kv,C,D], rope table f32[2,C,D/2], pos i64[1] | NULL];
// s: [M, W, K, heads, kv, D, past, C, schedule]  (W = (heads + 2 kv) D, D 32 or 64, K a multiple of 16;
//    schedule 0 the library's tile, or an MFMA tile 16..24 one head wide)
NC_EXPORT int32_t nc_matmul_i8_token_rope(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[6] && p[7] && p[8],
               "nc_matmul_i8_token_rope: null operand");
    const int64_t M = s[0], W = s[1], K = s[2], heads = s[3], kv = s[4], D = s[5], past = s[6], C = s[7];
    const int64_t *pos = (const int64_t *)p[9];
    NC_REQUIRE(M >= 0 && M < (1 << 24) && K > 0 && K % 16 == 0 && K < (1 << 24) && heads > 0 && kv > 0 &&
                   heads % kv == 0 && (D == 32 || D == 64) && W == (heads + 2 * kv) * D && C > 0 &&
                   C < (1 << 24) && (pos || (past >= 0 && past + M <= C)),
               "nc_matmul_i8_token_rope: bad shape (W = (heads + 2 kv) D, D 32 or 64, past + M <= C)");
    const int64_t schedule = s[8];
    NC_REQUIRE(schedule == 0 || (schedule >= kGemmFirstSchedule && schedule < kGemmFirstSchedule + kGemmTileCount),
               "nc_matmul_i8_token_rope: no such schedule (0, or an MFMA tile 16..24 one head wide)");
    if (M == 0) return NC_OK;
    int tile = 2;
    if (D == 64) tile = ((M + 63) / 64) * (W / 64) >= 576 ? 5 : 1;
    if (schedule) tile = (int)(schedule - kGemmFirstSchedule);
    GemmArgs a{p[0], (const int8_t *)p[1], (const float *)p[2], (const int8_t *)p[3], (const float *)p[4],
               (const float *)p[5], nullptr, nullptr, nullptr, (int)M, (int)W, (int)K};
    a.rope = RopeArgs{(float *)p[6], (float *)p[7], (const float *)p[8], pos, nc::error_word(), (int)heads,
                      (int)kv, pos ? 0 : (int)past, (int)C, (int)D};
    return nc::gemm_i8_token_rope(tile, a);
}
