// The per-token int8 projection, decode shape: y[m, n] for a few tokens m and
// every weight row n, streamed from HBM once.
//
//   acc[m, n] = sum_k xq[m, k] * q[n, k]           exact, int32
//   y[m, n]   = (f32(acc) * xs[m]) * scales[n]      two rounded multiplies
//             (+ bias[n]) (residual[m, n] + ...)    each one rounded add
//
// This is the build's primitive matmul_i8_token. The reference has no
// per-token mode (its int8 modes are ir.py:392-439); the epilogue order above
// is the one this library freezes, and the oracle restates it. The weight
// format is the reference's per-row int8 (quantize.py:55-70): q row-major
// [N, K], one f32 scale per row.
//
// Layout on the chip: a group of L lanes owns one weight row. Each lane reads
// 16 bytes at a time (global_load_dwordx4), and the L lanes of a group read
// L * 16 consecutive bytes, so at L = 8 each load instruction takes whole
// 128-byte lines. Activations are staged once per workgroup in LDS. The L
// partial sums are added with lane shuffles, exact in int32, and lane 0 of
// the group applies the epilogue.
#include "nc_common.h"
#include "nc_epilogue.h"

namespace {

using nc::i8x16;

template <int KS, int L, int WAVES, int MT, bool ACC_OUT, bool STACKED>
__global__ __launch_bounds__(64 * WAVES) void gemv_i8_token(
    void *__restrict__ out, const int8_t *__restrict__ xq, const float *__restrict__ xs,
    const int8_t *__restrict__ q, const float *__restrict__ ws, const float *__restrict__ bias,
    const float *__restrict__ residual, int M, int N, int Kr) {
    constexpr int ROWS = (64 / L) * WAVES;
    constexpr int STEP = L * 16;
    const int K = KS ? KS : Kr;
    extern __shared__ __align__(16) int8_t sx[];
    if constexpr (STACKED) {   // nc_matmul_i8_token_stacked: problem z has its own operands
        const size_t z = blockIdx.z;
        q += z * (size_t)N * K;
        ws += z * (size_t)N;
        xq += z * (size_t)M * K;
        xs += z * (size_t)M;
        out = static_cast<char *>(out) + z * (size_t)M * N * 4;
    }

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane & (L - 1), grp = lane / L;
    const int n = blockIdx.x * ROWS + wave * (64 / L) + grp;
    const int8_t *row = q + (size_t)(n < N ? n : 0) * K;

    // With K known here, the row's chunks are loaded into registers first, so
    // they are in flight while the activations are staged (a row left in the
    // loop below would wait for the staging's barrier before its first load).
    constexpr int KITERS = KS ? (KS + STEP - 1) / STEP : 1;
    i8x16 w[KITERS];
    if constexpr (KS > 0) {
#pragma unroll
        for (int it = 0; it < KITERS; ++it) {
            const int c = it * STEP + sub * 16;
            if (KS % STEP == 0 || c < KS) w[it] = nc::load16_stream(row + c);
        }
    }

    const int m0 = blockIdx.y * MT;
    const int mt = min(MT, M - m0);
    const int chunks = K / 16;
    for (int i = threadIdx.x; i < MT * chunks; i += 64 * WAVES) {
        const int m = i / chunks, c = i - m * chunks;
        i8x16 v = {};
        if (m < mt) v = nc::load16(xq + (size_t)(m0 + m) * K + c * 16);
        *reinterpret_cast<i8x16 *>(sx + m * K + c * 16) = v;
    }
    __syncthreads();

    int32_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0;
    if constexpr (KS > 0) {
#pragma unroll
        for (int it = 0; it < KITERS; ++it) {
            const int c = it * STEP + sub * 16;
            if (KS % STEP == 0 || c < KS) {
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    acc[m] = nc::dot16(w[it], *reinterpret_cast<const i8x16 *>(sx + m * K + c), acc[m]);
            }
        }
    } else if (n < N) {
        const int iters = (K + STEP - 1) / STEP;
        for (int it = 0; it < iters; ++it) {
            const int c = it * STEP + sub * 16;
            if (K % STEP == 0 || c < K) {
                const i8x16 wv = nc::load16_stream(row + c);
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    acc[m] = nc::dot16(wv, *reinterpret_cast<const i8x16 *>(sx + m * K + c), acc[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = nc::group_sum_i32<L>(acc[m]);

    if (sub == 0 && n < N) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= mt) break;
            const size_t at = (size_t)(m0 + m) * N + n;
            if constexpr (ACC_OUT) {
                static_cast<int32_t *>(out)[at] = acc[m];
            } else {
                float v = __fmul_rn(__fmul_rn((float)acc[m], xs[m0 + m]), ws[n]);
                if (bias) v = __fadd_rn(v, bias[n]);
                if (residual) v = __fadd_rn(residual[at], v);
                static_cast<float *>(out)[at] = v;
            }
        }
    }
}

// The SwiGLU pair: gate row n and up row n read by the same lane group, sharing
// the activation chunks (the reference's gate and up share one k loop,
// fusion.py:677-711), then h[m, n] = silu(gate) * up with each projection's
// own epilogue (f32(acc) * xs[m]) * scales[n].
template <int KS, int L, int MT>
__global__ __launch_bounds__(64) void gemv_i8_token_swiglu(
    float *__restrict__ h, const int8_t *__restrict__ xq, const float *__restrict__ xs,
    const int8_t *__restrict__ qg, const float *__restrict__ wsg, const int8_t *__restrict__ qu,
    const float *__restrict__ wsu, int M, int N, int Kr) {
    constexpr int ROWS = 64 / L;
    constexpr int STEP = L * 16;
    const int K = KS ? KS : Kr;
    extern __shared__ __align__(16) int8_t sx[];
    const int m0 = blockIdx.y * MT;
    const int mt = min(MT, M - m0);
    const int chunks = K / 16;
    for (int i = threadIdx.x; i < MT * chunks; i += 64) {
        const int m = i / chunks, c = i - m * chunks;
        i8x16 v = {};
        if (m < mt) v = nc::load16(xq + (size_t)(m0 + m) * K + c * 16);
        *reinterpret_cast<i8x16 *>(sx + m * K + c * 16) = v;
    }
    __syncthreads();
    const int lane = threadIdx.x;
    const int sub = lane & (L - 1), grp = lane / L;
    const int n = blockIdx.x * ROWS + grp;
    int32_t ag[MT], au[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ag[m] = au[m] = 0;
    if (n < N) {
        const int8_t *rg = qg + (size_t)n * K, *ru = qu + (size_t)n * K;
        const int iters = (K + STEP - 1) / STEP;
#pragma unroll
        for (int it = 0; it < iters; ++it) {
            const int c = it * STEP + sub * 16;
            if (K % STEP == 0 || c < K) {
                const i8x16 wg = nc::load16_stream(rg + c), wu = nc::load16_stream(ru + c);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const i8x16 x = *reinterpret_cast<const i8x16 *>(sx + m * K + c);
                    ag[m] = nc::dot16(wg, x, ag[m]);
                    au[m] = nc::dot16(wu, x, au[m]);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        ag[m] = nc::group_sum_i32<L>(ag[m]);
        au[m] = nc::group_sum_i32<L>(au[m]);
    }
    if (sub == 0 && n < N) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= mt) break;
            const float x = xs[m0 + m];
            const float g = __fmul_rn(__fmul_rn((float)ag[m], x), wsg[n]);
            const float u = __fmul_rn(__fmul_rn((float)au[m], x), wsu[n]);
            h[(size_t)(m0 + m) * N + n] = nc::silu_mul(g, u);
        }
    }
}

// Any K, byte by byte: the path for widths that are not a whole number of
// 16-byte chunks (the reference's test widths 77 and 40, say). One wave per
// row; the same exact sum and the same epilogue.
template <bool ACC_OUT>
__global__ __launch_bounds__(64) void gemv_i8_token_bytes(
    void *__restrict__ out, const int8_t *__restrict__ xq, const float *__restrict__ xs,
    const int8_t *__restrict__ q, const float *__restrict__ ws, const float *__restrict__ bias,
    const float *__restrict__ residual, int M, int N, int K) {
    const int n = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int8_t *row = q + (size_t)n * K;
    const int8_t *x = xq + (size_t)m * K;
    int32_t acc = 0;
    for (int k = lane; k < K; k += 64) acc += (int32_t)row[k] * (int32_t)x[k];
    acc = nc::group_sum_i32<64>(acc);
    if (lane == 0) {
        const size_t at = (size_t)m * N + n;
        if constexpr (ACC_OUT) {
            static_cast<int32_t *>(out)[at] = acc;
        } else {
            float v = __fmul_rn(__fmul_rn((float)acc, xs[m]), ws[n]);
            if (bias) v = __fadd_rn(v, bias[n]);
            if (residual) v = __fadd_rn(residual[at], v);
            static_cast<float *>(out)[at] = v;
        }
    }
}

struct Args {
    void *out;
    const int8_t *xq;
    const float *xs;
    const int8_t *q;
    const float *ws;
    const float *bias;
    const float *residual;
    int M, N, K;
    int batch;
};

template <int KS, int L, int WAVES, int MT, bool ACC_OUT>
int32_t launch(const Args &a) {
    constexpr int ROWS = (64 / L) * WAVES;
    dim3 grid((a.N + ROWS - 1) / ROWS, (a.M + MT - 1) / MT, a.batch);
    size_t lds = (size_t)MT * a.K;
    if (a.batch > 1)
        hipLaunchKernelGGL((gemv_i8_token<KS, L, WAVES, MT, ACC_OUT, true>), grid, dim3(64 * WAVES), lds,
                           nc::stream(), a.out, a.xq, a.xs, a.q, a.ws, a.bias, a.residual, a.M, a.N, a.K);
    else
        hipLaunchKernelGGL((gemv_i8_token<KS, L, WAVES, MT, ACC_OUT, false>), grid, dim3(64 * WAVES), lds,
                           nc::stream(), a.out, a.xq, a.xs, a.q, a.ws, a.bias, a.residual, a.M, a.N, a.K);
    return nc::launched("gemv_i8_token");
}

template <bool ACC_OUT>
int32_t launch_bytes(const Args &a) {
    hipLaunchKernelGGL((gemv_i8_token_bytes<ACC_OUT>), dim3(a.N, a.M), dim3(64), 0, nc::stream(), a.out, a.xq, a.xs,
                       a.q, a.ws, a.bias, a.residual, a.M, a.N, a.K);
    return nc::launched("gemv_i8_token_bytes");
}

// The schedule space of the projection (one index space for the GEMV and
// the MFMA GEMM):
//   0            the default: gemv_schedule_default below for few tokens,
//                else the MFMA tile auto_tile picks;
//   1..7         the GEMV with lanes per row L and waves per workgroup
//                (7 is the default GEMV, L = 8, one wave); the token tile MT follows M;
//   16..16+8     the MFMA GEMM's tiles (nc_gemm.hip), K a multiple of 16.
// (index, lanes per row L, waves per workgroup)
#define NC_GEMV_SCHEDULES(X) X(1, 4, 1) X(2, 16, 1) X(3, 8, 2) X(4, 8, 4) X(5, 4, 2) X(6, 16, 2) X(7, 8, 1)
constexpr int kGemmFirst = 16;
constexpr int kGemmTiles = 9;
constexpr int kGemmMinTokens = 16;

// The MFMA tile for a shape when the caller asks for the default, from a sweep
// of every tile on MI355X over the model's shapes at M = 128 .. 1024 (with the
// GEMM's conflict-free LDS layout): 64 x 128 (8 waves) for the largest
// problems and for long k loops with many tiles; 64 x 64 from 200 such tiles
// (gate at M = 512: 10.19 us against 11.65 with 32 x 64; down at M = 1024:
// 15.97 against 17.5-20.9); else 32 x 32 (at M = 512: q/o 4.53 us against
// 4.70 with 32 x 64, qkv 5.25 against 5.52 with 64 x 64, down 11.09 against
// 11.30 with 32 x 64 and 8 stages; gate at M = 128: 5.29 against 5.57).
int auto_tile(int M, int N, int K) {
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    const int t64 = tiles(64, 64);
    if (t64 >= 1792 || (K >= 2048 && t64 >= 256)) return 6;
    if (t64 >= 200) return 5;
    return 2;
}

// The SwiGLU pair's default: 64 x 64 with two register stages (its tiles
// stage two weight blocks, so deeper rings cost occupancy) from 400 such
// tiles, else 32 x 32 (measured at N = 4864, K = 896: M = 384 / 512 / 1024 /
// 2048: 15.7 / 19.3 / 30.5 / 54.1 us against 16.8 / 20.6 / 35.2 / 68.1 with
// 32 x 32 and 17.3 / 20.6 / 34.9 / 63.3 with 32 x 64; M = 128 / 256: 8.41 /
// 12.13 us with 32 x 32 against 11.0 / 14.6 with 64 x 64).
int auto_tile_pair(int M, int N, int K) {
    (void)K;
    const int t64 = ((M + 63) / 64) * ((N + 63) / 64);
    return t64 >= 400 ? 5 : 2;
}

template <int KS, int MT, bool ACC_OUT>
int32_t dispatch_schedule(const Args &a, int schedule) {
#define NC_GEMV_CASE(I, L, W) \
    case I: return launch<KS, L, W, MT, ACC_OUT>(a);
    switch (schedule) {
        case 0: return launch<KS, 8, 1, MT, ACC_OUT>(a);
        NC_GEMV_SCHEDULES(NC_GEMV_CASE)
        default: nc::set_message("gemv_i8_token: no such schedule"); return NC_BAD_ARGS;
    }
#undef NC_GEMV_CASE
}

template <int KS, bool ACC_OUT>
int32_t dispatch_tokens(const Args &a, int schedule) {
    if (a.M == 1) return dispatch_schedule<KS, 1, ACC_OUT>(a, schedule);
    if (a.M == 2) return dispatch_schedule<KS, 2, ACC_OUT>(a, schedule);
    if (a.M <= 4) return dispatch_schedule<KS, 4, ACC_OUT>(a, schedule);
    return dispatch_schedule<KS, 8, ACC_OUT>(a, schedule);
}

template <bool ACC_OUT>
int32_t run(const Args &a, int schedule) {
    if (a.M == 0 || a.N == 0) return NC_OK;
    if (schedule < 0 || (schedule > 7 && schedule < kGemmFirst) || schedule >= kGemmFirst + kGemmTiles) {
        nc::set_message("matmul_i8_token: no such schedule");
        return NC_BAD_ARGS;
    }
    const bool gemm_ok = a.batch == 1 && a.K % 16 == 0;
    if (schedule >= kGemmFirst && !gemm_ok) {
        nc::set_message("matmul_i8_token: the MFMA schedules need K a multiple of 16 and one problem");
        return NC_BAD_ARGS;
    }
    if (schedule == 0 && gemm_ok && a.M >= kGemmMinTokens) schedule = kGemmFirst + auto_tile(a.M, a.N, a.K);
    if (schedule >= kGemmFirst)
        return nc::gemm_i8_token(schedule - kGemmFirst, ACC_OUT ? 1 : 0, a.out, a.xq, a.xs, a.q, a.ws, a.bias,
                                 a.residual, nullptr, nullptr, a.M, a.N, a.K);
    if (a.K % 16 != 0 || (size_t)8 * a.K > 65536) {
        if (a.batch != 1) { nc::set_message("stacked GEMV needs K a multiple of 16"); return NC_BAD_ARGS; }
        return launch_bytes<ACC_OUT>(a);
    }
    if (a.K == 896) return dispatch_tokens<896, ACC_OUT>(a, schedule);
    if (a.K == 4864) return dispatch_tokens<4864, ACC_OUT>(a, schedule);
    return dispatch_tokens<0, ACC_OUT>(a, schedule);
}

}  // namespace

// What schedule index `schedule` of the projection is, for the tuner; a
// table lookup, no device call.
// out[0] = 0 (GEMV): out[1..3] = [lanes per row, waves per workgroup, bytes per lane load];
// out[0] = 1 (MFMA GEMM): out[1..9] = [BM, BN, BK, WM, WN, NS, threads, LDS bytes with one
// weight matrix, LDS bytes with the SwiGLU pair].
// Schedule 0 (the default) reports NC_BAD_ARGS: it is a choice, not a schedule.
NC_EXPORT int32_t nc_schedule_info(int32_t schedule, int64_t *out) {
    if (!out) return NC_BAD_ARGS;
#define NC_GEMV_INFO(I, L, W) \
    if (schedule == I) {      \
        out[0] = 0;           \
        out[1] = L;           \
        out[2] = W;           \
        out[3] = 16;          \
        return NC_OK;         \
    }
    NC_GEMV_SCHEDULES(NC_GEMV_INFO)
#undef NC_GEMV_INFO
    if (schedule >= kGemmFirst && schedule < kGemmFirst + kGemmTiles) {
        out[0] = 1;
        return nc::gemm_tile_info(schedule - kGemmFirst, out + 1);
    }
    return NC_BAD_ARGS;
}

// p: [y f32[M,N], xq i8[M,K], xs f32[M], q i8[N,K], scales f32[N], bias f32[N] | NULL,
//     residual f32[M,N] | NULL];  s: [M, N, K, schedule]
NC_EXPORT int32_t nc_matmul_i8_token(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_matmul_i8_token: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] >= 0 && s[2] > 0 && s[0] < (1 << 24) && s[1] < (1 << 24) && s[2] < (1 << 24),
               "nc_matmul_i8_token: bad shape");
    Args a{p[0], (const int8_t *)p[1], (const float *)p[2], (const int8_t *)p[3], (const float *)p[4],
           (const float *)p[5], (const float *)p[6], (int)s[0], (int)s[1], (int)s[2], 1};
    return run<false>(a, (int)s[3]);
}

// p: [acc i32[M,N], xq i8[M,K], q i8[N,K]];  s: [M, N, K, schedule]
NC_EXPORT int32_t nc_matmul_i8_token_acc(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2], "nc_matmul_i8_token_acc: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] >= 0 && s[2] > 0 && s[0] < (1 << 24) && s[1] < (1 << 24) && s[2] < (1 << 24),
               "nc_matmul_i8_token_acc: bad shape");
    Args a{p[0], (const int8_t *)p[1], nullptr, (const int8_t *)p[2], nullptr, nullptr, nullptr,
           (int)s[0], (int)s[1], (int)s[2], 1};
    return run<true>(a, (int)s[3]);
}

// B independent projections in one launch, problem z reading its own weights:
// the steady state of a stream of decode GEMVs over rotated weight copies.
// p: [y f32[B,M,N], xq i8[B,M,K], xs f32[B,M], q i8[B,N,K], scales f32[B,N]];
// s: [B, M, N, K, schedule]
NC_EXPORT int32_t nc_matmul_i8_token_stacked(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4], "nc_matmul_i8_token_stacked: null operand");
    NC_REQUIRE(s[0] > 0 && s[0] < 65536 && s[1] >= 0 && s[2] >= 0 && s[3] > 0 && s[1] < (1 << 24) &&
                   s[2] < (1 << 24) && s[3] < (1 << 24),
               "nc_matmul_i8_token_stacked: bad shape");
    Args a{p[0], (const int8_t *)p[1], (const float *)p[2], (const int8_t *)p[3], (const float *)p[4],
           nullptr, nullptr, (int)s[1], (int)s[2], (int)s[3], (int)s[0]};
    return run<false>(a, (int)s[4]);
}

namespace {
template <int KS, int MT>
int32_t launch_swiglu(float *h, const int8_t *xq, const float *xs, const int8_t *qg, const float *wsg,
                      const int8_t *qu, const float *wsu, int M, int N, int K) {
    constexpr int L = 8;
    dim3 grid((N + 64 / L - 1) / (64 / L), (M + MT - 1) / MT);
    hipLaunchKernelGGL((gemv_i8_token_swiglu<KS, L, MT>), grid, dim3(64), (size_t)MT * K, nc::stream(), h, xq, xs,
                       qg, wsg, qu, wsu, M, N, K);
    return nc::launched("gemv_i8_token_swiglu");
}

template <int KS>
int32_t swiglu_tokens(float *h, const int8_t *xq, const float *xs, const int8_t *qg, const float *wsg,
                      const int8_t *qu, const float *wsu, int M, int N, int K) {
    if (M == 1) return launch_swiglu<KS, 1>(h, xq, xs, qg, wsg, qu, wsu, M, N, K);
    if (M <= 4) return launch_swiglu<KS, 4>(h, xq, xs, qg, wsg, qu, wsu, M, N, K);
    return launch_swiglu<KS, 8>(h, xq, xs, qg, wsg, qu, wsu, M, N, K);
}
}  // namespace

// h = silu((f32(xq @ qg.T) * xs) * sg) * ((f32(xq @ qu.T) * xs) * su), one kernel.
// p: [h f32[M,N], xq i8[M,K], xs f32[M], qg i8[N,K], sg f32[N], qu i8[N,K], su f32[N]];
// s: [M, N, K]  (K a multiple of 16, at most 8192)
NC_EXPORT int32_t nc_matmul_i8_token_swiglu(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && p[3] && p[4] && p[5] && p[6],
               "nc_matmul_i8_token_swiglu: null operand");
    NC_REQUIRE(s[0] >= 0 && s[1] >= 0 && s[2] > 0 && s[2] % 16 == 0 && s[2] <= 8192 && s[0] < (1 << 24) &&
                   s[1] < (1 << 24),
               "nc_matmul_i8_token_swiglu: bad shape (K must be a multiple of 16, at most 8192)");
    const int M = (int)s[0], N = (int)s[1], K = (int)s[2];
    int schedule = (int)s[3];
    NC_REQUIRE(schedule == 0 || schedule == 7 || (schedule >= kGemmFirst && schedule < kGemmFirst + kGemmTiles),
               "nc_matmul_i8_token_swiglu: no such schedule (0, 7 or an MFMA tile)");
    if (M == 0 || N == 0) return NC_OK;
    float *h = (float *)p[0];
    auto xq = (const int8_t *)p[1];
    auto xs = (const float *)p[2];
    auto qg = (const int8_t *)p[3];
    auto sg = (const float *)p[4];
    auto qu = (const int8_t *)p[5];
    auto su = (const float *)p[6];
    if (schedule == 0 && M >= kGemmMinTokens) schedule = kGemmFirst + auto_tile_pair(M, N, K);
    if (schedule >= kGemmFirst)
        return nc::gemm_i8_token(schedule - kGemmFirst, 2, h, xq, xs, qg, sg, nullptr, nullptr, qu, su, M, N, K);
    if (K == 896) return swiglu_tokens<896>(h, xq, xs, qg, sg, qu, su, M, N, K);
    return swiglu_tokens<0>(h, xq, xs, qg, sg, qu, su, M, N, K);
}

namespace {
__global__ void silu_mul_rows(float *__restrict__ y, const float *__restrict__ g, const float *__restrict__ u,
                              int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = nc::silu_mul(g[i], u[i]);
}
}  // namespace

// y = silu(g) * u elementwise (nn.py:41-54, the epilogue fusion puts on gate and up).
// p: [y f32[n], g f32[n], u f32[n]];  s: [n]
NC_EXPORT int32_t nc_silu_mul(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[2] && s[0] >= 0 && s[0] < (1LL << 40), "nc_silu_mul: bad operand");
    if (s[0] == 0) return NC_OK;
    hipLaunchKernelGGL(silu_mul_rows, dim3((unsigned)((s[0] + 255) / 256)), dim3(256), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const float *)p[2], s[0]);
    return nc::launched("silu_mul_rows");
}
