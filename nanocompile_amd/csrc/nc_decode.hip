// Decode-step projections (one new token), each with its activation prologue
// fused in. (Attention with RoPE and the cache append fused in is
// nc_attention_decode, nc_attention.hip.)
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
    static_assert(PRO == kQuant ? (W >= 1 && W <= 4) : (W == 1 || W == 4),
                  "rms_norm: one wave, or the row order's 256 threads; a maximum alone: up to 4 waves");
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
    for (int i = 0; i < PER; ++i) mag = nc::nan_max(mag, fabsf(v[i]));
    mag = nc::wave_max_f32(mag);
    if constexpr (W > 1) {
        if (lane == 0) scratch[4 + wave] = mag;
        __syncthreads();
        mag = scratch[4];
#pragma unroll
        for (int w = 1; w < W; ++w) mag = nc::nan_max(mag, scratch[4 + w]);
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

// A lane's chunks of its weight row: B bytes (16, 8 or 4) a load, L lanes
// a row, loads issued back to back. Integer sums are exact in any order, so
// every (L, B) gives the same accumulators.
template <int K, int L, int B>
struct RowChunks {
    static_assert(B == 16 || B == 8 || B == 4, "16-, 8- or 4-byte chunks");
    static constexpr int STEP = L * B;
    static constexpr int ITERS = K / STEP;
    static constexpr int DW = B / 4;                       // dwords a chunk
    static_assert(K % STEP == 0, "K must be a multiple of L B");
    int32_t w[ITERS][DW];

    __device__ __forceinline__ void load(const int8_t *__restrict__ row, int sub) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int32_t *q = reinterpret_cast<const int32_t *>(row + it * STEP + sub * B);
#pragma unroll
            for (int d = 0; d < DW; ++d) w[it][d] = __builtin_nontemporal_load(q + d);
        }
    }

    __device__ __forceinline__ int32_t dot(const int8_t *__restrict__ sxq, int sub) const {
        int32_t acc = 0;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int32_t *x = reinterpret_cast<const int32_t *>(sxq + it * STEP + sub * B);
#pragma unroll
            for (int d = 0; d < DW; ++d) acc = nc::dot4(w[it][d], x[d], acc);
        }
        return acc;
    }
};

// One decode projection: W waves a workgroup, 64 / L rows a wave (row pairs
// for SwiGLU), L lanes per row. The weight loads are issued first, so they
// are in flight while the workgroup computes its activation prologue, which
// its W waves share.
template <int K, int PRO, int EPI, int L, int W, int B>
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
    RowChunks<K, L, B> w1, w2;
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


// The 896-wide projections: one wave, 8 lanes a row, 16-byte loads (one
// 128-byte line a load), 8 rows a workgroup. The long down projection: 4 waves,
// whose 4864-wide prologue would otherwise cost each lane 76 correctly rounded
// divisions, and a whole wave a row with 4-byte loads (a 256-byte line a
// load), so a workgroup holds 4 rows and the 896 rows spread over 224
// workgroups, not the 56 that 16 lanes of 16 bytes a row give. Measured on
// MI355X, decode tok/s in one box: down with 4 waves x (64 lanes, 4 B) 1642-1650,
// (32 lanes, 8 B) 1608-1611, (16 lanes, 16 B) 1589; with 2 or 1 waves x
// (64 lanes, 4 B) 1530 / 1496; the 896-wide projections with 4 waves of 32
// lanes of 4 B (the prologue shared) 1508-1592, with 2 or 4 rows a one-wave
// workgroup (more workgroups) unchanged.
template <int K, int PRO, int EPI, int L = (K >= 4096 ? 64 : kL), int W = (K >= 4096 ? 4 : 1),
          int B = (K >= 4096 ? 4 : 16)>
int32_t launch_decode(void **p, int N, float eps) {
    constexpr int ROWS = W * 64 / L;
    hipLaunchKernelGGL((gemv_decode<K, PRO, EPI, L, W, B>), dim3((N + ROWS - 1) / ROWS), dim3(64 * W), 0, nc::stream(),
                       (float *)p[0], (const float *)p[1], (const float *)p[2], eps, (const int8_t *)p[3],
                       (const float *)p[4], (const float *)p[5], (const int8_t *)p[6], (const float *)p[7], N);
    return nc::launched("gemv_decode");
}

// The schedules a tuner may choose for the model's two widths: (lanes a row,
// waves a workgroup, bytes a load), schedule s at row s - 1 (schedule 0 is the
// library's choice, the first row). Every row computes the same bits: the
// prologue's order does not depend on W (the row-sum order's 256 virtual
// threads either way) and integer dot products are exact in any order. An
// rms_norm prologue takes 1 or 4 waves.
#define NC_DECODE_896(X) X(1, 8, 1, 16) X(2, 4, 1, 16) X(3, 16, 1, 8) X(4, 8, 4, 16) X(5, 16, 4, 8)
#define NC_DECODE_4864(X) X(1, 64, 4, 4) X(2, 16, 4, 16) X(3, 32, 4, 8) X(4, 64, 2, 4) X(5, 32, 2, 8)
constexpr int kDecodeSchedules = 5;

template <int K, int PRO, int EPI>
int32_t launch_scheduled(void **p, int N, float eps, int schedule) {
#define NC_DECODE_CASE(S, L, W, B)                                                            \
    case S:                                                                                   \
        if constexpr (PRO == kQuant || W == 1 || W == 4) return launch_decode<K, PRO, EPI, L, W, B>(p, N, eps); \
        break;
    if constexpr (K == 896) {
        switch (schedule) { NC_DECODE_896(NC_DECODE_CASE) default: break; }
    } else if constexpr (K == 4864) {
        switch (schedule) { NC_DECODE_4864(NC_DECODE_CASE) default: break; }
    }
#undef NC_DECODE_CASE
    nc::set_message("nc_decode_projection: no such schedule for this width and kind");
    return NC_BAD_ARGS;
}

}  // namespace

// A decode projection schedule's launch shape, for the tuner (no device call):
// out = [lanes a row, waves a workgroup, bytes a load]; NC_BAD_ARGS when the
// schedule does not exist for width K and kind (an rms_norm prologue, kinds 0
// and 2, takes 1 or 4 waves).
NC_EXPORT int32_t nc_decode_schedule_info(int64_t K, int64_t kind, int64_t schedule, int64_t *out) {
    if (!out || kind < 0 || kind > 2) return NC_BAD_ARGS;
#define NC_DECODE_INFO(S, L, W, B)                                        \
    if (schedule == S && (kind == 1 || W == 1 || W == 4)) {               \
        out[0] = L;                                                       \
        out[1] = W;                                                       \
        out[2] = B;                                                       \
        return NC_OK;                                                     \
    }
    if (K == 896) { NC_DECODE_896(NC_DECODE_INFO) }
    if (K == 4864 && kind == 1) { NC_DECODE_4864(NC_DECODE_INFO) }
#undef NC_DECODE_INFO
    return NC_BAD_ARGS;
}

// One decode projection with its activation prologue (see the file header).
// p: [out f32[N] (in: the residual for kind 1), x f32[K], gamma f32[K] | NULL,
//     q i8[N,K], scales f32[N], bias f32[N] | NULL, q2 i8[N,K] | NULL, scales2 f32[N] | NULL];
// s: [N, K, kind, eps as float32 bits, schedule] with kind 0 = rms_norm prologue + bias (q, k, v),
//    1 = quantize prologue + residual (o, down), 2 = rms_norm prologue + SwiGLU pair (gate, up);
//    schedule 0 the library's shape, 1..5 a row of the width's table (nc_decode_schedule_info).
//    K is 896 or 4864 (the model's widths; any other K uses the unfused kernels).
NC_EXPORT int32_t nc_decode_projection(void **p, const int64_t *s) {
    NC_REQUIRE(p && s && p[0] && p[1] && p[3] && p[4], "nc_decode_projection: null operand");
    const int64_t N = s[0], K = s[1], kind = s[2];
    const float eps = nc::bits_to_float(s[3]);
    NC_REQUIRE(N > 0 && N < (1 << 24) && kind >= 0 && kind <= 2, "nc_decode_projection: bad shape");
    NC_REQUIRE(kind == 1 || p[2], "nc_decode_projection: rms_norm needs gamma");
    NC_REQUIRE(kind != 0 || p[5], "nc_decode_projection: q, k, v need their bias");
    NC_REQUIRE(kind != 2 || (p[6] && p[7]), "nc_decode_projection: SwiGLU needs the up projection");
    const int64_t schedule = s[4];
    NC_REQUIRE(schedule >= 0 && schedule <= kDecodeSchedules, "nc_decode_projection: no such schedule");
    if (schedule > 0) {
        if (K == 896 && kind == 0) return launch_scheduled<896, kNorm, kBias>(p, (int)N, eps, (int)schedule);
        if (K == 896 && kind == 1) return launch_scheduled<896, kQuant, kResidual>(p, (int)N, eps, (int)schedule);
        if (K == 896 && kind == 2) return launch_scheduled<896, kNorm, kSwiglu>(p, (int)N, eps, (int)schedule);
        if (K == 4864 && kind == 1) return launch_scheduled<4864, kQuant, kResidual>(p, (int)N, eps, (int)schedule);
        nc::set_message("nc_decode_projection: schedules exist for the widths 896 and 4864 only");
        return NC_BAD_ARGS;
    }
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
