// Shared device helpers for the gfx950 kernels of nanocompile_amd.
//
// Everything here is exact or has one stated order:
//  * int8 dot products go through v_dot4_i32_i8 (__builtin_amdgcn_sdot4),
//    which is exact in int32 for every operand this library produces
//    (|acc| <= 127 * 127 * K, below 2^31 for K < 133,000);
//  * float reductions across a wavefront are a fixed xor butterfly
//    (offsets 32, 16, 8, 4, 2, 1), so every lane ends with the same bits and
//    the host oracle can replay the same tree;
//  * rounding follows the reference's two rules: C's roundf (half away from
//    zero, exact) for activations (ir.py:244-247, interpreter.py:192-201), and
//    the weight quantizer's float32 floor(|s| + 0.5) (quantize.py:68).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define NC_EXPORT extern "C" __attribute__((visibility("default")))

#define NC_OK 0
#define NC_FAIL_INDEX 1      // a gather index out of range (loopir.Fail code 1)
#define NC_BAD_ARGS 2        // the host launcher rejected a shape or pointer
#define NC_LAUNCH_FAILED 3   // the HIP runtime refused the launch
#define NC_FAIL_CAPACITY 4   // a device-side position ran past the KV cache's capacity

namespace nc {

// 16 int8 values as four dwords: one global_load_dwordx4.
struct alignas(16) i8x16 { int32_t w[4]; };

__device__ __forceinline__ int32_t dot4(int32_t a, int32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot4(a, b, acc, false);
}

__device__ __forceinline__ int32_t dot16(const i8x16 &a, const i8x16 &b, int32_t acc) {
    acc = dot4(a.w[0], b.w[0], acc);
    acc = dot4(a.w[1], b.w[1], acc);
    acc = dot4(a.w[2], b.w[2], acc);
    acc = dot4(a.w[3], b.w[3], acc);
    return acc;
}

__device__ __forceinline__ i8x16 load16(const int8_t *p) {
    return *reinterpret_cast<const i8x16 *>(p);
}

__device__ __forceinline__ i8x16 load16_stream(const int8_t *p) {
    // Weights are read once per step: a non-temporal load keeps them from
    // evicting the activations and the KV cache from L2.
    i8x16 v;
    const int32_t *q = reinterpret_cast<const int32_t *>(p);
    v.w[0] = __builtin_nontemporal_load(q + 0);
    v.w[1] = __builtin_nontemporal_load(q + 1);
    v.w[2] = __builtin_nontemporal_load(q + 2);
    v.w[3] = __builtin_nontemporal_load(q + 3);
    return v;
}

// Lane exchanges without an LDS round trip (__shfl_xor compiles to
// ds_bpermute, ~100 cycles of latency a step). For a commutative f, one
// gfx950 lane swap gives every lane f(v[i], v[i ^ 32]) (v_permlane32_swap)
// or f(v[i], v[i ^ 16]) (v_permlane16_swap): swapping v with itself leaves
// v[i] in one result and v[i ^ off] in the other, in an order that differs
// between the two halves, which commutativity makes immaterial. The partners
// i ^ 8, 4, 2, 1 come from DPP within rows of 16 lanes: row_ror:8 is xor 8;
// xor 4 takes row_ror:4 into the banks of lanes with bit 2 set (source
// lane - 4) and row_ror:12 into the others (source lane + 4); xor 2 and xor 1
// are quad permutations.
// With every row and bank enabled and a source lane for every lane (the
// rotations and quad permutations here), a DPP move never keeps its old
// value and never reads an invalid lane, so neither the old value nor
// bound_ctrl changes the result; mov_dpp with bound_ctrl set is the form the
// compiler folds into the instruction that uses it (v_add_f32_dpp and the
// like). The xor-4 partner writes half the banks in each of two moves, so the
// first move's result is the second's old value.
template <int CTRL>
__device__ __forceinline__ int32_t dpp_all(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

template <int CTRL, int BANKS>
__device__ __forceinline__ int32_t dpp_mov(int32_t old, int32_t v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, 0xF, BANKS, false);
}

template <int OFF>
__device__ __forceinline__ int32_t xor_partner(int32_t v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8, "DPP partners within a row of 16");
    if constexpr (OFF == 1) return dpp_all<0xB1>(v);                  // quad_perm [1, 0, 3, 2]
    else if constexpr (OFF == 2) return dpp_all<0x4E>(v);             // quad_perm [2, 3, 0, 1]
    else if constexpr (OFF == 4) return dpp_mov<0x12C, 0x5>(dpp_mov<0x124, 0xA>(v, v), v);
    else return dpp_all<0x128>(v);                                    // row_ror:8
}

template <int OFF>
__device__ __forceinline__ float xor_partner(float v) {
    return __int_as_float(xor_partner<OFF>(__float_as_int(v)));
}

// f(v[i], v[i ^ OFF]) in every lane, OFF a power of two <= 32, f commutative.
template <int OFF, typename T, typename F>
__device__ __forceinline__ T butterfly_step(T v, F f) {
    if constexpr (OFF >= 16) {
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                                 : __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return f(__builtin_bit_cast(T, (uint32_t)r[0]), __builtin_bit_cast(T, (uint32_t)r[1]));
    } else {
        return f(v, xor_partner<OFF>(v));
    }
}

// The xor butterfly over aligned groups of G lanes (G a power of two <= 64):
// steps G / 2, ..., 2, 1, each lane combining with lane i ^ step.
template <int G, typename T, typename F>
__device__ __forceinline__ T butterfly(T v, F f) {
    if constexpr (G >= 64) v = butterfly_step<32>(v, f);
    if constexpr (G >= 32) v = butterfly_step<16>(v, f);
    if constexpr (G >= 16) v = butterfly_step<8>(v, f);
    if constexpr (G >= 8) v = butterfly_step<4>(v, f);
    if constexpr (G >= 4) v = butterfly_step<2>(v, f);
    if constexpr (G >= 2) v = butterfly_step<1>(v, f);
    return v;
}

// Sum over the L lanes of an aligned group (L a power of two <= 64). Integer
// addition is exact, so the order is immaterial.
template <int L>
__device__ __forceinline__ int32_t group_sum_i32(int32_t v) {
    return butterfly<L>(v, [](int32_t a, int32_t b) { return a + b; });
}

// Sum over a whole wavefront, the butterfly (v[i] + v[i ^ off]) for
// off = 32, 16, 8, 4, 2, 1. Addition commutes, so all lanes agree bitwise.
__device__ __forceinline__ float wave_sum_f32(float v) {
    return butterfly<64>(v, [](float a, float b) { return __fadd_rn(a, b); });
}

// max that propagates NaN from either side, as the reference's reduce_max
// does (acc < v || v != v, fusion.py:603-609) and numpy's max does; fmaxf
// would drop a NaN and give a NaN row a finite int8 scale.
__device__ __forceinline__ float nan_max(float a, float b) { return (a < b || b != b) ? b : a; }

// Maximum over a wavefront, the same xor butterfly; NaN propagates.
__device__ __forceinline__ float wave_max_f32(float v) {
    return butterfly<64>(v, [](float a, float b) { return nan_max(a, b); });
}

// Correctly rounded float32 square root. Not __fsqrt_rn: without
// OCML_BASIC_ROUNDED_OPERATIONS, HIP maps that to the approximate native
// sqrt. llvm.sqrt.f32 is expanded to the correctly rounded sequence under
// -fhip-fp32-correctly-rounded-divide-sqrt, which the build passes (and which
// also makes plain float division correctly rounded).
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }

// C's roundf: half away from zero, exact for every float.
__device__ __forceinline__ float round_half_away(float v) { return __builtin_roundf(v); }

// Per-token activation quantization of one value (the reference's
// quantize_activations with one block spanning the row, quantize.py:116-121):
// clamp(round(x / scale), -127, 127), the division correctly rounded.
__device__ __forceinline__ int8_t quantize_value(float x, float scale) {
    float r = round_half_away(div_rn(x, scale));
    r = r <= 127.0f ? r : 127.0f;
    r = -127.0f <= r ? r : -127.0f;
    return static_cast<int8_t>(r);
}

// The activation scale from a row maximum: where(mag <= 0, 1, mag / 127).
__device__ __forceinline__ float token_scale(float magnitude) {
    return magnitude <= 0.0f ? 1.0f : div_rn(magnitude, 127.0f);
}

}  // namespace nc

// Host side: the library stream and error word (nc_runtime.hip), shared by
// every launcher.
namespace nc {
hipStream_t stream();
int device();              // the device nc_init bound the library to, or -1
int32_t *error_word();
// NC_OK, or NC_LAUNCH_FAILED with the message recorded for nc_last_error().
int32_t launched(const char *what);
void set_message(const char *text);

// The MFMA GEMM (nc_gemm.hip): tile index 0..8, epilogue 0 = dequantize
// (+ bias, + residual), 1 = raw int32 accumulators, 2 = SwiGLU pair (q2, ws2).
// K must be a multiple of 16.
int32_t gemm_i8_token(int tile, int epi, void *out, const int8_t *xq, const float *xs, const int8_t *q,
                      const float *ws, const float *bias, const float *residual, const int8_t *q2,
                      const float *ws2, int M, int N, int K);
// A tile's primitives: [BM, BN, BK, WM, WN, NS, threads, LDS bytes]; NC_BAD_ARGS past the table.
int32_t gemm_tile_info(int tile, int64_t *out);
// Looks up, with `device` current, the address of that device's copy of the
// attention workspace the library holds for nc_attention_decode_static
// (nc_attention.hip); called once per device by nc_init.
int32_t attention_scratch_init(int device);
// The per-token quantizer (nc_quant.hip) on M rows of K: xq, xs from x.
int32_t quantize_token_rows(int8_t *xq, float *xs, const float *x, int M, int K);
}  // namespace nc

namespace nc {
// A float32 passed through an int64 size slot (eps, scale): its bits in the low 32.
inline float bits_to_float(int64_t bits) {
    const uint32_t u = (uint32_t)bits;
    float f;
    __builtin_memcpy(&f, &u, sizeof f);
    return f;
}
}  // namespace nc

// A launcher's argument checks: on failure, record why and return NC_BAD_ARGS.
#define NC_REQUIRE(cond, text)                 \
    do {                                       \
        if (!(cond)) {                         \
            nc::set_message(text);             \
            return NC_BAD_ARGS;                \
        }                                      \
    } while (0)
