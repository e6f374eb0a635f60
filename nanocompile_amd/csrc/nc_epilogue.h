// The projection epilogues, shared by every int8 kernel so that the GEMV, the
// fused decode kernels and the MFMA GEMM produce the same bits.
//
//  * dequantization: y = (f32(acc) * xs[m]) * scales[n], two roundings in that
//    order; f32(acc) rounds to nearest even above 2^24;
//  * SwiGLU: silu(g) * u in the reference's float32 order (nn.py:41-54):
//    p = 0 <= g; e = exp(p ? -g : g); sigmoid = (p ? 1 : e) / (e + 1);
//    (g * sigmoid) * u;
//  * RoPE of one half-split pair (nn.py:97-106): y[j] = x[j] * c + (-x[j + h]) * s,
//    y[j + h] = x[j + h] * c + x[j] * s.
#pragma once

#include "nc_common.h"
#include "nc_math.h"

namespace nc {

__device__ __forceinline__ float dequant(int32_t acc, float xs, float ws) {
    return __fmul_rn(__fmul_rn((float)acc, xs), ws);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    const bool p = 0.0f <= g;
    const float e = nc_expf(p ? -g : g);
    const float sig = div_rn(p ? 1.0f : e, __fadd_rn(e, 1.0f));
    return __fmul_rn(__fmul_rn(g, sig), u);
}

__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float &y0, float &y1) {
    y0 = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
    y1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
}

}  // namespace nc
