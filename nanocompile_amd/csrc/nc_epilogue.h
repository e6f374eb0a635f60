// The projection epilogues, shared by every int8 kernel so that the GEMV, the
// fused decode kernels and the MFMA GEMM produce the same bits.
//
//  * dequantization: y = (f32(acc) * xs[m]) * scales[n], two roundings in that
//    order; f32(acc) rounds to nearest even above 2^24;
//  * SwiGLU: silu(g) * u in the reference's float32 order (nn.py:41-54):
//    p = 0 <= g; e = exp(p ? -g : g); sigmoid = (p ? 1 : e) / (e + 1);
//    (g * sigmoid) * u.
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

}  // namespace nc
