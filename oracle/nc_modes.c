/* The reference's two int8 matmul modes, restated in C. TEST INFRASTRUCTURE ONLY.
 *
 * Both orders are written into the reference's loop IR, so they are bit for
 * bit what its generated C computes (tests/golden G2, G3 hold those outputs):
 *
 * matmul_i8 (lower.py:294-356, float activations): 32 accumulators; element
 *   32*k0 + 8*c + l of each whole 32-block into acc[8c + l] by fmaf; leftover
 *   whole 8-groups into acc[0..7]; the combine h[l] = (acc[l] + acc[8+l]) +
 *   (acc[16+l] + acc[24+l]), u[j] = h[j] + h[j+4], sum = (u0 + u1) + (u2 + u3);
 *   then the elements past the last group, multiply then add, in order;
 *   y = sum * scales[n].
 *
 * matmul_i8_vnni (lower.py:359-397, int8 activations in blocks): group
 *   g = 128*k0 + 32*c, lane l: acc[8c + l] = fmaf(f32(Dp4), xs[g / block], acc),
 *   Dp4 = sum_j (w[g+4l+j] + 128) * x[g+4l+j] (loopir.py:137-150); leftover
 *   32-byte groups into acc[0..7]; the same combine; y = (sum - offset) * scales[n].
 */
#include <math.h>
#include <stdint.h>

#define EXPORT __attribute__((visibility("default")))

static float combine(const float *acc) {
    float h[8];
    for (int l = 0; l < 8; ++l) h[l] = (acc[l] + acc[8 + l]) + (acc[16 + l] + acc[24 + l]);
    float u[4];
    for (int j = 0; j < 4; ++j) u[j] = h[j] + h[j + 4];
    return (u[0] + u[1]) + (u[2] + u[3]);
}

EXPORT void nc_host_matmul_i8_f32(float *y, const float *x, const int8_t *q, const float *scales, int64_t m,
                                  int64_t n, int64_t k) {
    const int64_t wide = k / 32 * 32, groups = (k % 32) / 8, tail = wide + groups * 8;
    for (int64_t r = 0; r < m; ++r) {
        const float *xr = x + r * k;
        for (int64_t o = 0; o < n; ++o) {
            const int8_t *w = q + o * k;
            float acc[32] = {0};
            for (int64_t k0 = 0; k0 < k / 32; ++k0)
                for (int c = 0; c < 4; ++c)
                    for (int l = 0; l < 8; ++l) {
                        const int64_t at = 32 * k0 + 8 * c + l;
                        acc[8 * c + l] = fmaf((float)w[at], xr[at], acc[8 * c + l]);
                    }
            for (int64_t k1 = 0; k1 < groups; ++k1)
                for (int l = 0; l < 8; ++l) {
                    const int64_t at = wide + 8 * k1 + l;
                    acc[l] = fmaf((float)w[at], xr[at], acc[l]);
                }
            float sum = combine(acc);
            for (int64_t at = tail; at < k; ++at) sum = sum + (float)w[at] * xr[at];
            y[r * n + o] = sum * scales[o];
        }
    }
}

static int32_t dp4(const int8_t *w, const int8_t *x) {
    int32_t s = 0;
    for (int j = 0; j < 4; ++j) s += ((int32_t)w[j] + 128) * (int32_t)x[j];
    return s;
}

EXPORT void nc_host_matmul_i8_vnni(float *y, const int8_t *xq, const float *xs, const float *offset,
                                   const int8_t *q, const float *scales, int64_t m, int64_t n, int64_t k,
                                   int64_t block) {
    const int64_t stride = k / 128 * 128, groups = (k % 128) / 32, blocks = k / block;
    for (int64_t r = 0; r < m; ++r) {
        const int8_t *xr = xq + r * k;
        const float *sr = xs + r * blocks;
        for (int64_t o = 0; o < n; ++o) {
            const int8_t *w = q + o * k;
            float acc[32] = {0};
            for (int64_t k0 = 0; k0 < k / 128; ++k0)
                for (int c = 0; c < 4; ++c) {
                    const int64_t g = 128 * k0 + 32 * c;
                    for (int l = 0; l < 8; ++l)
                        acc[8 * c + l] = fmaf((float)dp4(w + g + 4 * l, xr + g + 4 * l), sr[g / block], acc[8 * c + l]);
                }
            for (int64_t k1 = 0; k1 < groups; ++k1) {
                const int64_t g = stride + 32 * k1;
                for (int l = 0; l < 8; ++l)
                    acc[l] = fmaf((float)dp4(w + g + 4 * l, xr + g + 4 * l), sr[g / block], acc[l]);
            }
            y[r * n + o] = (combine(acc) - offset[r]) * scales[o];
        }
    }
}
