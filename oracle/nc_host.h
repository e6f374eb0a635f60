/* Shared declarations of the host C oracle/baseline. TEST INFRASTRUCTURE ONLY. */
#ifndef NC_HOST_H
#define NC_HOST_H
#include <stdint.h>

typedef void (*task_fn)(void *ctx, int64_t i);

/* Runs fn(ctx, i) for i in [0, n) on the pool; returns when all are done. */
void nc_pool_run(task_fn fn, void *ctx, int64_t n);

void nc_host_matmul_i8_token(float *y, const int8_t *xq, const float *xs, const int8_t *q, const float *ws,
                             const float *bias, const float *residual, int64_t m, int64_t n, int64_t k);
#endif
