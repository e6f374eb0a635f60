"""The prefill projection on the i8 MFMA, bit for bit against the oracle.

Every MFMA tile is checked on the block's four projection shapes at the
prefill length 512 (config 4), on ragged shapes (rows past a tile edge, K not
a whole number of k stages, K = 16), on the largest accumulators, and with
each epilogue (dequantize, bias, residual, SwiGLU). The int32 accumulators
are exact in any order, so they must equal the closed form; the f32 epilogue
is the frozen one, so outputs must equal the host restatement's bits.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import reference as R
from tests.conftest import bits

pytestmark = pytest.mark.gpu

MODEL_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864)]   # (N, K): q/o, k/v, gate/up, down
TILES = list(range(16, 25))


def random_int8(rng, shape):
    return rng.integers(-127, 128, shape).astype(np.int8)


@pytest.mark.parametrize("schedule", TILES)
@pytest.mark.parametrize("n,k", MODEL_SHAPES)
def test_prefill_accumulators_are_exact(gpu, host, n, k, schedule):
    from nanocompile_amd import kernels
    print(f"gemm acc m=512 n={n} k={k} schedule={schedule}", flush=True)
    rng = np.random.default_rng(n + k + schedule)
    xq, q = random_int8(rng, (512, k)), random_int8(rng, (n, k))
    got = kernels.matmul_i8_token_acc(xq, q, schedule=schedule).numpy()
    assert np.array_equal(got, host.matmul_i8_token_acc(xq, q))


@pytest.mark.parametrize("schedule", TILES)
@pytest.mark.parametrize("m,n,k", [(16, 24, 16), (17, 203, 48), (100, 77, 896), (130, 130, 1040), (33, 1, 208)])
def test_ragged_shapes_are_exact(gpu, m, n, k, schedule):
    from nanocompile_amd import kernels
    print(f"gemm ragged m={m} n={n} k={k} schedule={schedule}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 3 + k + schedule)
    xq, q = random_int8(rng, (m, k)), random_int8(rng, (n, k))
    got = kernels.matmul_i8_token_acc(xq, q, schedule=schedule).numpy()
    assert np.array_equal(got, R.matmul_i8_token_acc(xq, q))


@pytest.mark.parametrize("schedule", TILES)
def test_largest_accumulators(gpu, schedule):
    from nanocompile_amd import kernels
    k = 4864
    xq = np.full((40, k), 127, np.int8)
    xq[1::2] = -127
    q = np.full((24, k), -127, np.int8)
    q[::3] = 127
    got = kernels.matmul_i8_token_acc(xq, q, schedule=schedule).numpy()
    assert np.array_equal(got, R.matmul_i8_token_acc(xq, q))
    assert np.abs(got).max() == 127 * 127 * k


@pytest.mark.parametrize("schedule", [0] + TILES)
@pytest.mark.parametrize("n,k", MODEL_SHAPES)
def test_prefill_projection_is_bitwise(gpu, host, n, k, schedule):
    """From f32 activations: quantize per token, project, bias and residual epilogues."""
    from nanocompile_amd import kernels
    print(f"gemm projection m=512 n={n} k={k} schedule={schedule}", flush=True)
    rng = np.random.default_rng(3 * n + k + schedule)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((512, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    b = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal((512, n)).astype(np.float32)
    q, s = R.quantize_int8(w)
    xq, xs = R.quantize_token(x)
    dxq, dxs = kernels.quantize_token(x)
    assert np.array_equal(dxq.numpy(), xq) and np.array_equal(bits(dxs.numpy()), bits(xs))
    y = kernels.matmul_i8_token(dxq, dxs, q, s, schedule=schedule).numpy()
    assert np.array_equal(bits(y), bits(host.matmul_i8_token(xq, xs, q, s)))
    y = kernels.matmul_i8_token(dxq, dxs, q, s, bias=b, residual=r, schedule=schedule).numpy()
    assert np.array_equal(bits(y), bits(R.matmul_i8_token(xq, xs, q, s, bias=b, residual=r)))


@pytest.mark.parametrize("schedule", [0] + TILES)
@pytest.mark.parametrize("m,n,k", [(512, 4864, 896), (64, 256, 128), (19, 40, 96)])
def test_prefill_swiglu_is_bitwise(gpu, host, m, n, k, schedule):
    from nanocompile_amd import kernels
    print(f"gemm swiglu m={m} n={n} k={k} schedule={schedule}", flush=True)
    rng = np.random.default_rng(m + n + k + schedule)
    xq = random_int8(rng, (m, k))
    xs = (rng.random(m) * 0.05 + 1e-3).astype(np.float32)
    qg, qu = random_int8(rng, (n, k)), random_int8(rng, (n, k))
    sg = (rng.random(n) * 1e-3).astype(np.float32)
    su = (rng.random(n) * 1e-3).astype(np.float32)
    h = kernels.matmul_i8_token_swiglu(xq, xs, qg, sg, qu, su, schedule=schedule).numpy()
    assert np.array_equal(bits(h), bits(host.matmul_i8_token_swiglu(xq, xs, qg, sg, qu, su)))


def test_gemv_and_gemm_agree_at_the_crossover(gpu):
    """The default routes 15 tokens to the GEMV and 16 to the MFMA GEMM: same bits either way."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(5)
    q, s = random_int8(rng, (896, 896)), (rng.random(896) * 1e-3).astype(np.float32)
    xq, xs = random_int8(rng, (16, 896)), (rng.random(16) * 0.1).astype(np.float32)
    gemm = kernels.matmul_i8_token(xq, xs, q, s).numpy()
    gemv = kernels.matmul_i8_token(xq, xs, q, s, schedule=7).numpy()
    assert np.array_equal(bits(gemm), bits(gemv))
    assert np.array_equal(bits(kernels.matmul_i8_token(xq[:15], xs[:15], q, s).numpy()), bits(gemv[:15]))


def test_unknown_schedules_are_refused(gpu):
    from nanocompile_amd import hip, kernels
    xq, q = np.zeros((32, 100), np.int8), np.zeros((8, 100), np.int8)
    for schedule in (8, 15, 25, -1):
        with pytest.raises(hip.KernelError, match="schedule"):
            kernels.matmul_i8_token_acc(np.zeros((32, 96), np.int8), np.zeros((8, 96), np.int8), schedule=schedule)
    with pytest.raises(hip.KernelError, match="multiple of 16"):
        kernels.matmul_i8_token_acc(xq, q, schedule=16)
