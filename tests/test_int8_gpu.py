"""The int8 hot path on the GPU, bit for bit against the oracle.

Integers (accumulators, quantized values) must be identical; float outputs
whose operation order is the oracle's must be identical too. Shapes cover the
model's projections, the reference's odd test widths (test_int8.py:146:
77 and 40 have no whole 16-byte chunks, 160 and 96 leave partial groups),
empty inputs, a single row, and the largest accumulators.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import reference as R
from tests.conftest import bits

pytestmark = pytest.mark.gpu

MODEL_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864)]   # (N, K) of q/o, k/v, gate/up, down
ODD_SHAPES = [(72, 896), (24, 4864), (40, 77), (16, 40), (40, 160), (24, 96), (1, 16), (33, 1024)]
SCHEDULES = range(7)


def random_int8(rng, shape):
    return rng.integers(-127, 128, shape).astype(np.int8)


@pytest.mark.parametrize("n,k", MODEL_SHAPES + ODD_SHAPES)
@pytest.mark.parametrize("m", [1, 2, 3, 7, 9, 17])
def test_accumulators_are_exact(gpu, m, n, k):
    from nanocompile_amd import kernels
    print(f"acc m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 100003 + n * 31 + k)
    xq, q = random_int8(rng, (m, k)), random_int8(rng, (n, k))
    got = kernels.matmul_i8_token_acc(xq, q).numpy()
    assert np.array_equal(got, R.matmul_i8_token_acc(xq, q))


@pytest.mark.parametrize("k", [896, 4864, 1024])
@pytest.mark.parametrize("schedule", SCHEDULES)
def test_every_schedule_is_exact(gpu, k, schedule):
    from nanocompile_amd import kernels
    print(f"schedule {schedule} k={k}", flush=True)
    rng = np.random.default_rng(schedule + k)
    for m in (1, 4, 8):
        xq, q = random_int8(rng, (m, k)), random_int8(rng, (203, k))   # 203 rows: a ragged last block
        assert np.array_equal(kernels.matmul_i8_token_acc(xq, q, schedule=schedule).numpy(),
                              R.matmul_i8_token_acc(xq, q))


def test_largest_accumulators(gpu):
    from nanocompile_amd import kernels
    k = 4864
    xq = np.full((2, k), 127, np.int8)
    xq[1] = -127
    q = np.full((3, k), 127, np.int8)
    q[1] = -127
    acc = kernels.matmul_i8_token_acc(xq, q).numpy()
    assert acc[0, 0] == 127 * 127 * k and acc[0, 1] == -127 * 127 * k and acc[1, 1] == 127 * 127 * k


def test_empty_and_single(gpu):
    from nanocompile_amd import kernels
    rng = np.random.default_rng(0)
    q = random_int8(rng, (5, 896))
    assert kernels.matmul_i8_token_acc(np.zeros((0, 896), np.int8), q).numpy().shape == (0, 5)
    xq = random_int8(rng, (1, 896))
    assert np.array_equal(kernels.matmul_i8_token_acc(xq, q[:1]).numpy(), R.matmul_i8_token_acc(xq, q[:1]))


@pytest.mark.parametrize("n,k", MODEL_SHAPES + [(40, 77), (24, 96)])
@pytest.mark.parametrize("m", [1, 3, 8])
def test_projection_epilogue_is_bitwise(gpu, m, n, k):
    """The full projection from f32 activations, every stage against the oracle."""
    from nanocompile_amd import kernels
    print(f"projection m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(k * 7 + n + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    bias = rng.standard_normal(n).astype(np.float32)
    residual = rng.standard_normal((m, n)).astype(np.float32)

    q, scales = kernels.quantize_int8(w)
    eq, es = R.quantize_int8(w)
    assert np.array_equal(q.numpy(), eq) and np.array_equal(bits(scales.numpy()), bits(es))

    xq, xs = kernels.quantize_token(x)
    exq, exs = R.quantize_token(x)
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))

    for b, r in ((None, None), (bias, None), (None, residual), (bias, residual)):
        y = kernels.matmul_i8_token(xq, xs, q, scales, bias=b, residual=r).numpy()
        assert np.array_equal(bits(y), bits(R.matmul_i8_token(exq, exs, eq, es, b, r)))


def test_weight_quantizer_special_rows(gpu):
    """The reference's special rows (test_int8.py:69-78) and the float32 floor quirk."""
    from nanocompile_amd import kernels
    from tests.test_oracle import special_rows
    w = special_rows()
    q, s = kernels.quantize_int8(w)
    eq, es = R.quantize_int8(w)
    assert np.array_equal(q.numpy(), eq) and np.array_equal(bits(s.numpy()), bits(es))
    quirk = np.array([[0.49999997, 127.0, -0.49999997, 0.0]], dtype=np.float32)
    assert list(kernels.quantize_int8(quirk)[0].numpy()[0]) == [1, 127, -1, 0]


@pytest.mark.parametrize("k", [67, 4864])
def test_token_quantizer_both_load_widths(gpu, k):
    """Rows of a multiple of 4 floats take 16-byte loads, others 4-byte ones: both are the oracle."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(k)
    x = rng.standard_normal((5, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    x[4] = 0.0
    xq, xs = kernels.quantize_token(x)
    exq, exs = R.quantize_token(x)
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))


def test_token_quantizer_edges(gpu):
    from nanocompile_amd import kernels
    x = np.zeros((4, 64), np.float32)
    x[1, :3] = [63.5, -127.0, 0.5]           # scale 1: halves away from zero
    x[2, 0] = np.float32(1e-30)              # tiny but positive magnitude
    x[3] = -3.0
    xq, xs = kernels.quantize_token(x)
    exq, exs = R.quantize_token(x)
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))
    assert xs.numpy()[0] == 1.0 and list(xq.numpy()[1, :3]) == [64, -127, 1]


def same_floats(a, b) -> bool:
    """Bitwise equal, except that any NaN matches any NaN (payloads are not specified)."""
    a, b = np.asarray(a), np.asarray(b)
    nan = np.isnan(a)
    return bool(np.array_equal(nan, np.isnan(b)) and np.array_equal(bits(a[~nan]), bits(b[~nan])))


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
@pytest.mark.parametrize("k", [67, 896, 4864])
def test_quantizers_propagate_nan(gpu, k):
    """A NaN or infinity in a row: the scale is NaN (or inf) as the reference's max gives it,
    and the int8 values are the reference's selects' (127 for NaN), in every quantizer."""
    from nanocompile_amd import kernels
    print(f"nan rows k={k}", flush=True)
    rng = np.random.default_rng(k + 11)
    x = rng.standard_normal((4, k)).astype(np.float32)
    x[0, k // 3] = np.nan
    x[1, k - 1] = np.inf
    x[2, 0] = -np.inf
    xq, xs = kernels.quantize_token(x)
    exq, exs = R.quantize_token(x)
    assert np.isnan(xs.numpy()[0]) and same_floats(xs.numpy(), exs)
    assert np.array_equal(xq.numpy(), exq)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    normed, nq, ns = kernels.rms_norm_quant(x, g, 1e-6)
    en, enq, ens = R.rms_norm_quant_gpu_order(x, g, 1e-6)
    assert same_floats(normed.numpy(), en) and same_floats(ns.numpy(), ens)
    assert np.isnan(ns.numpy()[:3]).all() and np.array_equal(nq.numpy(), enq)
    q, s = kernels.quantize_int8(x)
    eq, es = R.quantize_int8(x)
    assert np.isnan(s.numpy()[0]) and same_floats(s.numpy(), es) and np.array_equal(q.numpy(), eq)
    if k % 32 == 0:
        bq, bs, off = kernels.quantize_blocks(x, 32)
        ebq, ebs, eoff = R.quantize_blocks(x, 32)
        assert np.array_equal(bq.numpy(), ebq) and same_floats(bs.numpy(), ebs)
        assert same_floats(off.numpy(), eoff[:, 0])


@pytest.mark.parametrize("m", [1, 64, 512])
@pytest.mark.parametrize("k", [896, 4864, 64, 100])
def test_rms_norm_quant(gpu, m, k):
    """Bitwise against the GPU-order restatement; to rounding against the reference's order."""
    from nanocompile_amd import kernels
    print(f"rms_norm_quant m={m} k={k}", flush=True)
    rng = np.random.default_rng(m + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    normed, xq, xs = kernels.rms_norm_quant(x, g, 1e-6)
    en, exq, exs = R.rms_norm_quant_gpu_order(x, g, 1e-6)
    assert np.array_equal(bits(normed.numpy()), bits(en))
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))
    # The tree order lands within a few ulps of the exact value; the reference's
    # sequential float32 sum itself drifts up to ~2.2e-6 relative at K = 4864.
    exact = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    np.testing.assert_allclose(normed.numpy(), exact, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(normed.numpy(), R.rms_norm_reference(x, g, 1e-6), rtol=4e-6, atol=1e-6)


def test_shape_errors_are_raised_before_launch(gpu):
    from nanocompile_amd import kernels
    rng = np.random.default_rng(1)
    xq, xs = random_int8(rng, (2, 64)), np.ones(2, np.float32)
    q, s = random_int8(rng, (8, 64)), np.ones(8, np.float32)
    with pytest.raises(kernels.ShapeError, match="one f32 scale per row"):
        kernels.matmul_i8_token(xq, xs, q, np.ones(9, np.float32))
    with pytest.raises(kernels.ShapeError, match="must be i8"):
        kernels.matmul_i8_token(xq, xs, q.astype(np.float32), s)
    with pytest.raises(kernels.ShapeError, match="width"):
        kernels.matmul_i8_token(random_int8(rng, (2, 32)), xs, q, s)


def test_device_division_sqrt_and_round_are_correctly_rounded(gpu):
    """IEEE a / b and sqrt, and roundf, on the GPU: the epilogues and rms_norm depend on them."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    rng = np.random.default_rng(11)
    n = 1 << 20
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    from tests.test_oracle import ROUND_VALUES
    a[:16] = ROUND_VALUES                  # halves, 0.49999997, signed zeros, 2^23 + 1
    outs = [DeviceArray((n,), np.float32) for _ in range(3)]
    hip.call("nc_probe_fp32_ops", outs + [DeviceArray.from_host(a), DeviceArray.from_host(b)], [n])
    quotient, root, rounded = (o.numpy() for o in outs)
    assert np.array_equal(bits(quotient), bits((a / b).astype(np.float32)))
    assert np.array_equal(bits(root), bits(np.sqrt(np.abs(a)).astype(np.float32)))
    assert np.array_equal(bits(rounded), bits(R.round_half_away(a)))


def test_token_quantizer_at_half_integers(gpu):
    """Values placed at, and a few ulps to 2^-12 around, every k + 1/2 of their row's scale:
    where round(x / scale) depends on the division's last bit, the quantizer must still give
    the correctly rounded quotient's rounding, as the oracle does."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(17)
    rows = []
    for _ in range(64):
        mag = np.float32(rng.uniform(0.01, 100.0))
        scale = np.float32(mag / np.float32(127.0))
        k = rng.integers(-127, 127, 895).astype(np.float32) + np.float32(0.5)
        base = (k * scale).astype(np.float32)
        nudges = rng.choice([0, 1, -1, 2, -2], size=895)
        x = base.copy()
        toward = np.where(nudges > 0, np.float32(np.inf), np.float32(-np.inf))
        for step in (1, 2):
            x = np.where(np.abs(nudges) >= step, np.nextafter(x, toward).astype(np.float32), x)
        spread = rng.choice([0.0, 2.0 ** -20, -(2.0 ** -20), 2.0 ** -14, -(2.0 ** -14), 2.0 ** -12], size=895)
        x = np.where(spread != 0, ((k + spread) * scale).astype(np.float32), x)
        x = np.clip(x, -mag, mag).astype(np.float32)
        rows.append(np.concatenate([[mag], x]).astype(np.float32))
    x = np.stack(rows)
    xq, xs = kernels.quantize_token(x)
    eq, es = R.quantize_token(x)
    assert np.array_equal(xq.numpy(), eq) and np.array_equal(bits(xs.numpy()), bits(es))


@pytest.mark.parametrize("k", [1, 255, 1024, 4864, 5121, 8192, 9000])
def test_token_quantizer_every_row_width(gpu, k):
    """Each register-resident width class (up to 4, 8, 20, 32 values a thread) and the loop past it."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(k)
    x = rng.standard_normal((5, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    x[2] = 0.0
    xq, xs = kernels.quantize_token(x)
    exq, exs = R.quantize_token(x)
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))
