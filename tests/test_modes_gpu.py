"""The reference's int8 modes on the GPU, bit for bit against the reference's generated C.

tests/golden G2 and G3 hold what the reference's own compiled kernels produce
for matmul_i8 and matmul_i8_vnni at its test widths (test_int8.py:146) and
1, 3, 7 tokens, from inputs regenerated here from the recorded seeds.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import reference as R
from tests.conftest import bits

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"
WIDTHS = [(896, 72), (4864, 24), (77, 40), (40, 16), (160, 40), (96, 24)]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def inputs(k, n, tokens):
    from tests.golden.inputs import matmul_inputs
    return matmul_inputs(k, n, tokens, seed=k + tokens)


@pytest.mark.parametrize("k,n", WIDTHS)
def test_matmul_i8_is_the_references_generated_c(gpu, golden, k, n):
    from nanocompile_amd import kernels
    print(f"matmul_i8 k={k} n={n}", flush=True)
    for tokens in (1, 3, 7):
        w, x = inputs(k, n, tokens)
        q, s = R.quantize_int8(w)
        got = kernels.matmul_i8(x, q, s).numpy()
        assert np.array_equal(bits(got), bits(golden[f"g2_{k}_{n}_{tokens}"])), tokens


@pytest.mark.parametrize("k,n", [(k, n) for k, n in WIDTHS if k % 32 == 0])
def test_matmul_i8_vnni_is_the_references_generated_c(gpu, golden, k, n):
    from nanocompile_amd import kernels
    print(f"matmul_i8_vnni k={k} n={n}", flush=True)
    for tokens in (1, 3, 7):
        w, x = inputs(k, n, tokens)
        q, s = R.quantize_int8(w)
        xq, xs, off = kernels.quantize_blocks(x, 32)
        exq, exs, eoff = R.quantize_blocks(x, 32)
        assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))
        assert np.array_equal(bits(off.numpy()), bits(eoff[:, 0]))
        got = kernels.matmul_i8_vnni(xq, xs, off, q, s, 32).numpy()
        assert np.array_equal(bits(got), bits(golden[f"g3_{k}_{n}_{tokens}"])), tokens


def test_block_quantizer_is_the_references(gpu, golden):
    from nanocompile_amd import kernels
    _, x = inputs(96, 1, 5)
    xq, xs, off = kernels.quantize_blocks(x, 32)
    assert np.array_equal(xq.numpy(), golden["g3_quant_xq"])
    assert np.array_equal(bits(xs.numpy()), bits(golden["g3_quant_xs"]))
    assert np.array_equal(bits(off.numpy()), bits(golden["g3_quant_offset"][:, 0]))


@pytest.mark.parametrize("m,k,block", [(1, 896, 32), (2, 4864, 32), (3, 5120, 32), (2, 6400, 32), (1, 16384, 32),
                                       (2, 4864, 64)])
def test_block_quantizer_at_every_width_is_the_oracle(gpu, m, k, block):
    """Rows whose blocks a workgroup holds at once (up to 5120 values) and longer ones whose
    later blocks it loads one after another, and blocks of 64: bit for bit with the oracle."""
    from nanocompile_amd import kernels
    print(f"quantize_blocks m={m} k={k} block={block}", flush=True)
    rng = np.random.default_rng(k + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 30
    x[:, :block] = 0.0                                   # an all-zero block: scale 1
    xq, xs, off = kernels.quantize_blocks(x, block)
    eq, es, eoff = R.quantize_blocks(x, block)
    assert np.array_equal(xq.numpy(), eq)
    assert np.array_equal(bits(xs.numpy()), bits(es))
    assert np.array_equal(bits(off.numpy()), bits(eoff[:, 0]))


def test_block_quantizer_on_special_values(gpu):
    """Blocks of 32 built to separate a block's maximum taken in another grouping or order:
    +0 against -0, tied magnitudes of both signs, an infinity, subnormals, and (in the first
    row) NaNs of two payloads and signs. The row without NaN is the oracle's bit for bit; in
    the NaN row every other block is too, and the NaN block's scale is NaN and its values 127
    (the grouping that keeps the NaN's bits is held by test_codegen.py's ordered-tree test)."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(31)
    x = rng.standard_normal((2, 32 * 6)).astype(np.float32)
    blocks = x.reshape(2, 6, 32)
    blocks[:, 1] = np.where(rng.random(32) < 0.5, np.float32(0.0), np.float32(-0.0))
    blocks[:, 2, ::5] = 3.0
    blocks[:, 2, 2::7] = -3.0
    blocks[:, 3, 9] = np.inf
    blocks[:, 4] = (rng.standard_normal(32) * 1e-39).astype(np.float32)        # subnormals
    blocks[0, 5, 4] = np.uint32(0x7FC00001).view(np.float32)
    blocks[0, 5, 20] = np.uint32(0xFFC00002).view(np.float32)
    xq, xs, off = (a.numpy() for a in kernels.quantize_blocks(x, 32))
    exq, exs, eoff = R.quantize_blocks(x, 32)
    assert np.array_equal(xq[1], exq[1]) and np.array_equal(bits(xs[1]), bits(exs[1]))
    assert np.array_equal(bits(off[1:]), bits(eoff[1:, 0]))
    assert np.array_equal(xq[0, :160], exq[0, :160]) and np.array_equal(bits(xs[0, :5]), bits(exs[0, :5]))
    assert np.isnan(xs[0, 5]) and np.all(xq[0, 160:] == 127) and np.isnan(off[0])


@pytest.mark.parametrize("k,n,m", [(896, 896, 1), (4864, 896, 2), (896, 4864, 5), (128, 40, 3), (64, 8, 2),
                                   (896, 100, 2), (4864, 13, 1)])
def test_modes_at_model_shapes_match_the_host_restatement(gpu, host, k, n, m):
    """Model widths the golden set does not cover, with bias and residual epilogues."""
    from nanocompile_amd import kernels
    rng = np.random.default_rng(k + n + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    b, r = rng.standard_normal(n).astype(np.float32), rng.standard_normal((m, n)).astype(np.float32)
    q, s = R.quantize_int8(w)
    y = kernels.matmul_i8(x, q, s, bias=b, residual=r).numpy()
    expected = (r + (host.matmul_i8_f32(x, q, s) + b).astype(np.float32)).astype(np.float32)
    assert np.array_equal(bits(y), bits(expected))
    xq, xs, off = R.quantize_blocks(x, 32)
    y = kernels.matmul_i8_vnni(xq, xs, off[:, 0], q, s, 32).numpy()
    assert np.array_equal(bits(y), bits(host.matmul_i8_vnni(xq, xs, off, q, s)))


def test_vnni_rejects_blocks_that_are_not_powers_of_two(gpu):
    from nanocompile_amd import kernels
    xq = np.zeros((1, 96), np.int8)
    with pytest.raises(kernels.ShapeError, match="power of two"):
        kernels.matmul_i8_vnni(xq, np.ones((1, 2), np.float32), np.zeros(1, np.float32),
                               np.zeros((4, 96), np.int8), np.ones(4, np.float32), block=48)


@pytest.mark.parametrize("m,k", [(1, 896), (3, 4864), (128, 896), (2, 128), (2, 1030), (1, 16384)])
def test_rms_norm_index_order_is_the_references_order(gpu, m, k):
    """The reference modes' rms_norm: its row sum in index order (golden G4 pins the oracle)."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"rms_norm_index_order m={m} k={k}", flush=True)
    rng = np.random.default_rng(m * k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    dx, dg, out = DeviceArray.from_host(x), DeviceArray.from_host(g), DeviceArray((m, k), np.float32)
    hip.call("nc_rms_norm_index_order", [out, dx, dg], [m, k, float_bits(1e-6)])
    hip.sync()
    assert np.array_equal(bits(out.numpy()), bits(R.rms_norm_reference(x, g, 1e-6)))


@pytest.mark.parametrize("m,past,heads,kv,d", [(1, 0, 14, 2, 64), (1, 383, 14, 2, 64), (7, 0, 14, 2, 64),
                                               (5, 3, 4, 2, 32), (1, 12, 4, 2, 32), (128, 0, 14, 2, 64),
                                               (3, 300, 14, 2, 64), (2, 200, 4, 2, 128), (2, 700, 4, 2, 32),
                                               (2, 40, 4, 2, 48)])
def test_attention_index_order_is_the_oracle(gpu, host, m, past, heads, kv, d):
    """The reference modes' attention (every sum in the reference's order) bit for bit against the
    oracle, with the position given on the host and read from the device."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"attention_index_order m={m} past={past} heads={heads}/{kv} d={d}", flush=True)
    rng = np.random.default_rng(m + past + heads + d)
    capacity = past + m + 3
    qkv = rng.standard_normal((m, (heads + 2 * kv) * d)).astype(np.float32)
    kc = rng.standard_normal((kv, capacity, d)).astype(np.float32)
    vc = rng.standard_normal((kv, capacity, d)).astype(np.float32)
    scale = float(np.float32(d ** -0.5))
    q = qkv[:, :heads * d].reshape(m, heads, d)
    want = R.attention_index_order(q, kc, vc, past, scale, lambda v: host.math("nc_exp", v)).reshape(m, heads * d)
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    pos = DeviceArray.from_host(np.array([past], np.int64))
    for where in (None, pos):
        ctx = DeviceArray((m, heads * d), np.float32)
        hip.call("nc_attention_index_order", [ctx, dq, dk, dv, where],
                 [m, heads, kv, d, 0 if where is not None else past, capacity, float_bits(scale)])
        hip.sync()
        assert np.array_equal(bits(ctx.numpy()), bits(want)), where is not None


@pytest.mark.parametrize("m,n,k", [(1, 1152, 896), (3, 4864, 896), (2, 896, 4864), (5, 100, 896)])
def test_matmul_i8_normed_is_the_norm_then_the_matmul(gpu, m, n, k):
    """The int8 mode's fused rms_norm + matmul_i8 against the two calls, bit for bit."""
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"matmul_i8_normed m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    q, s = R.quantize_int8(w)
    dx, dg = DeviceArray.from_host(x), DeviceArray.from_host(g)
    normed = DeviceArray((m, k), np.float32)
    hip.call("nc_rms_norm_index_order", [normed, dx, dg], [m, k, float_bits(1e-6)])
    want = kernels.matmul_i8(normed, q, s, bias=b).numpy()
    dq, ds, db = DeviceArray.from_host(q), DeviceArray.from_host(s), DeviceArray.from_host(b)
    packed = DeviceArray.from_host(kernels.pack_chains(q))
    y = DeviceArray((m, n), np.float32)
    hip.call("nc_matmul_i8_normed", [y, dx, packed, dq, ds, db, None, dg], [m, n, k, float_bits(1e-6)])
    hip.sync()
    assert np.array_equal(bits(y.numpy()), bits(want))


@pytest.mark.parametrize("m,k", [(1, 896), (3, 896), (2, 1024), (4, 64)])
def test_quantize_blocks_normed_is_the_norm_then_the_quantizer(gpu, m, k):
    """int8-vnni's fused rms_norm + block quantizer against the two calls, bit for bit."""
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"quantize_blocks_normed m={m} k={k}", flush=True)
    rng = np.random.default_rng(m * 7 + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    dx, dg = DeviceArray.from_host(x), DeviceArray.from_host(g)
    normed = DeviceArray((m, k), np.float32)
    hip.call("nc_rms_norm_index_order", [normed, dx, dg], [m, k, float_bits(1e-6)])
    eq, es, eoff = (a.numpy() for a in kernels.quantize_blocks(normed, 32))
    xq, xs, off = DeviceArray((m, k), np.int8), DeviceArray((m, k // 32), np.float32), DeviceArray((m,), np.float32)
    hip.call("nc_quantize_blocks_normed", [xq, xs, off, dx, dg], [m, k, float_bits(1e-6)])
    hip.sync()
    assert np.array_equal(xq.numpy(), eq)
    assert np.array_equal(bits(xs.numpy()), bits(es)) and np.array_equal(bits(off.numpy()), bits(eoff))


@pytest.mark.parametrize("m,n,k", [(1, 4864, 896), (3, 100, 896), (2, 896, 4864)])
def test_up_projection_with_swiglu_is_the_projection_then_silu_mul(gpu, m, n, k):
    """The reference modes' up projection with silu(gate) * up in its epilogue, int8 and
    int8-vnni, against the projection then nc_silu_mul, bit for bit."""
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.hip import DeviceArray
    print(f"matmul_i8(_vnni)_silu m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    gate = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    gate[0, :4] = [0.0, -0.0, 80.0, -80.0]
    q, s = R.quantize_int8(w)
    dx, dq, ds, dgate = (DeviceArray.from_host(a) for a in (x, q, s, gate))
    for mode in ("int8", "int8-vnni"):
        if mode == "int8":
            up = kernels.matmul_i8(x, q, s)
            packed = DeviceArray.from_host(kernels.pack_chains(q))
            h = DeviceArray((m, n), np.float32)
            hip.call("nc_matmul_i8_silu", [h, dx, packed, dq, ds, dgate], [m, n, k])
        else:
            xq, xs, off = kernels.quantize_blocks(x, 32)
            up = kernels.matmul_i8_vnni(xq, xs, off, q, s, 32)
            packed = DeviceArray.from_host(kernels.pack_chains_vnni(q))
            h = DeviceArray((m, n), np.float32)
            hip.call("nc_matmul_i8_vnni_silu", [h, xq, xs, off, packed, dq, ds, dgate], [m, n, k, 32])
        want = DeviceArray((m, n), np.float32)
        hip.call("nc_silu_mul", [want, dgate, up], [m * n])
        hip.sync()
        assert np.array_equal(bits(h.numpy()), bits(want.numpy())), mode
