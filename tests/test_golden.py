"""The oracle against the reference's own outputs (tests/golden/, made by make_golden.py).

These fixtures were produced by running the reference's code (its quantizer,
its generated C kernels, its interpreter) on the inputs recorded here or
regenerated from the recorded seeds; the hashes catch a changed generator.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import reference as R
from oracle.host_model import inverse_frequencies
from tests.conftest import bits

HERE = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def golden():
    return np.load(HERE / "golden.npz", allow_pickle=False)


@pytest.fixture(scope="module")
def meta():
    return json.loads((HERE / "golden.json").read_text())


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


def test_g1_quantize_int8_is_the_references(golden, meta):
    from tests.test_oracle import special_rows
    values, scales = R.quantize_int8(special_rows())
    assert np.array_equal(values, golden["g1_special_values"])
    assert np.array_equal(bits(scales), bits(golden["g1_special_scales"]))
    w = (np.random.default_rng(1).standard_normal((4864, 896)) * 0.02).astype(np.float32)
    assert sha(w) == meta["g1_big"]["w_sha"], "the seeded generator changed"
    values, scales = R.quantize_int8(w)
    assert sha(values) == meta["g1_big"]["values_sha"] and sha(scales) == meta["g1_big"]["scales_sha"]


def test_g3_block_quantizer_is_the_references(golden, meta):
    from tests.golden.inputs import matmul_inputs
    _, x = matmul_inputs(96, 1, 5, seed=101)
    assert sha(x) == meta["g3_quant"]["x_sha"]
    xq, xs, offset = R.quantize_blocks(x, 32)
    assert np.array_equal(xq, golden["g3_quant_xq"])
    assert np.array_equal(bits(xs), bits(golden["g3_quant_xs"]))
    assert np.array_equal(bits(offset), bits(golden["g3_quant_offset"]))


def test_g4_rms_norm_reference_order_is_bitwise(golden):
    y = R.rms_norm_reference(golden["g4_rms_x"], golden["g4_rms_w"], 1e-6)
    assert np.array_equal(bits(y), bits(golden["g4_rms_y"]))


def test_g4_rms_norm_gpu_order_is_close(golden, host):
    normed, _, _ = host.rms_norm_quant(golden["g4_rms_x"], golden["g4_rms_w"], 1e-6)
    np.testing.assert_allclose(normed, golden["g4_rms_y"], rtol=2e-6, atol=1e-6)
    assert np.array_equal(bits(normed), bits(R.rms_norm_gpu_order(golden["g4_rms_x"], golden["g4_rms_w"], 1e-6)))


def test_g4_inverse_frequencies_are_bitwise(golden):
    assert np.array_equal(bits(inverse_frequencies(64, 1e6)), bits(golden["g4_inv_freq_64_1e6"]))
    assert np.array_equal(bits(inverse_frequencies(32, 1e6)), bits(golden["g4_inv_freq_32_1e6"]))


@pytest.mark.parametrize("seq,past", [(1, 12), (5, 3)])
def test_g4_softmax_with_causal_mask(golden, host, seq, past):
    """The reference's C (libm expf, sequential sums) to its own tolerance (test_codegen.py:28-29)."""
    key = f"g4_softmax_{seq}_{past}"
    y = host.softmax_causal(golden[key + "_s"], past)
    np.testing.assert_allclose(y, golden[key + "_y"], rtol=2e-6, atol=1e-6)
    assert np.array_equal(y == 0, golden[key + "_y"] == 0)          # the mask, exactly


def test_g4_silu_mul(golden, host):
    y = host.silu_mul(golden["g4_silu_g"], golden["g4_silu_u"])
    np.testing.assert_allclose(y, golden["g4_silu_y"], rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("seq,past", [(1, 511), (7, 0), (2, 100000)])
def test_g4_rope(golden, host, seq, past):
    key = f"g4_rope_{seq}_{past}"
    y = host.rope(golden[key + "_x"], inverse_frequencies(64, 1e6), past)
    np.testing.assert_allclose(y, golden[key + "_y"], rtol=2e-6, atol=1e-6)


def test_nc_math_against_the_c_library(host):
    """nc_expf/nc_sinf/nc_cosf (shared by the GPU kernels and the host oracle)
    within one ulp of the C library the reference calls, and correctly rounded
    against float64 on these samples."""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-104, 89, 200_000), rng.standard_normal(100_000) * 3]).astype(np.float32)
    t = np.concatenate([rng.uniform(-2e5, 2e5, 200_000), rng.uniform(-10, 10, 100_000)]).astype(np.float32)

    def ulps(a, b):
        ai, bi = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
        ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
        bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
        return np.abs(ai - bi)

    for ours, libm, xs, f64 in (("nc_exp", "exp", x, np.exp), ("nc_sin", "sin", t, np.sin), ("nc_cos", "cos", t, np.cos)):
        a, b = host.math(ours, xs), host.math(libm, xs)
        assert ulps(a, b).max() <= 1, ours
        with np.errstate(over="ignore"):
            exact = f64(xs.astype(np.float64)).astype(np.float32)
        assert (a != exact).mean() < 1e-5, ours
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 89.0, -104.5, 1e-30], np.float32)
    e = host.math("nc_exp", special)
    assert e[0] == 1 and e[1] == 1 and e[2] == np.inf and e[3] == 0 and np.isnan(e[4]) and e[6] == 0
    s = host.math("nc_sin", special)
    assert s[0] == 0 and np.signbit(s[1]) and np.isnan(s[2]) and np.isnan(s[3]) and s[7] == np.float32(1e-30)



def test_nc_math_exp_constants():
    """nc_expf's table holds the double nearest 2^(j / 64) for every j, its
    reduction constants split ln 2 / 64 exactly enough (the high part short
    enough (29 bits) that k * l_hi is exact for every |k| <= 9601) and 64 / ln 2 is the
    nearest double: checked against 50-digit decimal arithmetic."""
    import math
    import re
    from decimal import Decimal, getcontext

    getcontext().prec = 50
    text = (Path(__file__).resolve().parents[1] / "nanocompile_amd" / "csrc" / "nc_math.h").read_text()
    body = text[text.index("nc_exp2_64ths[64] = {"):]
    table = [float.fromhex(h) for h in re.findall(r"0x[0-9a-f.]+p[-+]\d+", body[:body.index("};")])]
    ln2 = Decimal(2).ln()
    assert table == [float((ln2 * j / 64).exp()) for j in range(64)]

    def constant(name):
        return float.fromhex(re.search(rf"const double {name} = (-?0x[0-9a-f.]+p[-+]\d+);", text).group(1))

    inv, hi, lo = constant("inv"), constant("l_hi"), constant("l_lo")
    assert inv == float(64 / ln2)
    assert abs(Decimal(hi) + Decimal(lo) - ln2 / 64) < Decimal(2) ** -95
    mantissa = int(math.frexp(hi)[0] * 2 ** 53)
    assert mantissa % 2 ** (53 - 29) == 0 and 9601 * 2 ** 29 < 2 ** 53

WIDTHS = [(896, 72), (4864, 24), (77, 40), (40, 16), (160, 40), (96, 24)]


def golden_matmul_inputs(k, n, tokens):
    from tests.golden.inputs import matmul_inputs
    w, x = matmul_inputs(k, n, tokens, seed=k + tokens)
    return w, x


@pytest.mark.parametrize("k,n", WIDTHS)
def test_g2_matmul_i8_order_is_the_references(golden, meta, host, k, n):
    """The host restatement of the 32-chain FMA order, bitwise against the reference's generated C."""
    for tokens in (1, 3, 7):
        w, x = golden_matmul_inputs(k, n, tokens)
        key = f"g2_{k}_{n}_{tokens}"
        assert sha(w) == meta[key]["w_sha"] and sha(x) == meta[key]["x_sha"]
        q, s = R.quantize_int8(w)
        assert np.array_equal(bits(host.matmul_i8_f32(x, q, s)), bits(golden[key]))


@pytest.mark.parametrize("k,n", [(k, n) for k, n in WIDTHS if k % 32 == 0])
def test_g3_matmul_i8_vnni_order_is_the_references(golden, meta, host, k, n):
    for tokens in (1, 3, 7):
        w, x = golden_matmul_inputs(k, n, tokens)
        key = f"g3_{k}_{n}_{tokens}"
        q, s = R.quantize_int8(w)
        xq, xs, off = R.quantize_blocks(x, 32)
        assert np.array_equal(bits(host.matmul_i8_vnni(xq, xs, off, q, s)), bits(golden[key]))


def test_the_interpreter_meanings_agree_with_the_orders_to_rounding(golden):
    """The reference's interpreter (simulated int8, f64 block combine) vs its C, as it documents."""
    for key in [k for k in golden.files if (k.startswith("g2_") or k.startswith("g3_")) and not k.endswith("_interp")
                and not k.startswith("g3_quant")]:
        np.testing.assert_allclose(golden[key], golden[key + "_interp"], rtol=1e-4, atol=1e-3)
