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


def _causal(s: np.ndarray, past: int) -> np.ndarray:
    """scores + the causal mask (nn.py:123-135): row i sees columns 0 .. past + i."""
    seq, total = s.shape[-2], s.shape[-1]
    allowed = np.arange(total)[None, :] <= np.arange(seq)[:, None] + past
    return (s + np.where(allowed, np.float32(0.0), np.float32(-np.inf))).astype(np.float32)


@pytest.mark.parametrize("seq,past", [(1, 12), (5, 3)])
def test_g4_softmax_in_index_order_is_the_references(golden, host, seq, past):
    """The reference's softmax row kernel with the causal mask, bit for bit, given the C
    library's expf (the reference's): the order of its sum and its divide are pinned."""
    s = golden[f"g4_softmax_{seq}_{past}_s"]
    y = R.softmax_index_order(_causal(s, past), lambda v: host.math("exp", v))
    assert np.array_equal(bits(y), bits(golden[f"g4_softmax_{seq}_{past}_y"]))


def test_attention_index_order_is_attention_and_a_dropped_max_is_caught(host):
    """Against float64 softmax attention (within float32 rounding) on Qwen2.5-0.5B's heads,
    prefill rows and decode at several positions; a restatement that forgot to subtract the
    maximum overflows exp on large scores and fails the same check."""
    rng = np.random.default_rng(9)
    heads, kv, d = 14, 2, 64
    exp = lambda v: host.math("nc_exp", v)                     # noqa: E731

    def float64_attention(q, kc, vc, past):
        out = np.zeros(q.shape, np.float64)
        for i in range(q.shape[0]):
            t = past + i + 1
            for h in range(heads):
                k, v = kc[h // (heads // kv), :t].astype(np.float64), vc[h // (heads // kv), :t].astype(np.float64)
                z = k @ q[i, h].astype(np.float64) * 0.125
                p = np.exp(z - z.max())
                out[i, h] = (p / p.sum()) @ v
        return out

    for m, past, spread in [(1, 0, 1.0), (1, 70, 1.0), (5, 3, 1.0), (3, 40, 60.0)]:
        q = (rng.standard_normal((m, heads, d)) * spread).astype(np.float32)
        kc = rng.standard_normal((kv, past + m, d)).astype(np.float32)
        vc = rng.standard_normal((kv, past + m, d)).astype(np.float32)
        got = R.attention_index_order(q, kc, vc, past, 0.125, exp)
        # scores of magnitude ~spread * 8 carry float32 rounding of that size into the softmax
        tol = dict(rtol=1e-5 * spread, atol=2e-6 * spread)
        np.testing.assert_allclose(got, float64_attention(q, kc, vc, past), **tol)
        if spread > 10:
            def no_max(z, ex):
                e = np.asarray(ex(z.astype(np.float32)), np.float32)
                return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
            original = R.softmax_index_order
            R.softmax_index_order = no_max
            try:
                with np.errstate(all="ignore"):
                    bad = R.attention_index_order(q, kc, vc, past, 0.125, exp)
            finally:
                R.softmax_index_order = original
            assert not np.allclose(bad, float64_attention(q, kc, vc, past), equal_nan=False, **tol)


def test_g6_fixture_is_the_workload_and_consistent():
    """G6 (make_g6.py) is config 5's exact workload: seed-0 weights, the seed-1 128-token
    prompt; in each mode the recorded argmax at each checked call is that call's token."""
    from nanocompile_amd.models.config import QWEN25_05B
    meta = json.loads((HERE / "g6.json").read_text())
    prompt = [int(t) for t in np.random.default_rng(meta["prompt_seed"]).integers(0, QWEN25_05B.vocab_size, 128)]
    assert meta["seed"] == 0 and prompt == meta["prompt"] and meta["checked_past"] == [0, 255, 383]
    with np.load(HERE / "g6.npz", allow_pickle=False) as z:
        for tag in ("int8", "vnni", "int8_ncmath", "vnni_ncmath"):
            tokens = meta[tag]["tokens"]
            assert len(tokens) == meta["new_tokens"] == 257
            for past, call in ((0, 0), (255, 128), (383, 256)):
                assert tokens[call] == meta[tag][f"argmax_{past}"]
                sampled = z[f"{tag}_logits_{past}"]
                assert sampled.shape == (-(-QWEN25_05B.vocab_size // meta["stride"]),)
                assert float(sampled.max()) <= float.fromhex(meta[tag][f"max_{past}"])


def test_g6_modes_differ_and_vnni_moves_with_the_math_library():
    """The two modes' logits differ well beyond the logits bar, so passing one is no accident of
    the other. int8 is insensitive to the math library (the same 257 tokens with the C library's
    exp/sin/cos and with this package's, logits within 1e-5); int8-vnni is not: the reference's
    own runs part at the 10th token and their prompt logits differ by more than 1% of the
    largest, the size of the difference a one-ulp change of the norm weights makes."""
    meta = json.loads((HERE / "g6.json").read_text())
    with np.load(HERE / "g6.npz", allow_pickle=False) as z:
        a, b = z["int8_logits_0"], z["vnni_logits_0"]
        assert np.max(np.abs(a - b)) / np.max(np.abs(a)) > 1e-3
        assert meta["int8"]["tokens"] == meta["int8_ncmath"]["tokens"]
        for past in (0, 255, 383):
            x, y = z[f"int8_logits_{past}"], z[f"int8_ncmath_logits_{past}"]
            assert np.max(np.abs(x - y)) / np.max(np.abs(x)) < 1e-5
        x, y = z["vnni_logits_0"], z["vnni_ncmath_logits_0"]
        assert np.max(np.abs(x - y)) / np.max(np.abs(x)) > 1e-2
    glibc, ours = meta["vnni"]["tokens"], meta["vnni_ncmath"]["tokens"]
    assert glibc[:9] == ours[:9] and glibc[9] != ours[9]
