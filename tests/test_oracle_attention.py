"""The host oracle's attention, pinned by the mathematics it restates.

The GPU kernels (and the oracle replaying them) compute softmax(q K^T * scale) V
(models/qwen2.py:113-155) in 64-key chunks, each normalised by its own max,
combined afterwards. That split is exact in real arithmetic, so the float32
result must agree with float64 attention to rounding at every context length,
on both sides of every chunk edge; a dropped rescale w_j, a wrong chunk edge or
a transposed K would be off by far more.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.host_model import inverse_frequencies


def rotate(x, pos, inv):
    """RoPE in float64 (nn.py:78-106): half-split pairs."""
    half = x.shape[-1] // 2
    ang = pos * inv.astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], axis=-1)


def attention64(q, K, V, scale):
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ V.astype(np.float64)


@pytest.mark.parametrize("past", [0, 62, 63, 64, 127, 128, 300, 700])
@pytest.mark.parametrize("d,heads,kv", [(64, 14, 2), (32, 4, 2)])
def test_oracle_attention_is_softmax_attention(host, past, d, heads, kv):
    rng = np.random.default_rng(past * 7 + d)
    m = 2
    cap = past + m + 3
    width = (heads + 2 * kv) * d
    qkv = rng.standard_normal((m, width)).astype(np.float32)
    kc = rng.standard_normal((kv, cap, d)).astype(np.float32)
    vc = rng.standard_normal((kv, cap, d)).astype(np.float32)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    raw = qkv.copy()
    ctx = host.rope_append_attention(qkv, kc, vc, inv, heads, kv, d, past, scale)
    group = heads // kv
    for i in range(m):
        pos = past + i
        for h in range(heads):
            g = h // group
            q = rotate(raw[i, h * d:(h + 1) * d], pos, inv)
            k_new = rotate(raw[i, (heads + g) * d:(heads + g + 1) * d], pos, inv)
            K = kc[g, : pos + 1].astype(np.float64).copy()
            K[past:pos + 1] = [rotate(raw[r, (heads + g) * d:(heads + g + 1) * d], past + r, inv)
                               for r in range(i + 1)]
            np.testing.assert_allclose(K[pos], k_new, rtol=0, atol=1e-5)
            V = vc[g, : pos + 1]
            expected = attention64(q, K, V, scale)
            got = ctx[i, h * d:(h + 1) * d].astype(np.float64)
            assert np.max(np.abs(got - expected)) <= 2e-6 * max(1.0, np.max(np.abs(V))), (i, h)


def test_single_chunk_is_the_plain_ratio(host):
    """Up to 64 keys there is one chunk and no rescaling: out = (sum p_t v_t) / (sum p_t)."""
    rng = np.random.default_rng(11)
    d, heads, kv, past = 64, 2, 1, 40
    qkv = rng.standard_normal((1, (heads + 2 * kv) * d)).astype(np.float32)
    kc = rng.standard_normal((kv, 64, d)).astype(np.float32)
    vc = np.zeros((kv, 64, d), np.float32)
    vc[0, :, 0] = 1.0                       # value 1 in column 0: the output is sum p / sum p = 1
    qkv[0, (heads + kv) * d:] = 0
    qkv[0, (heads + kv) * d] = 1.0          # the new token's value too
    inv = inverse_frequencies(d, 1e6)
    ctx = host.rope_append_attention(qkv, kc, vc, inv, heads, kv, d, past, float(np.float32(0.125)))
    np.testing.assert_allclose(ctx[0, 0], 1.0, rtol=2e-7)
    assert np.all(ctx[0, 1:d] == 0)


def test_nan_propagates(host):
    rng = np.random.default_rng(12)
    d, heads, kv, past = 32, 2, 1, 100
    qkv = rng.standard_normal((1, (heads + 2 * kv) * d)).astype(np.float32)
    kc = rng.standard_normal((kv, 128, d)).astype(np.float32)
    vc = rng.standard_normal((kv, 128, d)).astype(np.float32)
    kc[0, 70, 3] = np.nan
    ctx = host.rope_append_attention(qkv, kc, vc, inverse_frequencies(d, 1e6), heads, kv, d, past, 0.25)
    assert np.all(np.isnan(ctx))
