"""BASELINE configs 4 and 5 at their stated sizes, on the GPU, against the host C oracle.

Config 4's largest kernel: prefill attention over a 512-token prompt with
Qwen2.5-0.5B's heads (14 query heads over 2 KV heads of 64), past 0, with the
context's per-token int8 written by the combine step, bit for bit against the
oracle's chunked order (oracle/nc_model.c).

Config 5, the whole 24-layer model: seeded random-init weights, a 128-token
uniform-random prompt, then 256 greedy tokens (past up to 384), the same
workload bench.py times. The tokens of the device loop (``generate``: one
graph replay per token) must be the host C model's, and the logits must be
bitwise the host's at three positions: the prompt's last row (past 0), a
decode step at past 255, and the last decode step at past 383.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from nanocompile_amd.models.config import QWEN25_05B, random_weights
from oracle import reference as R
from oracle.host_model import inverse_frequencies
from tests.conftest import bits

pytestmark = pytest.mark.gpu

PROMPT, NEW_TOKENS = 128, 256
SEED = 0                        # bench.py's weights seed; the prompt draws from SEED + 1


def test_config4_prefill_attention_at_512_rows(gpu, host):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import attention_workspace_bytes, float_bits
    heads, kv, d, m = 14, 2, 64, 512
    print(f"config 4 attention m={m} heads={heads}/{kv} d={d}", flush=True)
    rng = np.random.default_rng(44)
    qkv = rng.standard_normal((m, (heads + 2 * kv) * d)).astype(np.float32)
    kc = np.zeros((kv, m, d), np.float32)
    vc = np.zeros((kv, m, d), np.float32)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    expected = host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, 0, scale)
    exq, exs = R.quantize_token(expected)

    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    dinv, ctx = DeviceArray.from_host(inv), DeviceArray((m, heads * d), np.float32)
    xq, xs = DeviceArray((m, heads * d), np.int8), DeviceArray((m,), np.float32)
    nbytes = attention_workspace_bytes(heads, d, m, m)
    work = DeviceArray((nbytes // 4,), np.float32)
    hip.call("nc_rope_append", [dq, dk, dv, dinv], [m, heads, kv, d, 0, m])
    hip.call("nc_attention", [ctx, dq, dk, dv, None, work, xq, xs],
             [m, heads, kv, d, 0, m, float_bits(scale), nbytes])
    hip.sync()
    assert np.array_equal(bits(ctx.numpy()), bits(expected))
    assert np.array_equal(xq.numpy(), exq) and np.array_equal(bits(xs.numpy()), bits(exs))
    assert np.array_equal(bits(dk.numpy()), bits(hk)) and np.array_equal(bits(dv.numpy()), bits(hv))


@pytest.fixture(scope="module")
def config5(gpu, host):
    from nanocompile_amd.models.qwen2 import Qwen2
    from oracle.host_model import HostQwen2
    print("config 5: drawing the 24-layer model's weights", flush=True)
    weights = random_weights(QWEN25_05B, seed=SEED)
    prompt = [int(t) for t in np.random.default_rng(SEED + 1).integers(0, QWEN25_05B.vocab_size, PROMPT)]
    host.set_threads(min(16, os.cpu_count() or 1))
    model = Qwen2(QWEN25_05B, weights, max_tokens=PROMPT)
    oracle_model = HostQwen2(QWEN25_05B, weights, capacity=PROMPT + NEW_TOKENS + 1)
    print("config 5: host C model decoding 257 tokens", flush=True)
    expected = oracle_model.greedy(prompt, NEW_TOKENS + 1)     # one more: its step runs at past 383
    return model, oracle_model, prompt, expected


def test_config5_device_loop_decodes_the_host_models_256_tokens(config5):
    model, _, prompt, expected = config5
    print("config 5: device loop, 256 tokens", flush=True)
    assert model.generate(prompt, NEW_TOKENS) == expected[:NEW_TOKENS]


def test_config5_logits_are_bitwise_at_past_0_255_and_383(config5):
    """The host's greedy tokens fed back in the same chunks on both sides: the prompt, then
    decode-token chunks through the prefill kernels, with single decode steps at past 255
    and 383 (the one-token fused kernels; the step at 383 is the one after the 256th token)."""
    model, oracle_model, prompt, expected = config5
    fed = expected[:NEW_TOKENS]                           # the inputs at positions 128 .. 383
    chunks = [prompt, fed[:127], fed[127:128], fed[128:255], fed[255:256]]
    assert sum(map(len, chunks)) == PROMPT + NEW_TOKENS and len(chunks[-1]) == 1
    cache = model.new_cache(PROMPT + NEW_TOKENS + 1)
    oracle_model.reset()
    checked = []
    for ids in chunks:
        past = cache.length
        print(f"config 5 logits: {len(ids)} tokens at past {past}", flush=True)
        got = model.forward(ids, cache=cache, last_only=True)
        want, token = oracle_model.forward(ids)
        if past in (0, 255, 383):
            assert np.array_equal(bits(got), bits(want)), past
            checked.append(past)
        assert int(np.argmax(got[-1])) == token
    assert checked == [0, 255, 383]
