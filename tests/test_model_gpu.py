"""The fused groups and the whole model on the GPU, against the host C oracle and the reference.

Against the host oracle (oracle/nc_model.c, the GPU kernels' orders replayed
in C with the same exp/sin/cos) everything is bitwise: every float, every
token. Against the reference's own outputs (tests/golden, made by running the
reference) the fused groups are held to the reference's tolerance.
"""

from __future__ import annotations

from dataclasses import replace
from pathlib import Path

import numpy as np
import pytest

from nanocompile_amd.models.config import QWEN25_05B, TINY, TINY_STD, random_weights
from oracle.host_model import inverse_frequencies
from tests.conftest import bits

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def run(name, outputs, inputs, sizes):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    outs = [DeviceArray(shape, np.float32) for shape in outputs]
    ins = [a if a is None else DeviceArray.from_host(np.ascontiguousarray(a)) for a in inputs]
    hip.call(name, outs + ins, sizes)
    hip.sync()
    return [o.numpy() for o in outs]


# -- fused groups -------------------------------------------------------------------


@pytest.mark.parametrize("seq,past", [(1, 12), (5, 3)])
def test_softmax_causal(gpu, host, golden, seq, past):
    key = f"g4_softmax_{seq}_{past}"
    s = golden[key + "_s"]
    (y,) = run("nc_softmax_causal", [s.shape], [s], [s.shape[0], seq, past])
    assert np.array_equal(bits(y), bits(host.softmax_causal(s, past)))
    np.testing.assert_allclose(y, golden[key + "_y"], rtol=2e-6, atol=1e-6)


def test_softmax_long_rows(gpu, host):
    rng = np.random.default_rng(3)
    s = (rng.standard_normal((3, 4, 1000 + 4)) * 5).astype(np.float32)
    (y,) = run("nc_softmax_causal", [s.shape], [s], [3, 4, 1000])
    assert np.array_equal(bits(y), bits(host.softmax_causal(s, 1000)))


def test_silu_mul(gpu, host, golden):
    g, u = golden["g4_silu_g"], golden["g4_silu_u"]
    (y,) = run("nc_silu_mul", [g.shape], [g, u], [g.size])
    assert np.array_equal(bits(y), bits(host.silu_mul(g, u)))
    np.testing.assert_allclose(y, golden["g4_silu_y"], rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("seq,past", [(1, 511), (7, 0), (2, 100000)])
def test_rope(gpu, host, golden, seq, past):
    key = f"g4_rope_{seq}_{past}"
    x = golden[key + "_x"]
    inv = inverse_frequencies(64, 1e6)
    (y,) = run("nc_rope", [x.shape], [x, inv], [x.shape[0], seq, 64, past])
    assert np.array_equal(bits(y), bits(host.rope(x, inv, past)))
    np.testing.assert_allclose(y, golden[key + "_y"], rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("m,past", [(1, 0), (1, 200), (6, 0), (5, 37)])
def test_rope_append_and_attention(gpu, host, m, past):
    """Qwen2.5-0.5B's attention shape: 14 query heads over 2 KV heads of 64."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"attention m={m} past={past}", flush=True)
    heads, kv, d, cap = 14, 2, 64, 256
    rng = np.random.default_rng(m * 1000 + past)
    qkv = rng.standard_normal((m, (heads + 2 * kv) * d)).astype(np.float32)
    kc = np.zeros((kv, cap, d), np.float32)
    vc = np.zeros((kv, cap, d), np.float32)
    kc[:, :past] = rng.standard_normal((kv, past, d))
    vc[:, :past] = rng.standard_normal((kv, past, d))
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    ctx = DeviceArray((m, heads * d), np.float32)
    hip.call("nc_rope_append", [dq, dk, dv, DeviceArray.from_host(inv)], [m, heads, kv, d, past, cap])
    from nanocompile_amd.kernels import attention_workspace_bytes
    nbytes = attention_workspace_bytes(heads, d, m, past + m)
    work = DeviceArray((nbytes // 4,), np.float32)
    hip.call("nc_attention", [ctx, dq, dk, dv, None, work], [m, heads, kv, d, past, cap, float_bits(scale), nbytes])
    hip.sync()
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    expected = host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, past, scale)
    assert np.array_equal(bits(dq.numpy()), bits(hq))
    assert np.array_equal(bits(dk.numpy()), bits(hk)) and np.array_equal(bits(dv.numpy()), bits(hv))
    assert np.array_equal(bits(ctx.numpy()), bits(expected))


def test_swiglu_pair(gpu, host):
    from nanocompile_amd import kernels
    rng = np.random.default_rng(9)
    for m in (1, 3, 9):
        xq = rng.integers(-127, 128, (m, 896)).astype(np.int8)
        xs = (rng.random(m) * 0.1).astype(np.float32)
        qg, qu = (rng.integers(-127, 128, (4864, 896)).astype(np.int8) for _ in range(2))
        sg, su = ((rng.random(4864) * 1e-3).astype(np.float32) for _ in range(2))
        (h,) = run("nc_matmul_i8_token_swiglu", [(m, 4864)], [xq, xs, qg, sg, qu, su], [m, 4864, 896])
        assert np.array_equal(bits(h), bits(host.matmul_i8_token_swiglu(xq, xs, qg, sg, qu, su)))
    del kernels


def test_lm_head_and_argmax(gpu):
    """The reference's k-order sum (checked in exact arithmetic bounds) and numpy.argmax."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    rng = np.random.default_rng(4)
    v, h = 1000, 96
    table = (rng.standard_normal((v, h)) * 0.1).astype(np.float32)
    x = rng.standard_normal((2, h)).astype(np.float32)
    table[777] = table[123]                                     # a tie: the first index must win
    x[1] = 0.0
    packed = DeviceArray((-(-v // 64) * 64, h), np.float32)
    hip.call("nc_pack_rows64", [packed, DeviceArray.from_host(table)], [v, h])
    logits, best, index = DeviceArray((2, v), np.float32), DeviceArray((2,), np.uint64), DeviceArray((2,), np.int64)
    hip.call("nc_argmax_clear", [best], [2])
    hip.call("nc_lm_head", [logits, best, DeviceArray.from_host(x), packed], [2, v, h])
    hip.call("nc_argmax_index", [index, best], [2])
    hip.sync()
    expected = np.zeros((2, v), np.float32)
    for k in range(h):                                           # the reference's order, one k at a time
        expected = (expected + (x[:, k:k + 1] * table[None, :, k]).astype(np.float32)).astype(np.float32)
    got = logits.numpy()
    assert np.array_equal(bits(got), bits(expected))
    assert list(index.numpy()) == [int(np.argmax(expected[0])), 0]
    # one key per workgroup (s[4] = 1), reduced by nc_argmax_index: no clear needed, same answers
    from nanocompile_amd.kernels import argmax_slots
    slots = argmax_slots(v)
    keys = DeviceArray((2, slots), np.uint64)
    keys.upload(np.full((2, slots), 12345, np.uint64))                  # stale keys are overwritten
    hip.call("nc_lm_head", [None, keys, DeviceArray.from_host(x), packed], [2, v, h, 0, 1])
    hip.call("nc_argmax_index", [index, keys], [2, slots])
    hip.sync()
    assert list(index.numpy()) == [int(np.argmax(expected[0])), 0]


@pytest.mark.parametrize("v", [64, 255, 256, 1000, 151936, 200000])   # 200000: keys past one round of loads
def test_argmax_per_workgroup_keys_break_ties_low(gpu, v):
    """Per-workgroup keys reduced by nc_argmax_index and by nc_decode_advance: numpy.argmax's first
    index, with the maximum placed in the last workgroup and tied in the first."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import argmax_slots
    print(f"argmax slots v={v}", flush=True)
    rng = np.random.default_rng(v)
    h = 896 if v == 151936 else 64
    table = (rng.standard_normal((v, h)) * 0.1).astype(np.float32)
    table[v - 1] = 1.0
    table[min(3, v - 1)] = 1.0                                  # a tie with an earlier row
    x = np.ones((1, h), np.float32)
    packed = DeviceArray((-(-v // 64) * 64, h), np.float32)
    hip.call("nc_pack_rows64", [packed, DeviceArray.from_host(table)], [v, h])
    slots = argmax_slots(v)
    keys, index = DeviceArray((slots,), np.uint64), DeviceArray((1,), np.int64)
    hip.call("nc_lm_head", [None, keys, DeviceArray.from_host(x), packed], [1, v, h, 0, 1])
    hip.call("nc_argmax_index", [index, keys], [1, slots])
    ids, tokens = DeviceArray((1,), np.int64), DeviceArray.from_host(np.zeros(4, np.int64))
    pos = DeviceArray.from_host(np.array([0], np.int64))
    hip.call("nc_decode_advance", [ids, tokens, keys, pos], [4, 0, 0, slots])
    hip.sync()
    assert index.numpy()[0] == min(3, v - 1) and tokens.numpy()[1] == min(3, v - 1)


# -- the model ------------------------------------------------------------------------


@pytest.fixture(scope="module")
def tiny(gpu, host):
    from nanocompile_amd.models.qwen2 import Qwen2
    from oracle.host_model import HostQwen2
    weights = random_weights(TINY, seed=5, std=TINY_STD)
    return Qwen2(TINY, weights, max_tokens=64), HostQwen2(TINY, weights, capacity=64)


PROMPTS = ([4, 5, 6], [7, 8], [1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5])


def test_tiny_greedy_tokens_are_the_oracles(tiny):
    from nanocompile_amd.models.qwen2 import greedy
    model, oracle_model = tiny
    for prompt in PROMPTS:
        expected = oracle_model.greedy(prompt, 12)
        assert greedy(model, prompt, 12) == expected
        assert greedy(model, prompt, 4, use_cache=False) == expected[:4]


def test_tiny_logits_are_bitwise_the_oracles(tiny):
    model, oracle_model = tiny
    ids = PROMPTS[3]
    oracle_model.reset()
    expected, _ = oracle_model.forward(ids, all_rows=True)
    got = model.forward(ids)
    assert np.array_equal(bits(got), bits(expected))


def test_tiny_cached_steps_are_one_pass(tiny):
    """Each row's arithmetic does not depend on how the tokens were batched."""
    model, _ = tiny
    ids = PROMPTS[3]
    whole = model.forward(ids)
    cache = model.new_cache(16)
    rows = [model.forward(ids[:5], cache=cache)]
    rows += [model.forward([t], cache=cache) for t in ids[5:]]
    assert np.array_equal(bits(np.concatenate(rows)), bits(whole))
    keys, values = cache.past()
    assert keys.shape == (2, 2, 11, 32) and np.isfinite(keys).all() and np.isfinite(values).all()


def test_tiny_token_out_of_range_is_a_kernel_error(tiny):
    from nanocompile_amd.hip import KernelError
    model, _ = tiny
    with pytest.raises(KernelError, match="out of range"):
        model.forward([1, 256])
    with pytest.raises(KernelError, match="out of range"):
        model.forward([-1])
    model.forward([1, 2])                                          # and the model still works


def test_full_width_model_matches_the_oracle(gpu, host):
    """Qwen2.5-0.5B's widths and vocabulary, two layers: prefill then decode, bitwise."""
    from nanocompile_amd.models.qwen2 import Qwen2, greedy
    from oracle.host_model import HostQwen2
    config = replace(QWEN25_05B, num_hidden_layers=2)
    weights = random_weights(config, seed=11)
    model = Qwen2(config, weights, max_tokens=64)
    oracle_model = HostQwen2(config, weights, capacity=64)
    prompt = list(np.random.default_rng(2).integers(0, config.vocab_size, 20))
    expected = oracle_model.greedy(prompt, 6)
    assert greedy(model, prompt, 6) == expected
    oracle_model.reset()
    logits, _ = oracle_model.forward(prompt)
    assert np.array_equal(bits(model.forward(prompt, last_only=True)), bits(logits))


@pytest.mark.parametrize("full", [False, True])
def test_fused_decode_step_is_the_unfused_step(gpu, tiny, full):
    """The one-token kernels (prologues and RoPE fused in) compute the unfused kernels' bits."""
    from nanocompile_amd.models.qwen2 import Qwen2
    if full:
        config = replace(QWEN25_05B, num_hidden_layers=2)
        model = Qwen2(config, random_weights(config, seed=13), max_tokens=32)
    else:
        model, _ = tiny
    assert model.fused_decode
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, model.config.vocab_size, 9)]
    rows = {}
    for fused in (True, False):
        model.fused_decode = fused
        cache = model.new_cache(16)
        out = [model.forward(prompt, cache=cache, last_only=True)]
        for t in (5, 17, 3):
            out.append(model.forward([t], cache=cache, last_only=True))
        rows[fused] = np.concatenate(out)
    model.fused_decode = True
    assert np.array_equal(bits(rows[True]), bits(rows[False]))


def test_device_greedy_loop_is_greedy(tiny):
    """generate(): the whole decode loop on the device, one graph replay per token."""
    from nanocompile_amd.models.qwen2 import greedy
    model, oracle_model = tiny
    for prompt in PROMPTS:
        expected = oracle_model.greedy(prompt, 20)
        assert model.generate(prompt, 20) == expected
        assert greedy(model, prompt, 20) == expected
    assert model.generate([9], 1) == oracle_model.greedy([9], 1)


def test_decode_advance_gathers_the_next_row(gpu):
    """nc_decode_advance with x: the argmax's token appended, pos advanced, the key cleared, and
    the token's embedding row in x; an argmax key that names no row is Fail code 1 and x zero."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray, KernelError
    rng = np.random.default_rng(3)
    V, H, cap = 50, 40, 8
    table = rng.standard_normal((V, H)).astype(np.float32)
    dt, x = DeviceArray.from_host(table), DeviceArray((H,), np.float32)
    ids, tokens = DeviceArray((1,), np.int64), DeviceArray.from_host(np.zeros(cap, np.int64))
    pos = DeviceArray.from_host(np.array([2], np.int64))
    token = 17
    best = DeviceArray.from_host(np.array([(123 << 32) | (0xFFFFFFFF - token)], np.uint64))
    hip.call("nc_decode_advance", [ids, tokens, best, pos, x, dt], [cap, H, V])
    hip.sync()
    assert tokens.numpy()[3] == token and ids.numpy()[0] == token and pos.numpy()[0] == 3
    assert best.numpy()[0] == 0 and np.array_equal(x.numpy(), table[token])
    best.upload(np.array([0], np.uint64))          # no argmax: the key names id 2^32 - 1
    hip.call("nc_decode_advance", [ids, tokens, best, pos, x, dt], [cap, H, V])
    with pytest.raises(KernelError, match="out of range"):
        hip.sync()
    assert not x.numpy().any()


def test_long_prompt_in_attention_slabs_is_bitwise_one_pass(gpu, monkeypatch):
    """A 300-token prompt whose attention workspace holds only a few rows' chunk results (so
    nc_attention takes the rows in slabs) gives the same logits and cache, bit for bit, as one pass."""
    from nanocompile_amd.kernels import attention_workspace_bytes
    from nanocompile_amd.models import qwen2
    weights = random_weights(TINY, seed=5, std=TINY_STD)
    model = qwen2.Qwen2(TINY, weights, max_tokens=320)
    prompt = np.random.default_rng(8).integers(0, TINY.vocab_size, 300)
    runs = []
    for rows in (None, 5):
        if rows is not None:                       # 5 rows' worth of chunk results: 60 slabs of 5 rows
            per_row = attention_workspace_bytes(TINY.num_attention_heads, TINY.head_dim, 1, 310)
            monkeypatch.setattr(qwen2, "WORKSPACE_BYTES", per_row * rows)
        cache = model.new_cache(310)
        assert rows is None or cache.work_bytes == attention_workspace_bytes(
            TINY.num_attention_heads, TINY.head_dim, rows, 310)
        logits = model.forward(prompt, cache)
        step = model.forward([int(np.argmax(logits[-1]))], cache, last_only=True)
        filled = cache.length                      # rows past it are whatever the allocation held
        runs.append((bits(logits), bits(step), bits(cache.keys.numpy()[:, :, :filled]),
                     bits(cache.values.numpy()[:, :, :filled])))
    for a, b in zip(*runs):
        assert np.array_equal(a, b)
