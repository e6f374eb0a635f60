"""Attention on the GPU, bit for bit against the host oracle's chunked order.

Both kernels stage each 64-key chunk in LDS once per KV head (and, in a
prompt, per block of 4 query rows), attend every query head of the group to
it, and combine the chunk results in a second launch; these tests cover both
sides of every chunk edge, long contexts, every head width, groups of more
than 8 query heads, prompts taken in slabs when the workspace is small, the
position read from the device, back-to-back calls, and a captured graph
replayed at advancing positions.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.host_model import inverse_frequencies
from tests.conftest import bits

pytestmark = pytest.mark.gpu


def workspace(heads, d, rows, keys):
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import attention_workspace_bytes
    n = attention_workspace_bytes(heads, d, rows, keys)
    return DeviceArray((n // 4,), np.float32), n


def setup(rng, heads, kv, d, cap, m=1):
    width = (heads + 2 * kv) * d
    qkv = rng.standard_normal((m, width)).astype(np.float32)
    kc = rng.standard_normal((kv, cap, d)).astype(np.float32)
    vc = rng.standard_normal((kv, cap, d)).astype(np.float32)
    return qkv, kc, vc


@pytest.mark.parametrize("d,heads,kv", [(64, 14, 2), (32, 4, 2), (16, 4, 1), (64, 18, 2)])
@pytest.mark.parametrize("past", [0, 1, 63, 64, 65, 127, 128, 200, 511, 512, 1000, 3000])
def test_decode_attention_is_the_oracle(gpu, host, d, heads, kv, past):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"attention_decode d={d} past={past}", flush=True)
    rng = np.random.default_rng(past + d)
    cap = past + 5
    qkv, kc, vc = setup(rng, heads, kv, d, cap)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    expected = host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, past, scale)

    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    dinv, ctx = DeviceArray.from_host(inv), DeviceArray((1, heads * d), np.float32)
    pos = DeviceArray.from_host(np.array([past], np.int64))
    work, nbytes = workspace(heads, d, 1, cap)
    for use_pos in (False, True, True):
        hip.call("nc_attention_decode", [ctx, dq, dk, dv, dinv, pos if use_pos else None, None, work],
                 [heads, kv, d, 0 if use_pos else past, cap, float_bits(scale), nbytes])
        assert np.array_equal(bits(ctx.numpy()), bits(expected)), use_pos
    assert np.array_equal(bits(dk.numpy()), bits(hk)) and np.array_equal(bits(dv.numpy()), bits(hv))


@pytest.mark.parametrize("d,heads,kv", [(64, 4, 2), (32, 4, 2), (16, 2, 2), (64, 18, 2)])
@pytest.mark.parametrize("slab", [None, 8, 13, 1])
def test_prefill_and_decode_attention_agree(gpu, host, d, heads, kv, slab):
    """A prompt through nc_attention is the oracle, in one pass or in slabs of rows when the
    workspace is smaller; its last row equals a decode step at the same position."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    print(f"attention prefill d={d} heads={heads} slab={slab}", flush=True)
    rng = np.random.default_rng(d + heads)
    m, past = 130, 70
    cap = past + m
    qkv, kc, vc = setup(rng, heads, kv, d, cap, m)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    expected = host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, past, scale)
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    dinv, ctx = DeviceArray.from_host(inv), DeviceArray((m, heads * d), np.float32)
    hip.call("nc_rope_append", [dq, dk, dv, dinv], [m, heads, kv, d, past, cap])
    work, nbytes = workspace(heads, d, slab or m, past + m)
    hip.call("nc_attention", [ctx, dq, dk, dv, None, work], [m, heads, kv, d, past, cap, float_bits(scale), nbytes])
    prefill = ctx.numpy()
    assert np.array_equal(bits(prefill), bits(expected))
    # the last row again (unrotated) as a decode step at its position, over the
    # cache the prefill filled (the step rewrites its own key with the same bits)
    dq2 = DeviceArray.from_host(qkv[-1:])
    one = DeviceArray((1, heads * d), np.float32)
    work, nbytes = workspace(heads, d, 1, cap)
    hip.call("nc_attention_decode", [one, dq2, dk, dv, dinv, None, None, work],
             [heads, kv, d, past + m - 1, cap, float_bits(scale), nbytes])
    assert np.array_equal(bits(one.numpy()[0]), bits(prefill[-1]))
    assert np.array_equal(bits(dk.numpy()), bits(hk))


@pytest.mark.parametrize("d,heads,kv,m,past", [(64, 14, 2, 512, 0), (64, 14, 2, 130, 70), (64, 4, 2, 37, 5),
                                                (64, 8, 1, 66, 0), (64, 18, 2, 40, 30), (32, 4, 2, 33, 64)])
def test_every_prefill_schedule_is_the_oracle(gpu, host, d, heads, kv, m, past):
    """Each prefill schedule (2, 4, 8 or 16 rows a chunk workgroup) gives the oracle's bits, in one
    pass and with a small workspace taking the rows in slabs."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    rng = np.random.default_rng(m + heads + past)
    cap = past + m
    qkv, kc, vc = setup(rng, heads, kv, d, cap, m)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    expected = host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, past, scale)
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    dinv, ctx = DeviceArray.from_host(inv), DeviceArray((m, heads * d), np.float32)
    hip.call("nc_rope_append", [dq, dk, dv, dinv], [m, heads, kv, d, past, cap])
    for slab in (None, 11):
        work, nbytes = workspace(heads, d, slab or m, past + m)
        for schedule in range(5):
            print(f"prefill schedule {schedule} d={d} heads={heads}/{kv} m={m} past={past} slab={slab}", flush=True)
            ctx.upload(np.full((m, heads * d), np.nan, np.float32))
            hip.call("nc_attention", [ctx, dq, dk, dv, None, work],
                     [m, heads, kv, d, past, cap, float_bits(scale), nbytes, schedule])
            assert np.array_equal(bits(ctx.numpy()), bits(expected)), (schedule, slab)


def test_decode_attention_in_a_graph_at_advancing_positions(gpu, host):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray, Graph
    from nanocompile_amd.kernels import float_bits
    rng = np.random.default_rng(9)
    heads, kv, d, cap = 14, 2, 64, 300
    qkv, kc, vc = setup(rng, heads, kv, d, cap)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(0.125))
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    dinv, ctx = DeviceArray.from_host(inv), DeviceArray((1, heads * d), np.float32)
    pos = DeviceArray.from_host(np.array([0], np.int64))
    work, nbytes = workspace(heads, d, 1, cap)
    graph = Graph.capture(lambda: hip.call("nc_attention_decode", [ctx, dq, dk, dv, dinv, pos, None, work],
                                           [heads, kv, d, 0, cap, float_bits(scale), nbytes]))
    hk, hv = kc.copy(), vc.copy()
    for past in (10, 63, 64, 150, 299):
        print(f"graph replay at past={past}", flush=True)
        pos.upload(np.array([past], np.int64))
        graph.launch()
        hip.sync()
        expected = host.rope_append_attention(qkv.copy(), hk, hv, inv, heads, kv, d, past, scale)
        assert np.array_equal(bits(ctx.numpy()), bits(expected)), past


def test_decode_attention_rejects_bad_shapes(gpu):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    x = DeviceArray((4096,), np.float32)
    with pytest.raises(hip.KernelError, match="bad shape"):
        hip.call("nc_attention_decode", [x, x, x, x, x, None, None, x], [4, 2, 48, 3, 8, 0, 1 << 14])   # head_dim 48
    with pytest.raises(hip.KernelError, match="bad shape"):
        hip.call("nc_attention_decode", [x, x, x, x, x, None, None, x], [4, 2, 64, 8, 8, 0, 1 << 14])   # past + 1 > capacity
    with pytest.raises(hip.KernelError, match="null operand"):
        hip.call("nc_attention_decode", [x, x, None, x, x, None, None, x], [4, 2, 64, 3, 8, 0, 1 << 14])
    with pytest.raises(hip.KernelError, match="null operand"):
        hip.call("nc_attention_decode", [x, x, x, x, x, None, None, None], [4, 2, 64, 3, 8, 0, 1 << 14])
    with pytest.raises(hip.KernelError, match="workspace"):        # 4 heads x 1 chunk x 66 floats
        hip.call("nc_attention_decode", [x, x, x, x, x, None, None, x], [4, 2, 64, 3, 8, 0, 4 * 66 * 4 - 4])
    with pytest.raises(hip.KernelError, match="workspace"):
        hip.call("nc_attention", [x, x, x, x, None, x], [2, 4, 2, 64, 3, 8, 0, 4 * 66 * 4 - 4])


@pytest.mark.parametrize("d", [64, 32])
def test_rope_table_is_nc_cosf_and_nc_sinf(gpu, host, d):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    cap = 3000
    inv = inverse_frequencies(d, 1e6)
    table = DeviceArray((2, cap, d // 2), np.float32)
    hip.call("nc_rope_table", [table, DeviceArray.from_host(inv)], [cap, d])
    got = table.numpy()
    ang = (np.arange(cap, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    assert np.array_equal(bits(got[0]), bits(host.math("nc_cos", ang)))
    assert np.array_equal(bits(got[1]), bits(host.math("nc_sin", ang)))


@pytest.mark.parametrize("past", [0, 100, 300, 700])
def test_decode_attention_with_the_rope_table(gpu, host, past):
    """The table path (what the model runs) and the computing path give the oracle's bits."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    rng = np.random.default_rng(past + 1)
    heads, kv, d = 14, 2, 64
    cap = past + 9
    qkv, kc, vc = setup(rng, heads, kv, d, cap)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(0.125))
    expected = host.rope_append_attention(qkv.copy(), kc.copy(), vc.copy(), inv, heads, kv, d, past, scale)
    dinv = DeviceArray.from_host(inv)
    table = DeviceArray((2, cap, d // 2), np.float32)
    hip.call("nc_rope_table", [table, dinv], [cap, d])
    work, nbytes = workspace(heads, d, 1, cap)
    for tab in (table, None):
        dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
        ctx = DeviceArray((1, heads * d), np.float32)
        hip.call("nc_attention_decode", [ctx, dq, dk, dv, dinv, None, tab, work],
                 [heads, kv, d, past, cap, float_bits(scale), nbytes])
        assert np.array_equal(bits(ctx.numpy()), bits(expected)), tab is None



@pytest.mark.parametrize("m,past", [(1, 0), (5, 37), (512, 0), (130, 70)])
def test_rope_append_with_the_table_is_the_oracle(gpu, host, m, past):
    """nc_rope_append reading cos and sin from the cache's table gives the oracle's bits
    (rotated q in place, rotated k and v in the cache), as computing them does."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    print(f"rope_append table m={m} past={past}", flush=True)
    rng = np.random.default_rng(m + past)
    heads, kv, d = 14, 2, 64
    cap = past + m + 3
    qkv, kc, vc = setup(rng, heads, kv, d, cap, m)
    inv = inverse_frequencies(d, 1e6)
    dinv = DeviceArray.from_host(inv)
    table = DeviceArray((2, cap, d // 2), np.float32)
    hip.call("nc_rope_table", [table, dinv], [cap, d])
    results = []
    for tab in (table, None):
        dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
        hip.call("nc_rope_append", [dq, dk, dv, dinv, None, tab], [m, heads, kv, d, past, cap])
        results.append([bits(a.numpy()) for a in (dq, dk, dv)])
    for got, want in zip(results[0], results[1]):
        assert np.array_equal(got, want)
    hq, hk, hv = qkv.copy(), kc.copy(), vc.copy()
    host.rope_append_attention(hq, hk, hv, inv, heads, kv, d, past, 0.125)     # rotates and appends in place
    assert np.array_equal(results[0][0], bits(hq)) and np.array_equal(results[0][1], bits(hk))
    assert np.array_equal(results[0][2], bits(hv))


@pytest.mark.parametrize("d,heads,kv,m,past,slab", [(64, 14, 2, 130, 70, None), (64, 14, 2, 130, 70, 8),
                                                    (32, 4, 2, 9, 0, None), (64, 18, 2, 20, 5, None),
                                                    (64, 14, 2, 8, 1200, None)])
def test_prefill_attention_quantizes_ctx_per_token(gpu, host, d, heads, kv, m, past, slab):
    """nc_attention with xq and xs: ctx unchanged and its per-token int8 the oracle's, whether the
    combine quantizes (a row's chunk results in LDS) or a separate launch does (more than 16 heads,
    contexts whose chunk results do not fit)."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import float_bits
    from oracle import reference as R
    print(f"attention quantize d={d} heads={heads} m={m} past={past} slab={slab}", flush=True)
    rng = np.random.default_rng(m + past + heads)
    cap = past + m
    qkv, kc, vc = setup(rng, heads, kv, d, cap, m)
    inv = inverse_frequencies(d, 1e6)
    scale = float(np.float32(d ** -0.5))
    expected = host.rope_append_attention(qkv.copy(), kc.copy(), vc.copy(), inv, heads, kv, d, past, scale)
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    hip.call("nc_rope_append", [dq, dk, dv, DeviceArray.from_host(inv)], [m, heads, kv, d, past, cap])
    work, nbytes = workspace(heads, d, slab or m, past + m)
    ctx = DeviceArray((m, heads * d), np.float32)
    xq, xs = DeviceArray((m, heads * d), np.int8), DeviceArray((m,), np.float32)
    hip.call("nc_attention", [ctx, dq, dk, dv, None, work, xq, xs],
             [m, heads, kv, d, past, cap, float_bits(scale), nbytes])
    assert np.array_equal(bits(ctx.numpy()), bits(expected))
    eq, es = R.quantize_token(expected)
    assert np.array_equal(xq.numpy(), eq) and np.array_equal(bits(xs.numpy()), bits(es))


@pytest.mark.parametrize("heads,kv,d,k", [(14, 2, 64, 896), (4, 2, 32, 128)])
@pytest.mark.parametrize("m,past", [(1, 0), (16, 5), (130, 70), (512, 0)])
def test_qkv_projection_with_rope_is_projection_then_rope_append(gpu, heads, kv, d, k, m, past):
    """nc_matmul_i8_token_rope (RoPE and the cache append in the GEMM's epilogue) leaves qkv and
    both caches bit for bit as nc_matmul_i8_token followed by nc_rope_append with the table does,
    with the position from the host and from the device, under the library's tile and every MFMA
    tile one head wide."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    print(f"qkv rope epilogue heads={heads} d={d} m={m} past={past}", flush=True)
    rng = np.random.default_rng(m * 7 + past + d)
    w = (heads + 2 * kv) * d
    cap = past + m + 3
    xq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    xs = (rng.random(m) * 0.05 + 1e-3).astype(np.float32)
    q = rng.integers(-127, 128, (w, k)).astype(np.int8)
    qs = (rng.random(w) * 1e-3 + 1e-4).astype(np.float32)
    bias = rng.standard_normal(w).astype(np.float32)
    kc0 = rng.standard_normal((kv, cap, d)).astype(np.float32)
    vc0 = rng.standard_normal((kv, cap, d)).astype(np.float32)
    inv = inverse_frequencies(d, 1e6)
    table = DeviceArray((2, cap, d // 2), np.float32)
    hip.call("nc_rope_table", [table, DeviceArray.from_host(inv)], [cap, d])
    dxq, dxs, dq, dqs, db = (DeviceArray.from_host(a) for a in (xq, xs, q, qs, bias))
    pos = DeviceArray.from_host(np.array([past], np.int64))
    schedules = [0] + [sch for sch in range(16, 25) if hip.schedule_info(sch)["tile_n"] == d]
    for use_pos in (False, True):
        p = pos if use_pos else None
        host_past = 0 if use_pos else past
        qkv = DeviceArray((m, w), np.float32)
        kc, vc = DeviceArray.from_host(kc0), DeviceArray.from_host(vc0)
        hip.call("nc_matmul_i8_token", [qkv, dxq, dxs, dq, dqs, db, None], [m, w, k, 0])
        hip.call("nc_rope_append", [qkv, kc, vc, DeviceArray.from_host(inv), p, table],
                 [m, heads, kv, d, host_past, cap])
        expected = (qkv.numpy(), kc.numpy(), vc.numpy())
        for schedule in schedules:
            print(f"  schedule {schedule} position from the {'device' if use_pos else 'host'}", flush=True)
            qkv = DeviceArray((m, w), np.float32)
            kc, vc = DeviceArray.from_host(kc0), DeviceArray.from_host(vc0)
            hip.call("nc_matmul_i8_token_rope", [qkv, dxq, dxs, dq, dqs, db, kc, vc, table, p],
                     [m, w, k, heads, kv, d, host_past, cap, schedule])
            for a, b in zip((qkv.numpy(), kc.numpy(), vc.numpy()), expected):
                assert np.array_equal(bits(a), bits(b)), (use_pos, schedule)


def test_qkv_projection_with_rope_rejects_bad_shapes(gpu):
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    x = DeviceArray((1 << 16,), np.float32)
    with pytest.raises(hip.KernelError, match="bad shape"):        # W is not (heads + 2 kv) * D
        hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, x], [4, 1000, 896, 14, 2, 64, 0, 8])
    with pytest.raises(hip.KernelError, match="bad shape"):        # head_dim 48
        hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, x], [4, 18 * 48, 896, 14, 2, 48, 0, 8])
    with pytest.raises(hip.KernelError, match="bad shape"):        # past + M past the capacity
        hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, x], [4, 1152, 896, 14, 2, 64, 6, 8])
    with pytest.raises(hip.KernelError, match="null operand"):     # no table
        hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, None], [4, 1152, 896, 14, 2, 64, 0, 8])
    # tiles whose n is not one head (the epilogue rotates a tile as a head) are refused before launch
    for schedule, d in ((18, 64), (19, 64), (22, 64), (23, 64), (16, 32), (22, 32)):
        width = (14 + 2 * 2) * d
        with pytest.raises(hip.KernelError, match="not one head wide"):
            hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, x], [4, width, 896, 14, 2, d, 0, 8, schedule])
    with pytest.raises(hip.KernelError, match="no such schedule"):
        hip.call("nc_matmul_i8_token_rope", [x, x, x, x, x, None, x, x, x], [4, 1152, 896, 14, 2, 64, 0, 8, 25])
