"""nc_attention_decode_static: decode attention with its workspace in the library's own device array.

It must compute nc_attention_decode's bits (the same kernels with a caller's
workspace), on consecutive calls that share the array (the second smaller
than the first, so stale chunk results of the first are still there), with
the position given on the host or read on the device, and it must reject a
problem whose chunk results exceed the array before launching anything.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.host_model import inverse_frequencies
from tests.conftest import bits

pytestmark = pytest.mark.gpu

HEADS, KV, D = 14, 2, 64


def attend(entry, qkv, kc, vc, past, use_pos, table):
    """One call of ``entry`` on fresh device copies; returns (ctx, kcache, vcache) on the host."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    from nanocompile_amd.kernels import attention_workspace_bytes, float_bits
    cap = kc.shape[1]
    scale = float(np.float32(D ** -0.5))
    dq, dk, dv = DeviceArray.from_host(qkv), DeviceArray.from_host(kc), DeviceArray.from_host(vc)
    inv = DeviceArray.from_host(inverse_frequencies(D, 1e6))
    ctx = DeviceArray((1, HEADS * D), np.float32)
    pos = DeviceArray.from_host(np.array([past], np.int64)) if use_pos else None
    rope = None
    if table:
        rope = DeviceArray((2, cap, D // 2), np.float32)
        hip.call("nc_rope_table", [rope, inv], [cap, D])
    host_past = 0 if use_pos else past
    if entry == "nc_attention_decode":
        nbytes = attention_workspace_bytes(HEADS, D, 1, cap if use_pos else past + 1)
        work = DeviceArray((nbytes // 4,), np.float32)
        hip.call(entry, [ctx, dq, dk, dv, inv, pos, rope, work],
                 [HEADS, KV, D, host_past, cap, float_bits(scale), nbytes])
    else:
        hip.call(entry, [ctx, dq, dk, dv, inv, pos, rope], [HEADS, KV, D, host_past, cap, float_bits(scale)])
    hip.sync()
    return ctx.numpy(), dk.numpy(), dv.numpy()


@pytest.mark.parametrize("use_pos,table", [(False, True), (True, True), (True, False)])
def test_static_workspace_is_the_workspace_entry_point_twice_in_a_row(gpu, use_pos, table):
    rng = np.random.default_rng(17)
    # the second call is smaller: fewer keys, fewer chunks, a smaller cache
    for past, cap in ((1000, 1200), (70, 100)):
        print(f"static attention past={past} cap={cap} pos={use_pos} table={table}", flush=True)
        qkv = rng.standard_normal((1, (HEADS + 2 * KV) * D)).astype(np.float32)
        kc = rng.standard_normal((KV, cap, D)).astype(np.float32)
        vc = rng.standard_normal((KV, cap, D)).astype(np.float32)
        want = attend("nc_attention_decode", qkv, kc, vc, past, use_pos, table)
        got = attend("nc_attention_decode_static", qkv, kc, vc, past, use_pos, table)
        for a, b in zip(got, want):
            assert np.array_equal(bits(a), bits(b)), (past, cap)


def test_static_workspace_rejects_problems_beyond_it(gpu):
    """64 heads over 16384 keys need 4.3 MB of chunk results: refused before any launch."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray, KernelError
    from nanocompile_amd.kernels import float_bits
    heads, kv, cap = 64, 2, 16384
    qkv = DeviceArray(((heads + 2 * kv) * D,), np.float32)
    kc = DeviceArray((kv, cap, D), np.float32)
    inv = DeviceArray((D // 2,), np.float32)
    ctx = DeviceArray((heads * D,), np.float32)
    with pytest.raises(KernelError, match="1 MiB workspace"):
        hip.call("nc_attention_decode_static", [ctx, qkv, kc, kc, inv, None, None],
                 [heads, kv, D, cap - 1, cap, float_bits(0.125)])
    hip.sync()
