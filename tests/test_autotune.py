"""The GPU autotuner's host logic: the schedule table, the choice rule, the cache.

No GPU needed: nc_schedule_info is a table lookup in the library, and the
choice rule is tested with recorded costs (the reference tests its search the
same way, replaying costs: autotune.py:450-470).
"""

from __future__ import annotations

import json

import pytest

from nanocompile_amd import autotune, hip, kernels


@pytest.fixture(scope="module")
def library():
    try:
        return hip.load()
    except hip.LibraryMissing:
        pytest.skip("the HIP library is not built")


def test_schedule_table_matches_the_kernels(library):
    assert hip.schedule_info(0) is None and hip.schedule_info(8) is None and hip.schedule_info(25) is None
    gemv = [hip.schedule_info(s) for s in kernels.GEMV_SCHEDULES]
    assert all(g["kernel"] == "gemv" and g["load_bytes"] == 16 for g in gemv)
    assert {(g["lanes_per_row"], g["waves"]) for g in gemv} == {(4, 1), (16, 1), (8, 2), (8, 4), (4, 2), (16, 2), (8, 1)}
    assert hip.schedule_info(7)["lanes_per_row"] == 8 and hip.schedule_info(7)["waves"] == 1
    tiles = [hip.schedule_info(s) for s in kernels.GEMM_SCHEDULES]
    for t in tiles:
        assert t["kernel"] == "mfma"
        assert t["tile_m"] % t["wave_m"] == 0 and t["tile_n"] % t["wave_n"] == 0
        assert t["wave_m"] % 16 == 0 and t["wave_n"] % 16 == 0 and t["k_stage"] % 64 == 0
        assert t["threads"] == (t["tile_m"] // t["wave_m"]) * (t["tile_n"] // t["wave_n"]) * 64
        # two unpadded buffers of BM activation rows and one (or the SwiGLU pair's two) BN weight rows
        assert t["lds_bytes"] == 2 * (t["tile_m"] + t["tile_n"]) * t["k_stage"] <= 160 * 1024
        assert t["lds_bytes_pair"] == 2 * (t["tile_m"] + 2 * t["tile_n"]) * t["k_stage"] <= 160 * 1024
        assert t["stages"] >= 2 and t["stages"] % 2 == 0
    first = tiles[0]
    assert (first["tile_m"], first["tile_n"], first["k_stage"], first["stages"], first["lds_bytes"]) == \
        (64, 64, 128, 4, 32768)
    assert len({tuple(sorted(t.items())[1:]) for t in tiles}) == len(tiles)     # no duplicate tiles


def test_legal_space(library):
    space = autotune.legal_space("matmul_i8_token", 512, 896, 896)
    assert space[0] == {"schedule": 0, "kernel": "default"}
    assert [c["schedule"] for c in space[1:]] == list(kernels.GEMV_SCHEDULES) + list(kernels.GEMM_SCHEDULES)
    ragged = autotune.legal_space("matmul_i8_token", 3, 40, 77)
    assert all(c["kernel"] != "mfma" for c in ragged)                  # MFMA tiles need K % 16 == 0
    swiglu = autotune.legal_space("matmul_i8_token_swiglu", 64, 4864, 896)
    assert [c["schedule"] for c in swiglu[:2]] == [0, 7]
    with pytest.raises(ValueError):
        autotune.legal_space("matmul_i8", 1, 1, 1)


def test_choose_keeps_the_incumbent_inside_the_margin():
    recorded = {0: 10.0, 7: 12.0, 16: 9.8, 17: 11.0}

    def cost(stage, schedules):
        return [recorded[s] for s in schedules]

    winner, log, default_cost, winner_cost = autotune.choose([0, 7, 16, 17], cost, margin=0.03)
    assert winner == 0 and default_cost == winner_cost == 10.0          # 2% faster is not enough
    assert [e.stage for e in log] == ["sample", "confirm"]
    recorded[16] = 9.0
    winner, log, default_cost, winner_cost = autotune.choose([0, 7, 16, 17], cost, margin=0.03)
    assert (winner, default_cost, winner_cost) == (16, 10.0, 9.0)


def test_choose_confirms_with_its_own_measurement():
    """A candidate that won the sample but loses the confirmation is not chosen."""
    def cost(stage, schedules):
        table = {0: 10.0, 16: 8.0} if stage == "sample" else {0: 10.0, 16: 9.9}
        return [table[s] for s in schedules]

    winner, log, _, _ = autotune.choose([0, 16], cost, margin=0.03)
    assert winner == 0 and log[1].costs == [10.0, 9.9]


def test_choose_stops_when_the_incumbent_is_best():
    winner, log, d, w = autotune.choose([0, 16], lambda stage, s: [1.0, 2.0][: len(s)], margin=0.03)
    assert winner == 0 and len(log) == 1 and d == w == 1.0


def test_cache_log_roundtrip_versions_and_damage(tmp_path):
    """The cache is a log of JSON lines: the newest answer for (machine, key) wins, lines of
    another version and damaged lines are skipped, and an answer appended after a torn line
    still reads back."""
    path = tmp_path / "sub" / "tuning.jsonl"
    cache = autotune.TuningCache(path)
    assert cache.get("m", "k") is None
    cache.put("m", "k", {"winner": 17})
    cache.put("m", "k2", {"winner": 0})
    cache.put("other", "k", {"winner": 5})
    assert cache.get("m", "k") == {"winner": 17} and cache.get("other", "k") == {"winner": 5}
    cache.put("m", "k", {"winner": 16})                         # a newer answer replaces it
    assert cache.get("m", "k") == {"winner": 16} and cache.get("m", "k2") == {"winner": 0}
    assert len(path.read_text().splitlines()) == 4 and list(path.parent.iterdir()) == [path]
    with open(path, "a") as f:
        f.write(json.dumps({"v": autotune.CACHE_VERSION + 1, "machine": "m", "key": "k",
                            "entry": {"winner": 9}}) + "\n")   # another version: ignored
        f.write("[1, 2]\n{not json\n" + '{"v": 1, "machine": "m", "key": "k", "entry": 4}\n')
    assert cache.get("m", "k") == {"winner": 16}
    with open(path, "ab") as f:
        f.write(b'{"v": 1, "machine": "m", "key": "k", "ent')      # a write cut short
    assert cache.get("m", "k") == {"winner": 16}
    cache.put("m", "k", {"winner": 3})
    assert cache.get("m", "k") == {"winner": 3}
    path.write_bytes(b"\xff\xfe\x00")                          # not text at all
    assert cache.get("m", "k") is None
    cache.put("m", "k", {"winner": 2})
    assert cache.get("m", "k") == {"winner": 2}


def test_records_report_costs_and_speedup():
    r = autotune.TuneRecord("key", "op", (1, 2, 3), 5, 3, (2.0, 1.0))
    assert (r.default_cost, r.winner_cost, r.speedup) == (2.0, 1.0, 2.0)
    assert autotune.TuneRecord("key", "op", (), 1).speedup is None


def test_guard_regions_catch_writes_outside_the_output():
    """A candidate's output sits between sentinel guards; any write outside it is reported."""
    import numpy as np
    words = 100
    bits = autotune.guarded(words)
    assert autotune.guards_broken(bits) == []
    bits[autotune.GUARD:autotune.GUARD + words] = 7             # the output itself may hold anything
    assert autotune.guards_broken(bits) == []
    bits[autotune.GUARD - 1] = 0                                # one word before
    bits[autotune.GUARD + words + 2] = np.uint32(0x3F800000)    # three words after the last
    assert autotune.guards_broken(bits) == [-1, words + 2]


def test_problem_key_covers_shape_and_space():
    space = [{"schedule": 0, "kernel": "default"}]
    k1 = autotune.Autotuner.problem_key("matmul_i8_token", 512, 896, 896, space)
    assert k1 == autotune.Autotuner.problem_key("matmul_i8_token", 512, 896, 896, list(space))
    assert k1 != autotune.Autotuner.problem_key("matmul_i8_token", 128, 896, 896, space)
    assert k1 != autotune.Autotuner.problem_key("matmul_i8_token", 512, 896, 896, space + [{"schedule": 16}])


def test_decode_and_attention_schedule_tables(library):
    """The decode projections' (lanes a row, waves, bytes a load) and prefill attention's rows a
    workgroup: what the tuner searches, read from the library (no GPU)."""
    assert hip.decode_schedule_info(896, 0, 1) == {"lanes_per_row": 8, "waves": 1, "load_bytes": 16}
    assert hip.decode_schedule_info(4864, 1, 1) == {"lanes_per_row": 64, "waves": 4, "load_bytes": 4}
    for kind in (0, 2):                          # an rms_norm prologue takes 1 or 4 waves
        assert all(hip.decode_schedule_info(896, kind, s)["waves"] in (1, 4)
                   for s in range(1, 6) if hip.decode_schedule_info(896, kind, s))
    assert hip.decode_schedule_info(4864, 1, 4)["waves"] == 2
    assert hip.decode_schedule_info(4864, 0, 1) is None and hip.decode_schedule_info(896, 1, 6) is None
    assert hip.decode_schedule_info(896, 1, 0) is None
    for s in range(1, 6):
        shape = hip.decode_schedule_info(896, 1, s)
        assert 896 % (shape["lanes_per_row"] * shape["load_bytes"]) == 0
    assert [hip.attention_schedule_info(s) for s in range(6)] == [None, 2, 4, 8, 16, None]
