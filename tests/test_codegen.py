"""The loop-IR -> HIP path on the CPU: schedules, indices, memory plans, the build cache.

The generated kernels run on a GPU (tests/test_codegen_gpu.py). Here:

* every recorded program (the reference's fused, unfused and CPU-scheduled
  forms of a zoo of graphs, and the tiny golden Qwen2), with the GPU's
  default schedules applied (weights packed, indices simplified), runs in a
  bounds-checked interpreter (tests/loopir_interp.py) and must give the
  reference C's recorded outputs, bitwise except exp/sin/cos (the
  reference's own tolerance); no load or store may leave its buffer;
* the runtime's arena layout never lets two buffers that are alive at the
  same time overlap, gives each buffer its full size, and keeps a call's
  output apart from its operands;
* each schedule primitive refuses what would change the kernel's meaning;
* the simplifier removes exactly the divisions it can prove;
* the library source is deterministic, a second build is a cache hit, and
  a hipcc failure is a CompileError.
"""

from __future__ import annotations

import numpy as np
import pytest

from nanocompile_amd import codegen_hip, compiled, gpu_schedule, lir, simplify
from tests import loopir_interp as I
from tests import programs as P

I64 = lir.DType("i64")


def v(name):
    return lir.Var(name)


def c(x):
    return lir.Const(x, I64)


def b(op, a, bb):
    return lir.Binary(op, a, bb, I64)


def close(name, got, want):
    for key in want:
        g, w = got[key], want[key]
        assert g.dtype == w.dtype and g.shape == w.shape, key
        if key in P.approx(name):
            np.testing.assert_allclose(g, w, rtol=P.RTOL, atol=P.ATOL)
        else:
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), f"{name}.{key}"


@pytest.mark.parametrize("variant", ["program", "unfused", "scheduled"])
@pytest.mark.parametrize("name", P.zoo_names())
def test_scheduled_kernels_compute_the_references_outputs(name, variant):
    program = P.zoo(name, variant)
    scheduled = I.schedules(program)
    cases, weights = P.zoo_cases(name)
    for inputs, want, error in cases:
        got = I.run(program, scheduled, inputs, weights, I.bind(program, inputs))
        if error is not None:
            assert isinstance(got, tuple) and got[0] == "fail" and got[2] == 1, got
        else:
            close(name, got, want)


def test_tiny_qwen2_vnni_through_the_interpreter_is_golden():
    golden = np.load(P.GOLDEN / "golden.npz")
    progs = {w: P.qwen2("vnni", w) for w in ("full", "last")}
    scheds = {w: I.schedules(p) for w, p in progs.items()}
    weights = P.qwen2_weights("vnni")

    def run(which, inputs):
        p = progs[which]
        return I.run(p, scheds[which], inputs, weights, I.bind(p, inputs))

    driver = P.Driver(run)
    assert driver.greedy(P.PROMPTS[0], 3) == list(golden["g5_vnni_tokens_0"][:3])


def all_programs():
    out = [(f"{n}/{v}", P.zoo(n, v)) for n in P.zoo_names() for v in ("program", "unfused", "scheduled")]
    doc, _ = P.fixture()
    for tag, entry in doc["qwen2"].items():
        for which in entry:
            if which != "weight_names":
                out.append((f"qwen2_{tag}/{which}", P.qwen2(tag, which)))
    return out


@pytest.mark.parametrize("seq,past", [(1, 0), (3, 5), (11, 0), (1, 40)])
def test_arena_layout_keeps_live_buffers_apart(seq, past):
    for key, program in all_programs():
        bound = {"seq": seq, "past": past}
        if not set(program.symbols) <= set(bound):
            continue
        last = program.last_uses()
        plan = compiled.plan_memory(program, last, bound)
        layout = compiled.call_layout(program, bound, plan)
        first = {}
        for index, call in enumerate(program.calls):
            first.setdefault(call.output, index)
        live = {}
        for buf, at in layout.offsets.items():
            assert layout.sizes[buf] >= compiled._nbytes(buf, bound), key
            assert 0 <= at and at + layout.sizes[buf] <= layout.bytes, key
            if buf.kind == "temp":
                live[buf] = (first[buf], last.get(buf, first[buf]))
            else:
                live[buf] = (0, len(program.calls))
        bufs = list(live)
        for i, x in enumerate(bufs):
            for y in bufs[i + 1:]:
                (a0, a1), (b0, b1) = live[x], live[y]
                if a0 <= b1 and b0 <= a1:                       # alive at some common call
                    xa, ya = layout.offsets[x], layout.offsets[y]
                    assert xa + layout.sizes[x] <= ya or ya + layout.sizes[y] <= xa, (key, x, y)
        assert plan.region_bytes <= plan.unshared_bytes


def test_grid_binds_only_the_outermost_independent_loops():
    program = P.zoo("rms_norm")
    kernel = program.kernels[0]
    s = gpu_schedule.GpuSchedule(kernel)
    with pytest.raises(gpu_schedule.ScheduleError, match="outermost"):
        s.grid("j0")
    with pytest.raises(gpu_schedule.ScheduleError, match="multiple of 64"):
        s.block(100)
    s.grid("i0")
    with pytest.raises(gpu_schedule.ScheduleError, match="no loop"):
        s.cooperate("zz")
    carried = lir.Kernel("row", kernel.params, (lir.Loop("i0", c(4), (lir.Assign("acc", c(1)),)),))
    with pytest.raises(gpu_schedule.ScheduleError, match="carries"):
        gpu_schedule.GpuSchedule(carried).grid("i0")


def test_cooperate_refuses_stores_before_the_shared_loop():
    params = (lir.Param(lir.DType("f32"), True), lir.Param(lir.DType("f32"), False))
    f32 = lir.DType("f32")
    body = (lir.Loop("i0", c(4), (lir.Store(0, v("i0"), lir.Const(1.0, f32)),
                                  lir.Loop("j0", c(8), (lir.Store(0, b("add", v("i0"), v("j0")),
                                                                  lir.Load(1, v("j0"), f32)),)))),)
    s = gpu_schedule.GpuSchedule(lir.Kernel("row", params, body)).grid("i0")
    with pytest.raises(gpu_schedule.ScheduleError, match="store"):
        s.cooperate("j0")


def test_default_schedule_cooperates_on_row_kernels_and_packs_matmul_weights():
    rms = gpu_schedule.schedule_program(P.zoo("rms_norm"))
    assert rms[0][1].cooperate == "j0"
    q = P.qwen2("int8", "last")
    scheduled = gpu_schedule.schedule_program(q)
    packed = [k.primitive for k, _ in scheduled if any(p.packed for p in k.params)]
    assert packed and all(p.startswith("matmul") for p in packed)
    vnni = gpu_schedule.schedule_program(P.qwen2("vnni", "last"))
    for kernel, _ in vnni:                       # Dp4 reads four consecutive bytes: never packed
        if "vnni" in kernel.primitive:
            assert not any(p.packed for p in kernel.params)


def test_pack_refuses_operands_a_dp4_reads():
    program = P.zoo("mlp_int8-vnni_64")
    kernel = next(k for k in program.kernels if "vnni" in k.primitive)
    weight = next(x.a.param for x in gpu_schedule.scalars(kernel.body) if type(x).__name__ == "Dp4")
    with pytest.raises(gpu_schedule.ScheduleError, match="Dp4"):
        gpu_schedule.GpuSchedule(kernel).pack(weight, 64, 32)


def test_simplifier_removes_provable_divisions_only():
    ranges = {"i": (0, 255), "k": (0, 127)}
    flat = b("add", b("mul", v("i"), c(128)), v("k"))
    assert simplify.simplify(b("idiv", flat, c(128)), ranges) == v("i")
    assert simplify.simplify(b("mod", flat, c(128)), ranges) == v("k")
    wide = {"i": (0, 255), "k": (0, 128)}                       # k may reach 128: not provable
    assert simplify.simplify(b("idiv", flat, c(128)), wide).op == "idiv"
    assert simplify.coefficient(flat, "i") == 128 and simplify.coefficient(flat, "k") == 1
    assert simplify.coefficient(b("mul", v("i"), v("k")), "i") is None


def test_pack_rows_is_the_packed_parameter_layout():
    rng = np.random.default_rng(0)
    w = rng.integers(-127, 128, (100, 7)).astype(np.int8)
    packed = compiled.pack_rows(w, 64).reshape(-1)
    assert packed.size == 128 * 7
    for r, col in [(0, 0), (63, 6), (64, 0), (99, 3)]:
        assert packed[(r // 64) * 7 * 64 + col * 64 + r % 64] == w[r, col]


def test_library_source_is_deterministic_and_every_kernel_has_a_launcher():
    program = P.qwen2("int8", "last")
    first = codegen_hip.render_library(gpu_schedule.schedule_program(program))
    again = codegen_hip.render_library(gpu_schedule.schedule_program(P.qwen2("int8", "last")))
    assert first == again
    for i in range(len(program.kernels)):
        assert f"NC_EXPORT int32_t nc_k{i}(void **p, const int64_t *s)" in first
    assert "nc_bind_stream" in first


def test_build_cache_hits_and_compile_errors(tmp_path, monkeypatch):
    monkeypatch.setenv("NANOCOMPILE_AMD_CACHE", str(tmp_path))
    source = codegen_hip.render_library(gpu_schedule.schedule_program(P.zoo("binary_i8")))
    path, cached = codegen_hip.build_library(source)
    assert not cached and path.exists() and path.parent == tmp_path
    assert codegen_hip.build_library(source) == (path, True)
    assert [p.name for p in tmp_path.iterdir() if p.is_dir()] == []          # no scratch left behind
    with pytest.raises(codegen_hip.CompileError, match="hipcc failed"):
        codegen_hip.build_library(source + "\nthis is not C++;\n")


def test_json_programs_read_back_whole():
    program = P.qwen2("vnni", "full")
    assert program.symbols == ("seq", "past")
    assert [n for n, _, _ in program.inputs] == ["token_ids", "past_keys", "past_values"]
    assert set(program.outputs) == {"logits", "keys", "values"}
    assert len(program.calls) == 81 and len(program.kernels) == 33
    gathers = [call for call in program.calls if call.gather]
    assert gathers and gathers[0].gather["ids_input"] == "token_ids"
    assert lir.evaluate(program.calls[0].operands[0].shape[0], {"seq": 5, "past": 2}) == 5
