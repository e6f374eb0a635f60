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


def test_default_schedule_leads_row_kernels_and_spreads_int8_chains_over_lanes():
    """The defaults are what the tuner chose on the reference's programs: a row kernel's
    reductions in one lead wave; an int8 projection's 32 chains one a lane over row-major
    weights; a float matmul's weights packed; a reduction over the context (P.V) a workgroup."""
    rms = gpu_schedule.schedule_program(P.zoo("rms_norm"))
    assert rms[0][1].cooperate == "j0" and rms[0][1].lead
    q = P.qwen2("int8", "last")
    scheduled = gpu_schedule.schedule_program(q)
    int8 = [(k, l) for k, l in scheduled if k.primitive.startswith("matmul_i8")]
    assert int8 and all(l.lanes is not None and not any(p.packed for p in k.params) for k, l in int8)
    packed = [k.primitive for k, _ in scheduled if any(p.packed for p in k.params)]
    assert packed and all(p == "matmul" for p in packed)
    assert any(l.workgroup and l.lead for k, l in scheduled if k.primitive == "matmul")
    vnni = gpu_schedule.schedule_program(P.qwen2("vnni", "last"))
    for kernel, _ in vnni:                       # Dp4 reads four consecutive bytes: never packed
        if "vnni" in kernel.primitive:
            assert not any(p.packed for p in kernel.params)
    for i, kernel in enumerate(q.kernels):       # every default is a point of its class's space
        config = gpu_schedule.default_config(kernel, [c for c in q.calls if c.kernel == i])
        assert config in gpu_schedule.space(kernel)


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


# -- the schedule space: LDS staging, workgroup items, vector width ------------------------------


def _calls_of(program):
    out = {}
    for call in program.calls:
        out.setdefault(call.kernel, []).append(call)
    return out


def _staged_everywhere(program):
    """Each kernel with its operands staged where it can be (a row kernel's serial reads, or an
    item kernel as a workgroup), else the default; and how many were staged."""
    calls, out, staged = _calls_of(program), [], 0
    for i, kernel in enumerate(program.kernels):
        cls = gpu_schedule.kernel_class(kernel)
        config = dict(gpu_schedule.DEFAULTS[cls])
        config.update({"row": {"stage": True, "vector": 4}, "item": {"workgroup": True}}.get(cls, {}))
        try:
            out.append(gpu_schedule.apply(kernel, calls.get(i, []), config))
            staged += 1
        except gpu_schedule.ScheduleError:
            out.append(gpu_schedule.default(kernel, calls.get(i, [])))
    return out, staged


@pytest.mark.parametrize("variant", ["program", "unfused", "scheduled"])
@pytest.mark.parametrize("name", P.zoo_names())
def test_staged_kernels_compute_the_references_outputs(name, variant):
    """Staging rewrites reads to LDS windows: run with each window copied first (every copy read
    bounds-checked), the program still gives the reference C's outputs."""
    program = P.zoo(name, variant)
    scheduled, _ = _staged_everywhere(program)
    cases, weights = P.zoo_cases(name)
    for inputs, want, error in cases:
        got = I.run(program, scheduled, inputs, weights, I.bind(program, inputs))
        if error is not None:
            assert isinstance(got, tuple) and got[0] == "fail" and got[2] == 1, got
        else:
            close(name, got, want)


def test_staging_reaches_the_row_and_reduction_kernels():
    scheduled, staged = _staged_everywhere(P.zoo("rms_norm_quant"))
    assert staged == 2
    row, reduce = scheduled[0][1], scheduled[1][1]
    assert row.cooperate == "j0" and [st.param for st in row.stage] == [1]       # x, not gamma (read once)
    assert reduce.workgroup and [st.param for st in reduce.stage] == [1]
    st = row.stage[0]
    assert st.extent == c(896) and simplify.coefficient(st.base, "i0") == 896
    reads = [x for x in gpu_schedule.scalars(scheduled[0][0].body) if type(x).__name__ in ("Load", "Local")]
    assert {(type(x).__name__, getattr(x, "param", getattr(x, "name", None))) for x in reads} == {
        ("Local", "nc_s1"), ("Load", 2)}
    plain, launch = gpu_schedule.unstage(*scheduled[0])
    assert launch.stage == () and not any(type(x).__name__ == "Local" for x in gpu_schedule.scalars(plain.body))


def test_hoisted_workgroup_item_stages_nothing_only_its_hoisted_pass_reads():
    """P.V as a workgroup item with a lead wave and hoisting: the probabilities are read once an
    element, in the pass every thread runs, so no window is copied to LDS first (a pass and a
    barrier fewer); without hoisting the lead wave rereads them and they are staged."""
    q = P.qwen2("int8", "last")
    calls = _calls_of(q)
    pv = next(i for i, k in enumerate(q.kernels)
              if k.primitive == "matmul" and gpu_schedule._reduces_over_run_time_extent(k))
    base = dict(gpu_schedule.DEFAULTS["item"], threads=128, workgroup=True, lead=True, unroll=16)
    kernel, launch = gpu_schedule.apply(q.kernels[pv], calls[pv], dict(base, hoist=True))
    assert launch.hoist and launch.stage == ()
    src = codegen_hip.render_kernel(kernel, launch, pv)
    body = src[:src.index("_unstaged")]
    # two barriers an item: after the products pass, and before the next item's pass overwrites them
    # (none before the pass: the lead wave hands it nothing)
    assert "nc_s1" not in body and body.count("__syncthreads();") == 2
    _, unhoisted = gpu_schedule.apply(q.kernels[pv], calls[pv], base)
    assert [st.param for st in unhoisted.stage] == [1]


def test_stage_refuses_what_would_read_past_the_window():
    program = P.zoo("rms_norm_quant")
    row, reduce, quant = program.kernels[0], program.kernels[1], program.kernels[3]
    with pytest.raises(gpu_schedule.ScheduleError, match="workgroup"):
        gpu_schedule.GpuSchedule(reduce).grid("i0").stage(1)               # a thread per item
    s = gpu_schedule.GpuSchedule(row).grid("i0").cooperate("j0")
    with pytest.raises(gpu_schedule.ScheduleError, match="not an operand"):
        s.stage(0)
    s.stage(1)
    with pytest.raises(gpu_schedule.ScheduleError, match="already"):
        s.stage(1)
    # x2[i0], a per-row scale, is read at no loop index of the item
    with pytest.raises(gpu_schedule.ScheduleError, match="loop indices|does not read"):
        gpu_schedule.GpuSchedule(quant).grid("i0").workgroup().stage(2)
    f32 = lir.DType("f32")
    params = (lir.Param(f32, True), lir.Param(f32, False))
    # the only read sits in the untaken arm of a select: the unscheduled kernel may read nothing
    lazy = lir.Kernel("row", params, (lir.Loop("i0", c(4), (
        lir.Let("acc", lir.Const(0.0, f32)),
        lir.Loop("r", c(8), (lir.Assign("acc", lir.Select(lir.Binary("lt", v("r"), c(0), lir.DType("bool")),
                                                          lir.Load(1, b("add", b("mul", v("i0"), c(8)), v("r")), f32),
                                                          lir.Var("acc", f32), f32)),)),
        lir.Store(0, v("i0"), lir.Var("acc", f32)))),))
    s = gpu_schedule.GpuSchedule(lazy).grid("i0").workgroup()
    with pytest.raises(gpu_schedule.ScheduleError, match="whole window"):
        s.stage(1)
    # two windows of one operand
    two = lir.Kernel("row", params, (lir.Loop("i0", c(4), (
        lir.Let("acc", lir.Const(0.0, f32)),
        lir.Loop("r", c(8), (lir.Assign("acc", lir.Binary("add", lir.Load(1, v("r"), f32),
                                                          lir.Load(1, b("add", v("r"), c(8)), f32), f32)),)),
        lir.Store(0, v("i0"), lir.Var("acc", f32)))),))
    with pytest.raises(gpu_schedule.ScheduleError, match="more than one window"):
        gpu_schedule.GpuSchedule(two).grid("i0").workgroup().stage(1)


def test_workgroup_and_vectorize_compose_only_where_they_mean_something():
    program = P.zoo("rms_norm_quant")
    row, reduce = program.kernels[0], program.kernels[1]
    with pytest.raises(gpu_schedule.ScheduleError, match="shares a loop"):
        gpu_schedule.GpuSchedule(row).grid("i0").cooperate("j0").workgroup()
    with pytest.raises(gpu_schedule.ScheduleError, match="vectorized"):
        gpu_schedule.GpuSchedule(reduce).grid("i0").vectorize(4).workgroup()
    with pytest.raises(gpu_schedule.ScheduleError, match="spreads no loop"):
        gpu_schedule.GpuSchedule(reduce).grid("i0").workgroup().vectorize(4)
    with pytest.raises(gpu_schedule.ScheduleError, match="one of"):
        gpu_schedule.GpuSchedule(reduce).grid("i0").vectorize(3)


def test_space_starts_at_the_default_and_refuses_points_outside_it():
    program = P.zoo("rms_norm_quant")
    calls = _calls_of(program)
    for i, kernel in enumerate(program.kernels):
        cls = gpu_schedule.kernel_class(kernel)
        points = gpu_schedule.space(kernel)
        assert points[0] == gpu_schedule.DEFAULTS[cls]
        assert len({gpu_schedule.canonical(p) for p in points}) == len(points)
        chosen = gpu_schedule.default_config(kernel, calls[i])
        assert chosen in points
        assert gpu_schedule.apply(kernel, calls[i], chosen) == gpu_schedule.default(kernel, calls[i])
    row = program.kernels[0]
    assert gpu_schedule.kernel_class(row) == "row"
    with pytest.raises(gpu_schedule.ScheduleError, match="not a point"):
        gpu_schedule.apply(row, calls[0], {"threads": 96, "stage": False, "vector": 1, "unroll": 0})
    with pytest.raises(gpu_schedule.ScheduleError, match="not a point"):
        gpu_schedule.apply(row, calls[0], {"threads": 256, "workgroup": True, "vector": 1, "unroll": 0})
    elementwise = program.kernels[2]
    with pytest.raises(gpu_schedule.ScheduleError, match="unroll"):
        gpu_schedule.apply(elementwise, calls[2], dict(gpu_schedule.DEFAULTS["item"], unroll=4))


def test_candidate_library_holds_each_distinct_kernel_once_and_reports_failures_as_its_kernel():
    from nanocompile_amd import autotune
    program = P.zoo("gather")
    library = autotune.CandidateLibrary(program)
    entries = [n for per in library.entry for n in per]
    assert entries == list(range(len(entries)))
    for i, cands in enumerate(library.candidates):
        assert cands[0].config == gpu_schedule.default_config(program.kernels[i], library.calls_of.get(i, []))
        assert len({c.source for c in cands}) == len(cands)
        for n in library.entry[i]:
            assert f"NC_EXPORT int32_t nc_k{n}(void **p, const int64_t *s)" in library.source
    gather = next(i for i, k in enumerate(program.kernels) if k.primitive == "gather")
    codes = {int(x) for x in __import__("re").findall(r"nc_fail\(nc_err, (\d+)\)", library.source)}
    assert codes and all((code >> 8) - 1 == gather for code in codes)
    scheduled, source, names = library.choice([len(c) - 1 for c in library.candidates])
    assert source == library.source and names == [f"nc_k{per[-1]}" for per in library.entry]


def test_vectorized_items_are_unrolled_without_checks_only_when_whole():
    program = P.zoo("rms_norm_quant")
    calls = _calls_of(program)
    kernel, launch = gpu_schedule.apply(program.kernels[3], calls[3],
                                        dict(gpu_schedule.DEFAULTS["item"], threads=64, vector=4))
    text = codegen_hip.render_kernel(kernel, launch, 3)
    assert "const int64_t nc_q1 = (nc_e1 + 3) / 4;" in text
    assert "if (nc_i1 * 4 + 4 <= nc_e1) {" in text and "#pragma unroll" in text
    assert text.count("const int64_t nc_items = nc_e0 * nc_q1;") == 2          # kernel and launcher agree
    row, rl = gpu_schedule.apply(program.kernels[0], calls[0], dict(gpu_schedule.DEFAULTS["row"], threads=128,
                                                                      stage=True, vector=2, unroll=4))
    text = codegen_hip.render_kernel(row, rl, 0)
    assert "extern __shared__" in text and text.count("__syncthreads();") == 2      # after the copy, after the item
    assert "nc_g0_unstaged" in text and f"if (nc_lds > {gpu_schedule.MAX_STAGE_BYTES})" in text
    # the serial loop, unrolled by 4: batches of 4 staged values read ahead of the sum's chain
    assert "for (int64_t nc_base = 0; nc_base < 896; nc_base += 4) {" in text
    assert "nc_pf1_0[nc_u] = nc_s1[r];" in text and "float t1 = (nc_pf1_0[nc_u] * nc_pf1_0[nc_u]);" in text


def test_lead_shares_the_serial_parts_values_and_refuses_a_failing_serial_part():
    program = P.zoo("rms_norm_quant")
    calls = _calls_of(program)
    row, rl = gpu_schedule.apply(program.kernels[0], calls[0], dict(gpu_schedule.DEFAULTS["row"], lead=True))
    body = gpu_schedule.perfect_nest(row.body)[0].body
    assert [name for name, _ in gpu_schedule.live_ins(body[:-1], body[-1])] == ["acc0"]
    text = codegen_hip.render_kernel(row, rl, 0)
    assert "__shared__ float nc_lead_f32[1];" in text and "const float acc0 = nc_lead_f32[0];" in text
    assert text.count("__syncthreads();") == 2                   # after the lead wave, after the item
    with pytest.raises(gpu_schedule.ScheduleError, match="workgroup"):
        gpu_schedule.GpuSchedule(program.kernels[1]).grid("i0").lead()
    gather = P.zoo("gather")
    k = next(k for k in gather.kernels if k.primitive == "gather")
    s = gpu_schedule.GpuSchedule(k)
    s.grid(*gpu_schedule.grid_loops(k)[:1])
    if gpu_schedule.shared_loop(k, s.launch.grid):
        s.cooperate(gpu_schedule.shared_loop(k, s.launch.grid))
    else:
        s.workgroup()
    with pytest.raises(gpu_schedule.ScheduleError, match="stop one wave"):
        s.lead()


def test_every_candidate_packs_only_what_the_default_packs():
    """The tuner runs every candidate on the default's arguments: an operand the default reads
    packed may be read row-major by a candidate (its row-major copy is resident too), never the
    other way round."""
    from nanocompile_amd import autotune
    packed = unpacked = 0
    for program in (P.qwen2("int8", "full"), P.zoo("mlp_int8_64"), P.zoo("linear")):
        library = autotune.CandidateLibrary(program)
        for cands in library.candidates:
            default = [p.packed for p in cands[0].kernel.params]
            packed += any(default)
            for cand in cands[1:]:
                mine = [p.packed for p in cand.kernel.params]
                assert all(m is None or m == d for m, d in zip(mine, default))
                unpacked += any(d and not m for m, d in zip(mine, default))
    assert packed and unpacked


# -- staging legality as a property: refused, or it reads nothing the kernel would not -----------

_FORMS = ("v", "v+3", "2v", "rev")     # offset of a read within the row, as a function of the loop index


def _offset(form: str, var, extent: int):
    """The lir index offset of ``form`` over loop var ``var`` (extent ``extent``)."""
    x = v(var)
    return {"v": x, "v+3": b("add", x, c(3)), "2v": b("mul", x, c(2)),
            "rev": b("sub", c(extent - 1), x)}[form]


def _reads(form: str, extent: int) -> list[int]:
    return [{"v": k, "v+3": k + 3, "2v": 2 * k, "rev": extent - 1 - k}[form] for k in range(extent)]


from hypothesis import given, settings, strategies as hst  # noqa: E402


@hst.composite
def _row_kernels(draw):
    rows = draw(hst.integers(1, 3))
    e = draw(hst.integers(1, 9))
    e2 = draw(hst.sampled_from([e, e + 2]))
    serial = draw(hst.sampled_from(_FORMS))
    shared = draw(hst.sampled_from(_FORMS + ("none",)))
    lazy = draw(hst.booleans())              # the serial read only in a select's untaken arm
    cooperate = draw(hst.booleans())
    return rows, e, e2, serial, shared, lazy, cooperate


@settings(max_examples=150, deadline=None)
@given(_row_kernels())
def test_staging_is_refused_or_reads_only_what_the_kernel_reads(case):
    rows, e, e2, serial, shared, lazy, cooperate = case
    f32, boolean = lir.DType("f32"), lir.DType("bool")
    stride = 2 * max(e, e2) + 4                   # a row of x1 holds every offset any form reads
    base = b("mul", v("i0"), c(stride))
    read = lir.Load(1, b("add", base, _offset(serial, "r", e)), f32)
    acc = lir.Var("acc", f32)
    step = lir.Binary("add", acc, read, f32)
    if lazy:
        step = lir.Select(lir.Binary("lt", v("r"), c(0), boolean), step, acc, f32)
    body = [lir.Let("acc", lir.Const(0.0, f32)), lir.Loop("r", c(e), (lir.Assign("acc", step),))]
    if cooperate:
        value = acc if shared == "none" else lir.Binary(
            "mul", acc, lir.Load(1, b("add", base, _offset(shared, "j0", e2)), f32), f32)
        body.append(lir.Loop("j0", c(e2), (lir.Store(0, b("add", b("mul", v("i0"), c(e2)), v("j0")), value),)))
        out_size = rows * e2
    else:
        body.append(lir.Store(0, v("i0"), acc))
        out_size = rows
    params = (lir.Param(f32, True), lir.Param(f32, False))
    kernel = lir.Kernel("row", params, (lir.Loop("i0", c(rows), tuple(body)),))
    offsets = ([] if lazy else _reads(serial, e)) + (_reads(shared, e2) if cooperate and shared != "none" else [])
    size = (rows - 1) * stride + max(offsets) + 1 if offsets else 1
    x1 = np.random.default_rng(rows * 100 + e).standard_normal(size).astype(np.float32)
    want = np.full(out_size, np.nan, np.float32)
    assert I.compile_kernel(kernel)([want, x1], []) == 0          # the kernel itself stays in bounds

    s = gpu_schedule.GpuSchedule(kernel).grid("i0")
    s.cooperate("j0") if cooperate else s.workgroup()
    try:
        s.stage(1)
    except gpu_schedule.ScheduleError:
        must = (not lazy and serial in ("v", "v+3") and
                (not cooperate or shared == "none" or (shared == serial and e2 == e)))
        assert not must, f"refused a legal window: {case}"
        return
    staged, launch = s.done()
    got = np.full(out_size, np.nan, np.float32)
    assert I.compile_kernel(I.staged_ir(staged, launch))([got, x1], []) == 0   # OutOfBounds would raise
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case


# -- accumulators across lanes ----------------------------------------------------------------


def test_lanes_spread_the_references_accumulators_one_element_a_lane():
    """The int8 matmuls' 32 accumulator chains (quantize.py's recipe: element kc * 8 + kl) go one
    a lane; each lane's digits give back its own element, every element once."""
    found = 0
    for name in ("mlp_int8_64", "mlp_int8-vnni_64"):
        program = P.zoo(name)
        calls = _calls_of(program)
        for i, kernel in enumerate(program.kernels):
            if gpu_schedule.kernel_class(kernel) != "item":
                continue
            config = dict(gpu_schedule.DEFAULTS["item"], lanes=True)
            try:
                scheduled, launch = gpu_schedule.apply(kernel, calls[i], config)
            except gpu_schedule.ScheduleError:
                continue
            lanes = launch.lanes
            found += 1
            elements = []
            for lane in range(lanes.width):
                digits = {var: (lane // coeff) % extent for var, extent, coeff in lanes.loops}
                elements.append(simplify.value_range(lanes.index, {v: (d, d) for v, d in digits.items()})[0])
            assert elements == list(range(lanes.width)), (name, i)
            text = codegen_hip.render_kernel(scheduled, launch, i)
            assert f"const int nc_l = threadIdx.x & {lanes.width - 1};" in text
            assert "__shfl(" in text and "if (nc_l == 0) x0[" in text
            # four consecutive elements a lane: lane l's j-th is element 4 l + j, as the renderer
            # computes its digits (the others from 4 l, the unit digit 4 l % extent + j)
            four, fl = gpu_schedule.apply(kernel, calls[i], dict(config, lanes=4))
            assert fl.lanes.lanes == lanes.width // 4
            elements = []
            for lane in range(fl.lanes.lanes):
                for j in range(4):
                    digits = {var: ((lane * 4) // coeff) % extent if coeff != 1 else (lane * 4) % extent + j
                              for var, extent, coeff in fl.lanes.loops}
                    elements.append(simplify.value_range(fl.lanes.index, {v: (d, d) for v, d in digits.items()})[0])
            assert elements == list(range(lanes.width)), (name, i)
            assert "acc_0_l[nc_j] = " in codegen_hip.render_kernel(four, fl, i)
    assert found


def test_lanes_refuses_chains_that_are_not_independent():
    f32 = lir.DType("f32")
    params = (lir.Param(f32, True), lir.Param(f32, False))

    def kernel(index, extra=()):
        chain = lir.Loop("k0", c(4), (lir.Loop("kl", c(8), (lir.ArrayStore("acc", index, lir.Fma(
            lir.Load(1, b("add", b("mul", v("k0"), c(8)), v("kl")), f32), lir.Const(2.0, f32),
            lir.Local("acc", index, f32), f32)),) + tuple(extra)),))
        tail = lir.Store(0, v("i0"), lir.Local("acc", c(0), f32))
        return lir.Kernel("matmul", params, (lir.Loop("i0", c(3), (
            lir.Array("acc", 8, lir.Const(0.0, f32)), chain, tail)),))

    s = gpu_schedule.GpuSchedule(kernel(v("kl"))).grid("i0")
    assert s.lanes("acc").launch.lanes.width == 8
    with pytest.raises(gpu_schedule.ScheduleError, match="enumerate"):
        gpu_schedule.GpuSchedule(kernel(b("mul", v("kl"), c(2)))).grid("i0").lanes("acc")
    with pytest.raises(gpu_schedule.ScheduleError, match="more than update"):
        gpu_schedule.GpuSchedule(kernel(v("kl"), (lir.Store(0, v("kl"), lir.Const(1.0, f32)),))).grid("i0").lanes("acc")
    with pytest.raises(gpu_schedule.ScheduleError, match="no array"):
        gpu_schedule.GpuSchedule(kernel(v("kl"))).grid("i0").lanes("h")
    with pytest.raises(gpu_schedule.ScheduleError, match="vectorized|thread"):
        gpu_schedule.GpuSchedule(kernel(v("kl"))).grid("i0").vectorize(2).lanes("acc")


def test_hoist_computes_the_chains_operands_first_and_refuses_what_depends_on_the_chain():
    program = P.zoo("softmax_mask")
    calls = _calls_of(program)
    row = program.kernels[0]
    scheduled, launch = gpu_schedule.apply(row, calls[0], dict(gpu_schedule.DEFAULTS["row"], stage=True, lead=True,
                                                               hoist=True))
    assert [h.name for h in launch.hoist] == ["nc_h0", "nc_h1"]             # the max, then the sum of exps
    text = codegen_hip.render_kernel(scheduled, launch, 0)
    assert "nc_h1[r] = t" in text and "acc1 = (acc1 + nc_h1[r]);" in text
    assert "nc_g0_unstaged" in text                                    # the fallback when LDS is short
    # unrolled by 64, the lead wave's chain over the stored values reads them in batches ahead of
    # it (the context's length set at run time: whole batches, then one whose reads repeat the
    # last position and whose steps stop at the length)
    import re
    scheduled, launch = gpu_schedule.apply(row, calls[0], dict(gpu_schedule.DEFAULTS["row"], stage=True, lead=True,
                                                               hoist=True, unroll=64))
    text = codegen_hip.render_kernel(scheduled, launch, 0)
    batch = re.search(r"(nc_pf\d+_0)\[nc_u\] = nc_h1\[r\];", text)
    assert batch and f"acc1 = (acc1 + {batch.group(1)}[nc_u]);" in text
    assert text.index(batch.group(0)) < text.index(f"acc1 = (acc1 + {batch.group(1)}[nc_u]);")
    assert re.search(r"const int64_t r = nc_last \+ nc_u < (nc_n\d+) \? nc_last \+ nc_u : \1 - 1;", text)
    with pytest.raises(gpu_schedule.ScheduleError, match="lead"):
        gpu_schedule.GpuSchedule(row).grid("i0", "i1").cooperate("j0").hoist()
    f32 = lir.DType("f32")
    params = (lir.Param(f32, True), lir.Param(f32, False))
    acc = lir.Var("acc", f32)

    def kernel(lets, update):
        return lir.Kernel("row", params, (lir.Loop("i0", c(2), (
            lir.Let("acc", lir.Const(0.0, f32)), lir.Loop("r", c(8), tuple(lets) + (lir.Assign("acc", update),)),
            lir.Store(0, v("i0"), acc))),))

    x = lir.Load(1, b("add", b("mul", v("i0"), c(8)), v("r")), f32)
    ok = kernel([lir.Let("t", x)], lir.Binary("add", acc, lir.Var("t", f32), f32))
    assert gpu_schedule.GpuSchedule(ok).grid("i0").workgroup().lead().hoist().launch.hoist[0].value == lir.Var("t", f32)
    reads_acc = kernel([lir.Let("t", lir.Binary("mul", x, acc, f32))], lir.Binary("add", acc, lir.Var("t", f32), f32))
    two = kernel([lir.Let("t", x), lir.Let("u", x)],
                 lir.Binary("add", lir.Binary("add", acc, lir.Var("t", f32), f32), lir.Var("u", f32), f32))
    for bad in (reads_acc, two):
        with pytest.raises(gpu_schedule.ScheduleError, match="no loop"):
            gpu_schedule.GpuSchedule(bad).grid("i0").workgroup().lead().hoist()


def _nan_max_step(a, b):
    """One step of the reference's NaN-propagating maximum, as C evaluates it on float32."""
    return b if (a < b or b != b) else a


def _ordered_tree(values, threads: int, wave: int):
    """The grouping the generated ordered tree uses: each of ``threads`` threads folds a
    contiguous run in order from -inf, lanes of a ``wave``-wide wave combine by xor butterfly
    with the lower lanes' block on the left, then the waves' results are folded in wave order."""
    ninf = np.float32(-np.inf)
    run = -(-len(values) // threads) if values else 0
    m = []
    for t in range(threads):
        acc = ninf
        for v in values[t * run:min((t + 1) * run, len(values))]:
            acc = _nan_max_step(acc, v)
        m.append(acc)
    off = 1
    while off < wave:
        m = [_nan_max_step(m[i], m[i ^ off]) if (i & off) == 0 else _nan_max_step(m[i ^ off], m[i])
             for i in range(threads)]
        off <<= 1
    total = m[0]
    for w in range(1, threads // wave):
        total = _nan_max_step(total, m[w * wave])
    return total


def test_ordered_max_tree_is_the_serial_chain_bit_for_bit():
    """The NaN-propagating maximum's chain and the ordered tree codegen renders for it agree bit
    for bit on sequences built to separate them: NaNs of different payloads and signs (the chain
    keeps the last), +0 against -0 and equal values (the chain keeps the first), infinities,
    any length, any thread and wave count. A grouping that swapped a pair's sides, or dropped
    the accumulator's step, fails here."""
    bits_of = lambda x: np.float32(x).view(np.uint32)
    pool = [np.uint32(u).view(np.float32) for u in (0x7FC00000, 0x7FC00001, 0xFFC00002, 0x7F800001)]
    pool += [np.float32(v) for v in (0.0, -0.0, np.inf, -np.inf, 1.0, 1.0, 2.0, -3.5, 7.0, 7.0, -0.0)]
    rng = np.random.default_rng(5)
    for trial in range(3000):
        n = int(rng.integers(0, 40))
        values = [pool[int(i)] for i in rng.integers(0, len(pool), n)]
        init = pool[int(rng.integers(0, len(pool)))] if trial % 3 else np.float32(-np.inf)
        serial = init
        for v in values:
            serial = _nan_max_step(serial, v)
        for threads, wave in ((1, 1), (4, 2), (8, 4), (16, 4), (64, 8), (16, 16)):
            tree = _nan_max_step(init, _ordered_tree(values, threads, wave))
            assert bits_of(tree) == bits_of(serial), (values, init, threads, wave)
    # what the test would catch: a butterfly with its operands' sides swapped
    a, b = pool[0], pool[1]                                          # two NaNs: the chain keeps the last
    assert bits_of(_nan_max_step(a, b)) != bits_of(_nan_max_step(b, a))
    zero, negzero = np.float32(0.0), np.float32(-0.0)                # a tie: the chain keeps the first
    assert bits_of(_nan_max_step(zero, negzero)) != bits_of(_nan_max_step(negzero, zero))


def test_batches_never_read_what_the_statement_would_skip():
    """A batch reads its iterations' operands before running them, so a read under one arm of ?:
    is read ahead only as the whole ?: (evaluated as C does: the arm the statement would take;
    P.V's products read the past cache or the new rows by position, the other arm's index out
    of its array), and not at all when the condition depends on the iteration's own values."""
    prog = P.config5()[0]
    calls = _calls_of(prog)
    pv = prog.kernels[11]
    config = dict(gpu_schedule.default_config(pv, calls[11]), hoist=False, unroll=16)
    text = codegen_hip.render_kernel(*gpu_schedule.apply(pv, calls[11], config), 11)
    assert "nc_pf1_1[nc_u] = ((k < s1) ? x2[" in text
    assert "= x3[" not in text and "= x2[" not in text            # never read outside its ?:
    norm = prog.kernels[1]
    config = dict(gpu_schedule.DEFAULTS["row"], threads=512, stage=True, unroll=64, lead=True)
    text = codegen_hip.render_kernel(*gpu_schedule.apply(norm, calls[1], config), 1)
    assert "nc_pf1_0[nc_u] = nc_s1[r];" in text
    # the units of a statement, directly: a condition on the loop index takes the ?: whole; one on
    # the accumulator cannot be read ahead
    f32, i64 = lir.DType("f32"), lir.DType("i64")
    acc, r = lir.Var("acc", f32), lir.Var("r", i64)
    pick = lambda cond: lir.Select(cond, lir.Load(1, r, f32), lir.Load(2, b("sub", r, c(8)), f32), f32)
    by_index = pick(lir.Binary("lt", r, c(8), lir.DType("bool")))
    units: list = []
    st = lir.Assign("acc", lir.Binary("add", acc, by_index, f32))
    assert codegen_hip._prefetch_units(st, frozenset({"acc"}), frozenset(), {1, 2}, set(), units)
    assert units == [by_index]
    by_chain = pick(lir.Binary("lt", acc, lir.Const(0.0, f32), lir.DType("bool")))
    st = lir.Assign("acc", lir.Binary("add", acc, by_chain, f32))
    assert not codegen_hip._prefetch_units(st, frozenset({"acc"}), frozenset(), {1, 2}, set(), [])


def test_hoisted_nan_max_chain_renders_as_an_ordered_tree():
    program = P.zoo("softmax_mask")
    calls = _calls_of(program)
    scheduled, launch = gpu_schedule.apply(program.kernels[0], calls[0],
                                           dict(gpu_schedule.DEFAULTS["row"], stage=True, lead=True, hoist=True))
    text = codegen_hip.render_kernel(scheduled, launch, 0)
    # the maximum (nc_h0) as a tree over every thread; the sum of exps (nc_h1) stays the lead's chain
    assert "__shfl_xor(nc_m, nc_off, 64)" in text and "nc_h0_waves[threadIdx.x >> 6] = nc_m;" in text
    assert "acc0 = ((acc0 < nc_m) || (nc_m != nc_m)) ? nc_m : acc0;" in text
    assert "acc1 = (acc1 + nc_h1[r]);" in text


def test_unroll_batches_the_loop_around_lane_held_chains_but_not_register_array_stores():
    """With an item's accumulators held across lanes, its k loop updates one register a lane and
    may be unrolled: it runs in batches of the unroll factor, each batch loading its iterations'
    weight bytes and activations into register arrays before its multiply-adds (152 = 9 x 16 + 8:
    nine batches of 16, then one of 8), so a chain has 16 iterations' loads in flight. The tree
    after it, which stores into a register array, is never given a partial unroll hint (it would
    move the array to memory). Config 5's down projection, as the reference compiles it."""
    prog = P.config5()[0]
    kernel = prog.kernels[14]
    assert kernel.primitive == "matmul_i8+epilogue" and gpu_schedule.kernel_class(kernel) == "item"
    config = dict(gpu_schedule.DEFAULTS["item"], threads=128, lanes=1, unroll=16, pack=False)
    sched, launch = gpu_schedule.apply(kernel, (), config)
    unrolled = dict(launch.unroll)
    # one loop: the k loop (the tree's loop over the register array h stays without a hint)
    assert launch.lanes is not None and len(unrolled) == 1 and set(unrolled.values()) == {16}
    source = codegen_hip.render_kernel(sched, launch, 0, None)
    assert "#pragma unroll 16" not in source
    assert "for (int64_t nc_base = 0; nc_base < 144; nc_base += 16) {" in source
    assert "int8_t nc_pf1_0[16];" in source and "float nc_pf1_1[16];" in source
    assert "int8_t nc_pf1_0[8];" in source and "const int64_t k0 = 144 + nc_u;" in source
    # in each batch every load comes before the first multiply-add, which reads the arrays
    first = source.index("nc_pf1_0[nc_u] = x1[")
    assert first < source.index("nc_pf1_1[nc_u] = x2[") < source.index("acc_0_l = __builtin_fmaf(((float)(nc_pf1_0[nc_u]))")
    assert source.count("= x1[") == 2 and source.count("= x2[") == 2      # the batches' and the tail's
    # without lanes the same loop indexes the accumulator array: nothing to unroll
    with pytest.raises(gpu_schedule.ScheduleError):
        gpu_schedule.apply(kernel, (), dict(gpu_schedule.DEFAULTS["item"], threads=128, unroll=16, pack=False))


def test_lane_held_values_are_read_by_every_lane_and_only_the_store_is_guarded():
    """An item that stores its lane-held accumulators directly: the shuffle that fetches element
    e from lane e is evaluated by all of the item's lanes (outside ``if (nc_l == 0)``), and the
    scheduled program computes the unscheduled one's bits."""
    import re
    program = P.lane_store_program()
    kernel = program.kernels[0]
    s = gpu_schedule.GpuSchedule(kernel).grid("i0").lanes("acc")
    text = codegen_hip.render_kernel(s.kernel, s.launch, 0)
    assert "__shfl(" in text
    for line in text.splitlines():
        if "nc_l == 0" in line:
            assert "__shfl" not in line, line
    guarded = [m.group(0) for m in re.finditer(r"if \(nc_l == 0\)[^;]*;", text)]
    assert guarded and all("__shfl" not in g for g in guarded)
    x = np.random.default_rng(3).standard_normal((3, 32)).astype(np.float32)
    got = I.run(program, [(s.kernel, s.launch)], {"x": x}, {}, {})["y"]
    assert np.array_equal(got.view(np.uint32), P.lane_store_expected(x).view(np.uint32))


def test_lanes_refuses_element_loops_nested_from_the_smallest_coefficient():
    """acc[i + 2 j] with i outer: the lane's digits start at the outermost loop, which must carry
    the largest coefficient; the reversed nest is refused, not rendered wrongly."""
    f32 = lir.DType("f32")
    params = (lir.Param(f32, True), lir.Param(f32, False))

    def kernel(outer, inner, index):
        chain = lir.Loop(outer, c(2), (lir.Loop(inner, c(2), (lir.ArrayStore("acc", index, lir.Fma(
            lir.Load(1, index, f32), lir.Const(2.0, f32), lir.Local("acc", index, f32), f32)),)),))
        tail = lir.Store(0, v("i0"), lir.Local("acc", c(0), f32))
        return lir.Kernel("matmul", params, (lir.Loop("i0", c(3), (
            lir.Array("acc", 4, lir.Const(0.0, f32)), chain, tail)),))

    index = b("add", v("i"), b("mul", v("j"), c(2)))
    assert gpu_schedule.GpuSchedule(kernel("j", "i", index)).grid("i0").lanes("acc").launch.lanes.width == 4
    with pytest.raises(gpu_schedule.ScheduleError, match="largest coefficient"):
        gpu_schedule.GpuSchedule(kernel("i", "j", index)).grid("i0").lanes("acc")


def test_weights_are_resident_by_identity_not_by_id():
    """A compiled program keeps the arrays it uploaded and compares the next call's with ``is``:
    a fresh array that happens to get a freed array's id is not taken for the resident one."""
    prog = compiled.CompiledProgram.__new__(compiled.CompiledProgram)
    f32 = lir.DType("f32")
    prog.program = lir.Program("w", (), [], {"w": (f32, (4,))}, [], [], [], {})
    prog._held = None
    first = {"w": np.zeros(4, np.float32)}
    assert not prog._is_resident(first)
    prog._held = dict(first)
    assert prog._is_resident(first) and prog._is_resident({"w": first["w"]})
    assert not prog._is_resident({"w": first["w"].copy()})
    # the reused-id case: while held, the first array cannot be freed, so no new array shares
    # its id; an equal-valued new array is still a different object and is uploaded afresh
    ids = set()
    for _ in range(5):
        fresh = {"w": np.ones(4, np.float32)}
        ids.add(id(fresh["w"]))
        assert not prog._is_resident(fresh)
        del fresh
    assert id(first["w"]) not in ids
