"""The C ABI on the CPU: the library loads and exports every entry point include/splash_q4.h declares, and the
host-side planning and validation behave as the reference's ops::Linear / ops::MoE do (plans, storage rows,
scratch sizes, and std::invalid_argument before anything is launched). No GPU work is issued here."""
import pathlib
import re

import pytest

import splash_q4 as sq

ROOT = pathlib.Path(__file__).resolve().parent.parent


def declared_functions():
    text = sq.HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|uint32_t|const char \*)\s*(sq_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = sq.lib()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(sq.exported_symbols()) == names
    assert b"gfx950" in lib.sq_version()


def seg(n=4096, k=4096, fmt=sq.FMT_AF4G64, plane_bytes=None, meta_bytes=None, offset=0):
    p0, m = sq.plane_bytes(fmt, n, k) if fmt in sq.FORMATS else (1 << 30, 1 << 30)
    # fake device addresses: planning and validation never dereference them
    return sq.Segment(sq.Buffer(0x1000, plane_bytes if plane_bytes is not None else p0), sq.Buffer(None, 0),
                      sq.Buffer(0x2000000000, meta_bytes if meta_bytes is not None else m), n, k, offset, fmt)


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("rows", [1, 2, 4, 8, 16, 32])
def test_decode_plans(n, k, rows):
    proj = sq.projection(seg(n, k))
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    assert plan.config.tile == sq.TILE_STAGED
    s = plan.config.splits
    assert s & (s - 1) == 0 and 1 <= s <= 16 and (k // 32) % (2 * s) == 0
    assert plan.storage_rows == rows
    size, gate = sq.scratch_size(plan)
    assert size.partials == (s * rows * n * 4 if s > 1 else 0)
    assert size.counters == (n // 16 * 4 if s > 1 else 0)
    # the split depends on the tile kind the rows run, never on the rows: a row's result is the same in any batch
    # of its kind
    kind = 1 if rows <= 4 else 16 if rows <= 16 else 32
    assert s == sq.plan_for(sq.decode_workload(n, k, kind), proj).config.splits
    assert gate == 0


def split_law(n, k, budget, max_waves=16, pair=False, row=False, rows=16):
    """The fewest splits whose workgroups stream at most `budget` bytes, the grid kept within 256 compute units,
    among splits whose K slices fit one workgroup (at most `max_waves` waves of at most 32 groups). The row tile
    (`row`) of up to 16 rows runs a tile unsplit in four 16-column workgroups instead of split 64-column ones while
    the four fit the compute units and each streams at most 40 KB; a row tile already split doubles its split while
    the doubled split's 16-column workgroups fit the compute units and each K partition streams at least 32 KB; a
    split of more than two in 64-column workgroups gives way to the largest smaller one (of at least two) whose
    16-column workgroups fit the compute units and stream at most 30 KB each."""
    tiles, groups = n // 64, k // 32
    tile_bytes = (2 if pair else 1) * 64 * (k * 0.5 + groups * 2.0)
    best = None
    for s in (1, 2, 4, 8, 16):
        if groups % (2 * s) or groups // s > max_waves * 32:
            continue
        if best is not None and tiles * s > 256:
            break
        best = s
        if tile_bytes / s <= budget:
            break
    if row and rows <= 16 and best > 1 and tiles * best * 4 > 256 and tiles * 4 <= 256 and tile_bytes / 4 <= 40e3:
        return 1
    if row and best > 2 and tiles * best * 4 > 256:
        s = best // 2
        while s >= 2:
            if tiles * s * 4 <= 256:
                if tile_bytes / (4 * s) <= 30e3:
                    best = s
                break
            s //= 2
    while row and best > 1 and groups % (4 * best) == 0 and tiles * best * 8 <= 256 and tile_bytes / (2 * best) >= 32e3:
        best *= 2
    return best


@pytest.mark.parametrize("n,k,want", [(4096, 4096, 1), (1024, 4096, 1), (14336, 4096, 1), (4096, 14336, 4),
                                      (27648, 5120, 1), (4096, 16384, 4), (4096, 32768, 4)])
def test_split_law_column_tile(n, k, want):
    """Rows <= 4: workgroups of at most 160 KB."""
    s = sq.plan_for(sq.decode_workload(n, k, 1), sq.projection(seg(n, k))).config.splits
    assert s == want == split_law(n, k, 160e3)


@pytest.mark.parametrize("rows", [8, 16, 32])
@pytest.mark.parametrize("n,k,want", [(14336, 4096, 1), (1024, 4096, 4), (512, 4096, 4), (2048, 4096, 2),
                                      (4096, 4096, 1), (3072, 4096, 1), (4096, 8192, 4), (4096, 14336, 4),
                                      (1024, 2048, 1), (1024, 8192, 4), (2048, 8192, 4), (2048, 5120, 2)])
def test_split_law_row_tile(rows, n, k, want):
    """5..32 rows: workgroups of at most 80 KB; up to 16 rows, unsplit 16-column workgroups where the split would
    leave a few tiles in 64-column ones (4096 x 4096, 3072 x 4096: two splits at 32 rows), not where the split
    already fits 16-column ones (2048) or the unsplit ones would stream more than 40 KB (K 8192, 14336); a split of
    few tiles doubled while its 16-column workgroups fit the device and each split streams 32 KB (1024 and 512 x
    4096: four splits, not two); an unsplit tile stays unsplit (1024 x 2048); four splits in 64-column workgroups
    give way to two in 16-column ones of at most 30 KB (2048 x 5120), not of 37 KB (2048 x 8192)."""
    if rows == 32 and (n, k) in ((4096, 4096), (3072, 4096)):
        want = 2
    s = sq.plan_for(sq.decode_workload(n, k, rows), sq.projection(seg(n, k))).config.splits
    assert s == want == split_law(n, k, 80e3, row=True, rows=rows)


def test_prefill_plans():
    proj = sq.projection(seg(14336, 4096))
    plan = sq.plan_for(sq.prefill_workload(14336, 4096, 2048), proj)
    assert plan.config.tile == sq.TILE_PREFILL and plan.config.splits == 1 and plan.storage_rows == 2048
    size, _ = sq.scratch_size(plan)
    assert size.input == 2048 * 4096 * 2 and size.sums == 2048 * 4
    ragged = sq.plan_for(sq.prefill_workload(14336, 4096, 300), proj)
    assert ragged.storage_rows == 384
    short = sq.plan_for(sq.prefill_workload(14336, 4096, 32), proj)
    assert short.config.tile == sq.TILE_STAGED
    # 448 tiles of 256 rows: one whole round over the compute units, then 192 tiles as stream pieces, which store
    # the fp32 sums of at most two pieces a workgroup (256 x 256 x 4 bytes each, at most 256 workgroups) and keep a
    # counter a stream tile (at most a round and a half of tiles). 128 (N 4096 by K 14336) halve their K, whose fp32
    # halves [2][rows][N] the plan's partials hold; 32 tiles do neither.
    assert size.partials == 2 * 256 * 256 * 256 * 4 and size.counters == 384 * 4
    down = sq.projection(seg(4096, 14336))
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(4096, 14336, 2048), down))
    assert size.partials == 2 * 2048 * 4096 * 4 and size.counters == 0
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(4096, 14336, 300), down))
    assert size.partials == 0
    dev, bound = sq.device(), sq.LinearScratchSize()
    sq.call("sq_linear_prefill_scratch_size", sq.byref(dev), 4096, 14336, sq.byref(bound))
    assert bound.partials >= 2 * 2048 * 4096 * 4


def test_gate_up_plans():
    up, gate = sq.projection(seg(14336, 4096)), sq.projection(seg(14336, 4096))
    plan = sq.plan_for(sq.decode_workload(14336, 4096, 8, sq.EPILOGUE_GATE_UP), up, gate)
    assert plan.config.one_gate_up_pass == 1
    size, gate_bytes = sq.scratch_size(plan)
    assert gate_bytes == 0
    two = sq.plan_config(sq.decode_workload(14336, 4096, 8, sq.EPILOGUE_GATE_UP), sq.LinearConfig(sq.TILE_STAGED, 2, 0, 0, 0))
    assert sq.scratch_size(two)[1] == 8 * 14336 * 2
    # On the row tile a pair whose one pass would take K splits runs as two passes under the single tensor's split
    # law (and reports the gate scratch the first pass writes); unsplit pairs and the column tile keep one pass. A
    # column-tile pair of more tiles than compute units (17408 columns: 272) takes the byte budget's split past them.
    for (n, k), rows, want in [((14336, 4096), 4, (1, 1)), ((14336, 4096), 16, (1, 1)), ((14336, 4096), 32, (0, 1)),
                               ((17408, 5120), 1, (1, 4)), ((17408, 5120), 4, (1, 4)), ((17408, 5120), 8, (0, 1)),
                               ((17408, 5120), 32, (0, 1))]:
        up, gate = sq.projection(seg(n, k)), sq.projection(seg(n, k))
        plan = sq.plan_for(sq.decode_workload(n, k, rows, sq.EPILOGUE_GATE_UP), up, gate)
        assert (plan.config.one_gate_up_pass, plan.config.splits) == want, (n, k, rows)
        assert sq.scratch_size(plan)[1] == (0 if want[0] else rows * n * 2)


@pytest.mark.parametrize("workload,config,message", [
    (sq.decode_workload(100, 4096, 1), None, "invalid linear matrix"),
    (sq.decode_workload(4096, 4096, 33), None, "invalid linear decode workload"),
    (sq.decode_workload(4096, 4096, 0), None, "invalid linear decode workload"),
    (sq.decode_workload(4096, 4096, 8, sq.EPILOGUE_UP_WITH_GATE), None, "invalid linear decode workload"),
    (sq.prefill_workload(4096, 4096, 2049), None, "invalid linear prefill workload"),
    (sq.prefill_workload(4096, 4096, 64, sq.EPILOGUE_GATE_UP), None, "invalid linear prefill workload"),
    (sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_REGISTER, 1, 0, 0, 0), "register tile"),
    (sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_STAGED, 3, 0, 0, 0), "whole 32-input groups"),
    (sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_STAGED, 32, 0, 0, 0), "whole 32-input groups"),
    (sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_PREFILL, 1, 0, 0, 0), "invalid block prefill"),
    (sq.prefill_workload(4096, 4096, 64), sq.LinearConfig(sq.TILE_STAGED, 1, 0, 0, 0), "up to 32 rows"),
    (sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_STAGED, 1, 0, 1, 0), "one pass"),
])
def test_invalid_plans_raise(workload, config, message):
    with pytest.raises(sq.InvalidArgument, match=message):
        if config is None:
            sq.plan_for(workload)
        else:
            sq.plan_config(workload, config)


def test_fp32_destination_only_plain_decode():
    with pytest.raises(sq.InvalidArgument, match="fp32 destination"):
        sq.plan_config(sq.prefill_workload(4096, 4096, 64), sq.LinearConfig(sq.TILE_PREFILL, 1, 0, 0, 0), sq.OUTPUT_F32)
    plan = sq.plan_config(sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_STAGED, 4, 0, 0, 0), sq.OUTPUT_F32)
    assert plan.destination == sq.OUTPUT_F32


def test_projection_and_plane_validation():
    with pytest.raises(sq.InvalidArgument, match="plane0"):
        sq.call("sq_require_segment_planes", sq.byref(seg(plane_bytes=1024)), b"projection", 0)
    with pytest.raises(sq.InvalidArgument, match="meta"):
        sq.call("sq_require_segment_planes", sq.byref(seg(meta_bytes=16)), b"projection", 0)
    sq.call("sq_require_segment_planes", sq.byref(seg()), b"projection", 0)
    with pytest.raises(sq.InvalidArgument, match="not one this build runs"):
        sq.call("sq_require_segment_planes", sq.byref(seg(fmt=12, plane_bytes=1 << 30, meta_bytes=1 << 30)), b"projection", 0)
    # segments must tile the leading columns in order
    bad = sq.projection([seg(2048, 4096), seg(2048, 4096, offset=1024)], output_size=4096)
    with pytest.raises(sq.InvalidArgument, match="do not tile"):
        sq.plan_for(sq.decode_workload(4096, 4096, 1), bad)


def test_add_validates_buffers_before_launch():
    """Undersized buffers throw on the host (Linear.cpp:203-221); nothing reaches a GPU."""
    proj = sq.projection(seg(4096, 4096))
    plan = sq.plan_config(sq.decode_workload(4096, 4096, 8), sq.LinearConfig(sq.TILE_STAGED, 4, 0, 0, 0))
    fake = lambda nbytes: sq.Buffer(0x4000, nbytes)
    scratch = sq.LinearScratch(sq.Buffer(None, 0), sq.Buffer(None, 0), fake(4 * 8 * 4096 * 4), fake(4096 // 64 * 4),
                               sq.Buffer(None, 0))
    cases = [
        (sq.LinearBuffers(fake(8 * 4096 * 2 - 2), fake(8 * 4096 * 2), sq.Buffer(None, 0), sq.Buffer(None, 0), scratch), "projection input"),
        (sq.LinearBuffers(fake(8 * 4096 * 2), fake(100), sq.Buffer(None, 0), sq.Buffer(None, 0), scratch), "projection output"),
        (sq.LinearBuffers(fake(8 * 4096 * 2), fake(8 * 4096 * 2), sq.Buffer(None, 0), sq.Buffer(None, 0),
                          sq.LinearScratch()), "projection partials"),
    ]
    for buffers, message in cases:
        with pytest.raises(sq.InvalidArgument, match=message):
            sq.call("sq_linear_add", None, sq.byref(buffers), sq.byref(proj), sq.byref(plan), None)
    residual_plan = sq.plan_config(sq.decode_workload(4096, 4096, 8, sq.EPILOGUE_RESIDUAL), sq.LinearConfig(sq.TILE_STAGED, 1, 0, 0, 0))
    buffers = sq.LinearBuffers(fake(8 * 4096 * 2), fake(8 * 4096 * 2), fake(10), sq.Buffer(None, 0), sq.LinearScratch())
    with pytest.raises(sq.InvalidArgument, match="projection residual"):
        sq.call("sq_linear_add", None, sq.byref(buffers), sq.byref(proj), sq.byref(residual_plan), None)
    gate_plan = sq.plan_config(sq.decode_workload(4096, 4096, 8, sq.EPILOGUE_GATE_UP), sq.LinearConfig(sq.TILE_STAGED, 1, 0, 0, 0))
    with pytest.raises(sq.InvalidArgument, match="gate projection"):
        sq.call("sq_linear_add", None, sq.byref(buffers), sq.byref(proj), sq.byref(gate_plan), None)


def test_scratch_bounds_cover_every_plan():
    dev = sq.device()
    out = sq.LinearScratchSize()
    sq.call("sq_linear_decode_scratch_size", sq.byref(dev), 14336, 4096, sq.byref(out))
    for rows in range(1, 33):
        for e in (sq.EPILOGUE_NONE, sq.EPILOGUE_RESIDUAL):
            size, _ = sq.scratch_size(sq.plan_for(sq.decode_workload(14336, 4096, rows, e)))
            assert size.partials <= out.partials and size.counters <= out.counters
    # The bound holds the plans of projections of every format, and the one-pass gate/up pairs (whose partials
    # hold both tensors' columns) among them.
    for n, k in [(14336, 4096), (17408, 5120), (2048, 2048), (4096, 14336)]:
        sq.call("sq_linear_decode_scratch_size", sq.byref(dev), n, k, sq.byref(out))
        pairs = 0
        for fmt in sq.FORMATS:
            up, gate = sq.projection(seg(n, k, fmt)), sq.projection(seg(n, k, fmt))
            for rows in range(1, 33):
                for e in (sq.EPILOGUE_NONE, sq.EPILOGUE_RESIDUAL, sq.EPILOGUE_GATE_UP):
                    plan = sq.plan_for(sq.decode_workload(n, k, rows, e), up, gate if e == sq.EPILOGUE_GATE_UP else None)
                    size, _ = sq.scratch_size(plan)
                    assert size.partials <= out.partials and size.counters <= out.counters, (n, k, fmt, rows, e)
                    pairs += plan.config.one_gate_up_pass and plan.config.splits > 1
        assert n != 17408 or pairs, "a split one-pass pair among the plans"
    sq.call("sq_linear_prefill_scratch_size", sq.byref(dev), 14336, 4096, sq.byref(out))
    assert out.input == 2048 * 4096 * 2


def moe_plan(kind, shape, count, config=None):
    plan = sq.MoePlan()
    if kind == "rows":
        sq.call("sq_moe_decode_rows_plan", sq.byref(shape), count, sq.byref(plan))
    else:
        sq.call(f"sq_moe_{kind}_plan", sq.byref(shape), count, sq.byref(config) if config is not None else None,
                sq.byref(plan))
    return plan


def test_moe_plans_and_workspace():
    shape = sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64)
    plan = moe_plan("prefill", shape, 512)
    assert plan.tile_rows == 32 and plan.config.expert_tile == 32
    routes = 512 * 8
    assert plan.maximum_tiles == min(routes // 32 + 128, routes)
    w = plan.workspace
    assert w.selected_experts == routes * 4 and w.route_rows == routes * 4
    assert w.tile_descriptors == plan.maximum_tiles * 8 and w.tile_count == 40
    assert w.expert_intermediate == plan.maximum_tiles * 32 * 768 * 2
    assert w.expert_output == plan.maximum_tiles * 32 * 2048 * 2
    # The grouped input holds the router's scores (a row of 256 expert slots per row) until the routed work
    # overwrites them with the block's input rows in the tiles' read order (MoE.cpp:64-84).
    assert w.grouped_input == max(512 * 256 * 4, 512 * 2048 * 2)
    assert sq.lib().sq_moe_router_width(sq.byref(shape)) == 256
    wide = sq.MoeShape(2048, 300, 8, 768, sq.FMT_AF4G64)
    assert sq.lib().sq_moe_router_width(sq.byref(wide)) == 512
    assert moe_plan("prefill", wide, 10).workspace.grouped_input == max(10 * 512 * 4, 10 * 2048 * 2)
    narrow = sq.MoeShape(256, 300, 8, 128, sq.FMT_AF4G64)   # the scores outweigh the input rows
    assert moe_plan("prefill", narrow, 10).workspace.grouped_input == 10 * 512 * 4
    plan = moe_plan("prefill", shape, 8)
    assert plan.tile_rows == 8   # 8 rows x 8 routes <= 128 experts
    with pytest.raises(sq.InvalidArgument, match="invalid MoE workspace shape"):
        moe_plan("prefill", sq.MoeShape(2000, 128, 8, 768, sq.FMT_AF4G64), 8)
    with pytest.raises(sq.InvalidArgument, match="invalid MoE rows"):
        moe_plan("rows", shape, 33)
    with pytest.raises(sq.InvalidArgument, match="invalid MoE prefill rows"):
        moe_plan("prefill", shape, 2049)


def test_moe_decode_plan_takes_lanes():
    """MoE::decodePlan(shape, lanes, config) (MoE.cpp:567-571): a lane is 8 rows, at most 4 lanes; the policy's
    config is 8-row staged tiles in decode, and a 32-row tile or the register tile is refused (MoE.cpp:196-206)."""
    shape = sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64)
    for lanes in (1, 2, 4):
        plan = moe_plan("decode", shape, lanes)
        assert plan.rows == 8 * lanes and plan.tile_rows == 8 and plan.phase == sq.PHASE_DECODE
        assert plan.workspace.selected_experts == 8 * lanes * 8 * 4
        assert plan.maximum_tiles == min(8 * lanes * 8 // 8 + 128, 8 * lanes * 8)
    for lanes in (0, 5):
        with pytest.raises(sq.InvalidArgument, match="invalid MoE decode batch width"):
            moe_plan("decode", shape, lanes)
    config = sq.MoeConfig()
    sq.call("sq_moe_config_for", sq.byref(shape), 16, sq.PHASE_DECODE, sq.byref(config))
    assert (config.expert_tile, config.gguf_tile, config.router_tile, config.cpu_bf16_experts) == (8, 0, 0, 0)
    assert moe_plan("decode", shape, 2, config).rows == 16
    with pytest.raises(sq.InvalidArgument, match="invalid MoE expert tile configuration"):
        moe_plan("decode", shape, 2, sq.MoeConfig(32, 0, 0, 0))
    with pytest.raises(sq.InvalidArgument, match="register expert tile"):
        moe_plan("decode", shape, 2, sq.MoeConfig(8, sq.MOE_GGUF_TILE_REGISTER, 0, 0))
    with pytest.raises(sq.InvalidArgument, match="invalid MoE expert tile configuration"):
        moe_plan("prefill", shape, 64, sq.MoeConfig(16, 0, 0, 0))
    # A prefill caller's config is taken as given: 8-row tiles on a chunk the policy would give 32.
    assert moe_plan("prefill", shape, 512, sq.MoeConfig(8, 0, sq.FLOAT_TILE_NEURAL_ACCELERATOR, 1)).tile_rows == 8
    sq.call("sq_moe_config_for", sq.byref(shape), 512, sq.PHASE_PREFILL, sq.byref(config))
    assert config.expert_tile == 32
    # The rows entry (no counterpart in the reference) takes any 1..32 rows.
    assert moe_plan("rows", shape, 3).rows == 3


def test_moe_plan_fields_must_match():
    """A plan whose fields were changed after planning is refused rather than run with another workspace."""
    shape = sq.MoeShape(512, 16, 4, 256, sq.FMT_AF4G64)
    plan = moe_plan("prefill", shape, 100)
    plan.tile_rows = 8
    buffers = sq.MoeBuffers()
    weights = sq.MoeWeights()
    with pytest.raises(sq.InvalidArgument, match="do not match"):
        sq.call("sq_moe_add", None, sq.byref(buffers), sq.byref(weights), sq.byref(plan))


def test_moe_verify_rows_refusals():
    """Verify rows are a decode step's, one uint32 per lane of 8 rows (MoE.cpp:467-475)."""
    shape = sq.MoeShape(512, 16, 4, 256, sq.FMT_AF4G64)
    n_i, n_h = 16 * 256, 16 * 512
    seg = lambda n, k: sq.Segment(_fake(n * k // 2, 1 << 28), sq.Buffer(), _fake(n * k // 16, 1 << 29), n, k, 0,
                                  sq.FMT_AF4G64)
    weights = sq.MoeWeights(seg(n_i, 512), seg(n_i, 512), seg(n_h, 256), _fake(64, 1 << 27), 16)
    for kind, count, verify_bytes, message in (("prefill", 16, 8, "only a verify step"),
                                               ("decode", 2, 4, "MoE verify rows")):
        plan = moe_plan(kind, shape, count)
        w = plan.workspace
        scratch = sq.MoeScratch(*[_fake(max(getattr(w, n), 16), (1 << 30) + (i << 24))
                                  for i, n in enumerate(sq._MOE_WORKSPACE)])
        io = _fake(plan.rows * 512 * 2, 1 << 26)
        buffers = sq.MoeBuffers(io, sq.Buffer(), io, scratch, _fake(verify_bytes, 1 << 25))
        with pytest.raises(sq.InvalidArgument, match=message):
            sq.call("sq_moe_add", None, sq.byref(buffers), sq.byref(weights), sq.byref(plan))


def test_moe_shared_slice_plans():
    """Shared slices add their routes to every row and one tile per tile_rows rows each (MoE.hpp:200-205); only the
    compiled routings plan (kCompiledMoeRoutings, MoE.hpp:34-46)."""
    gated = sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64, sq.ROUTER_SOFTMAX, 1, 1)
    plan = moe_plan("prefill", gated, 500)
    assert plan.maximum_tiles == min(500 * 8 // 32 + 128, 500 * 8) + 16
    assert plan.workspace.selected_experts == 500 * 9 * 4 and plan.workspace.route_rows == 500 * 9 * 4
    assert plan.workspace.expert_output == plan.maximum_tiles * 32 * 2048 * 2
    two = sq.MoeShape(2048, 64, 6, 512, sq.FMT_AF4G64, sq.ROUTER_SIGMOID_NORMALIZED, 2, 0)
    plan = moe_plan("rows", two, 3)
    assert plan.tile_rows == 8 and plan.maximum_tiles == min(3 * 6 // 8 + 64, 18) + 2
    for router, slices, gate in ((sq.ROUTER_SOFTMAX, 2, 0), (sq.ROUTER_SOFTMAX, 1, 0),
                                 (sq.ROUTER_SIGMOID_NORMALIZED, 2, 1), (sq.ROUTER_SIGMOID_NORMALIZED, 0, 0)):
        with pytest.raises(sq.InvalidArgument, match="invalid MoE workspace shape"):
            moe_plan("prefill", sq.MoeShape(2048, 64, 6, 512, sq.FMT_AF4G64, router, slices, gate), 8)
    with pytest.raises(sq.InvalidArgument, match="unknown MoE router"):
        moe_plan("prefill", sq.MoeShape(2048, 64, 6, 512, sq.FMT_AF4G64, 2, 0, 0), 8)


def test_cxx_face_plans_and_throws(tmp_path):
    """include/splash_q4.hpp compiles as C++17, plans through the library and turns a refused plan back into the
    reference's std::invalid_argument (host only)."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    exe = tmp_path / "wrapper_check"
    lib_dir = sq.LIBRARY.parent
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(sq.HEADER.parent), str(ROOT / "tests" / "cxx_wrapper_check.cpp"),
                    "-L", str(lib_dir), "-lsplash_q4", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert "decode rows 8 tile 0" in out and "prefill tile 1" in out
    assert "moe decode rows 16 tile 8; moe prefill tile 32" in out
    assert "expert load groups 8" in out   # max(128 x 16, 256 x 8) pairs / 256 threads
    assert "invalid_argument:" in out


def test_prefill_buffers_are_aligned():
    """The prefill tile moves 16-byte vectors: a buffer off 16-byte alignment is refused on the host."""
    proj = sq.projection(seg(4096, 4096))
    plan = sq.plan_for(sq.prefill_workload(4096, 4096, 256), proj)
    size, _ = sq.scratch_size(plan)
    scratch = sq.LinearScratch(sq.Buffer(0x10000, size.input), sq.Buffer(0x20000, size.sums), sq.Buffer(None, 0),
                               sq.Buffer(None, 0), sq.Buffer(None, 0))
    buffers = sq.LinearBuffers(sq.Buffer(0x40000, 256 * 4096 * 2), sq.Buffer(0x80002, 256 * 4096 * 2),
                               sq.Buffer(None, 0), sq.Buffer(None, 0), scratch)
    with pytest.raises(sq.InvalidArgument, match="16-byte aligned"):
        sq.call("sq_linear_add", None, sq.byref(buffers), sq.byref(proj), sq.byref(plan), None)


def _fake(nbytes, at=1 << 20):
    """A buffer view the host validates but nothing dereferences (every call below is refused before a launch)."""
    return sq.Buffer(at, nbytes)


def test_plan_input_layouts():
    """LinearPlan::input: the prefill tile reads the half-rows table, the decode tiles plain rows."""
    layout = sq.c_uint32()
    for workload, want in ((sq.prefill_workload(1024, 2048, 512), sq.LINEAR_INPUT_HALF_ROWS),
                           (sq.decode_workload(1024, 2048, 4), sq.LINEAR_INPUT_PLAIN)):
        sq.call("sq_linear_plan_input", sq.byref(sq.plan_for(workload)), sq.byref(layout))
        assert layout.value == want


def test_norm_and_float_rows_refusals():
    """The producers' validation (host only): whole 64-input spans, the Apple9 table refused, a table scratch that
    holds the rows, float rows F32 or BF16 only, destination columns inside the stride."""
    rows, width = 8, 2048
    io = _fake(rows * width * 2)
    weights = sq.NormWeights(_fake(width * 2), 0)
    table = sq.LinearScratch(_fake(rows * width * 2, 1 << 24), _fake(rows * 4, 1 << 25), sq.Buffer(), sq.Buffer(),
                             sq.Buffer())
    with pytest.raises(sq.InvalidArgument, match="64-input spans"):
        sq.call("sq_norm_add_rms", None, io, sq.byref(weights), io, 100, 1, None, sq.LINEAR_INPUT_PLAIN, None)
    with pytest.raises(sq.InvalidArgument, match="register tile"):
        sq.call("sq_norm_add_rms", None, io, sq.byref(weights), io, width, rows, sq.byref(table),
                sq.LINEAR_INPUT_TABLE16, None)
    small = sq.LinearScratch(_fake(rows * width, 1 << 24), _fake(rows * 4, 1 << 25), sq.Buffer(), sq.Buffer(),
                             sq.Buffer())
    with pytest.raises(sq.InvalidArgument, match="norm table scratch"):
        sq.call("sq_norm_add_rms", None, io, sq.byref(weights), io, width, rows, sq.byref(small),
                sq.LINEAR_INPUT_HALF_ROWS, None)
    with pytest.raises(sq.InvalidArgument, match="unknown linear input layout"):
        sq.call("sq_norm_add_rms", None, io, sq.byref(weights), io, width, rows, None, 7, None)
    q4k = sq.Segment(_fake(64 * 2048), sq.Buffer(), sq.Buffer(), 64, 2048, 0, sq.FMT_Q4K)
    with pytest.raises(sq.InvalidArgument, match="F32 or BF16"):
        sq.call("sq_float_add", None, io, sq.byref(q4k), io, rows, 64, 0, sq.OUTPUT_F32, sq.FLOAT_TILE_SIMDGROUP)
    f32 = sq.Segment(_fake(64 * 2048 * 4), sq.Buffer(), sq.Buffer(), 64, 2048, 0, sq.FLOAT32_ROWS)
    with pytest.raises(sq.InvalidArgument, match="outside its destination"):
        sq.call("sq_float_add", None, io, sq.byref(f32), _fake(rows * 64 * 4), rows, 64, 8, sq.OUTPUT_F32,
                sq.FLOAT_TILE_SIMDGROUP)


def test_float_tile_policy_and_refusals():
    """Linear::ggufFloatTile: the matrix-core tile from 64 rows on, the lane chains below; the matrix-core tile takes
    inputs in multiples of 256 and an unknown tile is refused."""
    dev, tile = sq.device(), sq.c_uint32()
    for rows, want in ((1, sq.FLOAT_TILE_SIMDGROUP), (63, sq.FLOAT_TILE_SIMDGROUP),
                       (64, sq.FLOAT_TILE_NEURAL_ACCELERATOR), (2048, sq.FLOAT_TILE_NEURAL_ACCELERATOR)):
        sq.call("sq_linear_float_tile", sq.byref(dev), rows, 256, sq.FLOAT32_ROWS, sq.byref(tile))
        assert tile.value == want, rows
    rows = 64
    f32 = sq.Segment(_fake(64 * 2112 * 4), sq.Buffer(), sq.Buffer(), 64, 2112, 0, sq.FLOAT32_ROWS)
    io = _fake(rows * 2112 * 4)
    with pytest.raises(sq.InvalidArgument, match="multiples of 256"):
        sq.call("sq_float_add", None, io, sq.byref(f32), io, rows, 64, 0, sq.OUTPUT_F32,
                sq.FLOAT_TILE_NEURAL_ACCELERATOR)
    with pytest.raises(sq.InvalidArgument, match="unknown float tile"):
        sq.call("sq_float_add", None, io, sq.byref(f32), io, rows, 64, 0, sq.OUTPUT_F32, 2)
    # the MoE policy takes its router tile from the same rule
    shape = sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64, sq.ROUTER_SOFTMAX, 0, 0)
    for rows, phase in ((512, sq.PHASE_PREFILL), (16, sq.PHASE_DECODE)):
        config = sq.MoeConfig()
        sq.call("sq_moe_config_for", sq.byref(shape), rows, phase, sq.byref(config))
        sq.call("sq_linear_float_tile", sq.byref(dev), rows, 128, sq.FLOAT32_ROWS, sq.byref(tile))
        assert config.router_tile == tile.value


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (27648, 5120)])
def test_decode_storage_rows_match_every_plan(n, k):
    """Linear::decodeStorageRows is the storage_rows of every decode plan of its rows, whatever the epilogue, and of
    the lane plans (lanes x 8 rows)."""
    dev, out = sq.device(), sq.c_uint32()
    proj = sq.projection(seg(n, k))
    for rows in range(1, 33):
        sq.call("sq_linear_decode_storage_rows", sq.byref(dev), rows, n, k, sq.byref(out))
        for e in (sq.EPILOGUE_NONE, sq.EPILOGUE_RESIDUAL, sq.EPILOGUE_GATE_UP):
            assert sq.plan_for(sq.decode_workload(n, k, rows, e)).storage_rows == out.value, (rows, e)
        assert sq.plan_for(sq.decode_workload(n, k, rows), proj).storage_rows == out.value
    for lanes in range(1, 5):
        plan = sq.LinearPlan()
        sq.call("sq_linear_decode_plan", sq.byref(dev), sq.byref(proj), lanes, sq.EPILOGUE_NONE, None, sq.byref(plan))
        sq.call("sq_linear_decode_storage_rows", sq.byref(dev), 8 * lanes, n, k, sq.byref(out))
        assert plan.storage_rows == out.value
    with pytest.raises(sq.InvalidArgument, match="invalid linear decode workload"):
        sq.call("sq_linear_decode_storage_rows", sq.byref(dev), 33, n, k, sq.byref(out))


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (27648, 5120), (5120, 27648), (8192, 3072)])
def test_prefill_scratch_size_covers_every_chunk(n, k):
    """Linear::prefillScratchSize bounds the scratch of every prefill chunk of 1..2048 rows, the halved-K partials of
    the row bands that halve included (the reference's arenas are sized from it)."""
    dev, bound = sq.device(), sq.LinearScratchSize()
    sq.call("sq_linear_prefill_scratch_size", sq.byref(dev), n, k, sq.byref(bound))
    halved = streamed = 0
    for rows in range(1, 2049):
        size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(n, k, rows)))
        for f in ("input", "sums", "partials", "counters"):
            assert getattr(size, f) <= getattr(bound, f), (rows, f)
        if rows > 32 and size.partials:
            # halved K: [2][rows][N] fp32 and no counters; stream pieces: 256 workgroups' two slots and counters
            stream = size.counters > 0
            assert size.partials == (2 * 256 * 256 * 256 * 4 if stream else 2 * rows * n * 4), rows
            halved += not stream
            streamed += stream
    if (n, k) == (14336, 4096):
        # rows 257..512 halve; rows 1793..2048 (448 tiles: more than one round, in row blocks that divide the 256
        # compute units) run their last round's tiles as stream pieces
        assert halved == 256 and streamed == 256 and bound.partials == 2 * 256 * 256 * 256 * 4


def test_moe_add_routes_refusals():
    """MoE::addRoutes validates on the host before any launch: the shape, the rows, the router's rows, the buffers'
    sizes and alignment, and the tile."""
    shape = sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64, sq.ROUTER_SOFTMAX, 0, 0)
    rows = 16
    x, scores = _fake(rows * 2048 * 2), _fake(rows * 256 * 4, 1 << 24)
    sel, wts = _fake(rows * 8 * 4, 1 << 25), _fake(rows * 8 * 4, 1 << 26)
    router = sq.Segment(_fake(128 * 2048 * 4, 1 << 27), sq.Buffer(), sq.Buffer(), 128, 2048, 0, sq.FLOAT32_ROWS)
    call = lambda **kw: sq.call("sq_moe_add_routes", None, kw.get("x", x), sq.byref(kw.get("router", router)),
                                sq.Buffer(), kw.get("scores", scores), kw.get("sel", sel), kw.get("wts", wts),
                                kw.get("rows", rows), sq.byref(kw.get("shape", shape)), kw.get("tile", 0))
    with pytest.raises(sq.InvalidArgument, match="router scores"):
        call(scores=_fake(rows * 128 * 4, 1 << 24))
    with pytest.raises(sq.InvalidArgument, match="selected experts"):
        call(sel=_fake(rows * 4, 1 << 25))
    with pytest.raises(sq.InvalidArgument, match="routing weights"):
        call(wts=_fake(rows * 4, 1 << 26))
    with pytest.raises(sq.InvalidArgument, match="invalid MoE routing rows"):
        call(rows=0)
    with pytest.raises(sq.InvalidArgument, match="router does not match"):
        call(router=sq.Segment(_fake(64 * 2048 * 4, 1 << 27), sq.Buffer(), sq.Buffer(), 64, 2048, 0, sq.FLOAT32_ROWS))
    with pytest.raises(sq.InvalidArgument, match="invalid MoE routing shape"):
        call(shape=sq.MoeShape(2048, 128, 8, 768, sq.FMT_AF4G64, sq.ROUTER_SOFTMAX, 1, 0))
    with pytest.raises(sq.InvalidArgument, match="16-byte aligned"):
        call(x=_fake(rows * 2048 * 2, (1 << 20) + 8))
    with pytest.raises(sq.InvalidArgument, match="router tile"):
        call(tile=2)


def test_static_scratch_entry_point_refusals():
    """sq_linear_add_static refuses, on the host and before touching any device, a plan whose scratch exceeds its
    static array, and a prepared-input handoff (its table is its own)."""
    proj = sq.projection(seg(14336, 4096))
    plan = sq.plan_for(sq.prefill_workload(14336, 4096, 2048), proj)   # a 16 MiB fp16 table plus row scales
    buffers = sq.LinearBuffers(_fake(2048 * 4096 * 2), _fake(2048 * 14336 * 2, 1 << 34), sq.Buffer(), sq.Buffer(),
                               sq.LinearScratch())
    with pytest.raises(sq.InvalidArgument, match="the static scratch holds 16777216"):
        sq.call("sq_linear_add_static", None, sq.byref(buffers), sq.byref(proj), sq.byref(plan), None)
    buffers.prepared = sq.PreparedInput(_fake(16), sq.LINEAR_INPUT_HALF_ROWS)
    with pytest.raises(sq.InvalidArgument, match="prepared must be empty"):
        sq.call("sq_linear_add_static", None, sq.byref(buffers), sq.byref(proj), sq.byref(plan), None)


def test_moe_expert_load_refusals():
    """MoE::addExpertLoad validates its projections and buffers on the host before any launch; the groups follow
    MoE::expertLoadGroups (MoE.cpp:545-551); no jobs launch nothing."""
    params = sq.ExpertLoadParams()
    for z, (fmt, rows, cols) in enumerate([(sq.FMT_Q4K, 128, 512), (sq.FMT_AF4G64, 64, 2048), (sq.FMT_Q6K, 256, 256)]):
        q = params.projections[z]
        q.format_id, q.rows, q.columns = fmt, rows, cols
        q.row_bytes = cols // (256 if fmt in (sq.FMT_Q4K, sq.FMT_Q6K) else 64) * (144 if fmt == sq.FMT_Q4K else
                                                                              210 if fmt == sq.FMT_Q6K else 36)
        q.slot_bytes[0] = q.slot_bytes[1] = q.slot_bytes[2] = 1 << 20
    assert sq.lib().sq_moe_expert_load_groups(sq.byref(params)) == 64 * 64 // 256
    jobs = 4
    good = dict(staging=_fake(1 << 24), arena=_fake(1 << 26, 1 << 30), slots=_fake(jobs * 4, 1 << 24),
                sources=_fake(jobs * 24, 1 << 25), grid=_fake(12, 1 << 26), jobs=jobs)

    def call(p=params, **kw):
        a = {**good, **kw}
        sq.call("sq_moe_expert_load", None, a["staging"], a["arena"], a["slots"], a["sources"], sq.byref(p),
                a["jobs"], a["grid"])

    def edited(z, **fields):
        p = sq.ExpertLoadParams.from_buffer_copy(params)
        for k, v in fields.items():
            if k == "slot_bytes":
                p.projections[z].slot_bytes[v[0]] = v[1]
            else:
                setattr(p.projections[z], k, v)
        return p
    call(jobs=0)   # nothing to launch
    with pytest.raises(sq.InvalidArgument, match="gate takes a format"):
        call(edited(0, format_id=99))
    with pytest.raises(sq.InvalidArgument, match="up takes whole plane tiles"):
        call(edited(1, rows=96))
    with pytest.raises(sq.InvalidArgument, match="down takes whole plane tiles"):
        call(edited(2, columns=384))
    with pytest.raises(sq.InvalidArgument, match="gate rows are shorter"):
        call(edited(0, row_bytes=100))
    with pytest.raises(sq.InvalidArgument, match="down slots are smaller"):
        call(edited(2, slot_bytes=(1, 256 * 8 * 8 - 1)))
    with pytest.raises(sq.InvalidArgument, match="expert load slots"):
        call(slots=_fake(jobs * 4 - 4, 1 << 24))
    with pytest.raises(sq.InvalidArgument, match="expert load sources"):
        call(sources=_fake(jobs * 24 - 8, 1 << 25))
    with pytest.raises(sq.InvalidArgument, match="expert load grid"):
        call(grid=_fake(8, 1 << 26))
    with pytest.raises(sq.InvalidArgument, match="8-byte"):
        call(sources=_fake(jobs * 24, (1 << 25) + 4))
    with pytest.raises(sq.InvalidArgument, match="staging and arena"):
        call(staging=sq.Buffer())
