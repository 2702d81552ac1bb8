"""MoE blocks through the C ABI against the oracle (kernels/shared/moe.metal, moe_gguf.metal): the top-k selection
bit for bit (ties to the lower expert id), the router's weights (renormalised softmax, or sigmoids over their sum)
and the shared slices' (sigmoid of the scalar gate's product, or 1), the grouping (tiles in expert order, each
expert's routes in route order, then the shared slices' tiles, padding marked ~0u), and the combined output against
an fp64 SwiGLU of every route with the kernels' bf16 rounding points, within BASELINE's tolerances."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import DeviceAffine, make_weights, to_device, to_host, torch
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


class Block:
    """Routed experts in `fmt`; `shared` shared slices with gate and up in shared_fmt and down in down_fmt, laid out
    as the reference's BlockExpertProjection (slice s's rows s * N on); a scalar gate when `gated`. `formats` names
    any projection's own format ("gate", "up", "down", "shared_gate", ...), as the reference's blocks carry them."""

    def __init__(self, rng, experts, hidden, intermediate, fmt=oracle.FMT_AF4G64, shared=0, gated=False,
                 router=oracle.ROUTER_SOFTMAX, shared_fmt=None, down_fmt=None, formats=None, device_repack=False):
        self.e, self.h, self.i, self.fmt = experts, hidden, intermediate, fmt
        self.shared, self.gated, self.router = shared, gated, router
        self.parts = {}
        formats = formats or {}
        plan = [("gate", experts * intermediate, hidden, fmt), ("up", experts * intermediate, hidden, fmt),
                ("down", experts * hidden, intermediate, fmt)]
        if shared:
            sf = fmt if shared_fmt is None else shared_fmt
            df = sf if down_fmt is None else down_fmt
            plan += [("shared_gate", shared * intermediate, hidden, sf), ("shared_up", shared * intermediate, hidden, sf),
                     ("shared_down", shared * hidden, intermediate, df)]
        plan = [(name, n, k, formats.get(name, f)) for name, n, k, f in plan]
        for name, n, k, f in plan:
            # device_repack: af4g64 planes from the library's MLX repack, values from numpy (helpers.DeviceAffine)
            self.parts[name] = (DeviceAffine(rng, n, k) if device_repack and f == oracle.FMT_AF4G64
                                else make_weights(rng, f, n, k))
        self.slots = to_device(np.arange(experts, dtype=np.uint32))
        self.scalar_gate = rng.normal(0, 0.05, hidden).astype(np.float32) if gated else None

    def segment(self, name):
        if name not in self.parts:
            return sq.Segment()
        return self.parts[name].segment()

    def weights(self):
        self._gate = to_device(self.scalar_gate) if self.gated else None
        router = sq.Segment()
        if getattr(self, "router_rows", None) is not None:
            self._router = to_device(self.router_rows)
            router = sq.Segment(sq.view(self._router), sq.view(None), sq.view(None), self.e, self.h, 0,
                                sq.FLOAT32_ROWS)
        return sq.MoeWeights(self.segment("gate"), self.segment("up"), self.segment("down"), sq.view(self.slots), self.e,
                             self.segment("shared_gate"), self.segment("shared_up"), self.segment("shared_down"),
                             sq.view(self._gate), router)

    def weights_of(self, name, expert, halves=False):
        """Expert `expert`'s rows of projection `name` as fp32 values (or, halves, their fp16 rounding); ids from the
        expert count on are the shared slices."""
        if expert >= self.e:
            name, expert = "shared_" + name, expert - self.e
        part = self.parts[name]
        rows = self.i if name.endswith("gate") or name.endswith("up") else self.h
        if halves:
            return part.halves[expert * rows:(expert + 1) * rows].view(np.float16).astype(np.float32)
        return part.values[expert * rows:(expert + 1) * rows]

    def shape(self, top_k):
        return sq.MoeShape(self.h, self.e, top_k, self.i, self.fmt, self.router, self.shared, int(self.gated))

    def route(self, x, scores, top_k):
        return oracle.route_select(scores, top_k, self.router, self.shared, x, self.scalar_gate)


def make_plan(shape, rows, phase):
    """prefill: MoE::prefillPlan with the policy's config; lanes: MoE::decodePlan(shape, rows / 8 lanes); decode: the
    rows entry (any 1..32 rows)."""
    plan = sq.MoePlan()
    if phase == "prefill":
        sq.call("sq_moe_prefill_plan", sq.byref(shape), rows, None, sq.byref(plan))
    elif phase == "lanes":
        assert rows % 8 == 0
        sq.call("sq_moe_decode_plan", sq.byref(shape), rows // 8, None, sq.byref(plan))
    else:
        sq.call("sq_moe_decode_rows_plan", sq.byref(shape), rows, sq.byref(plan))
    return plan


def run_moe(block, x, scores, top_k, residual=None, phase="prefill", verify=None):
    """One MoE layer as sq_moe_add_routing then sq_moe_add_routed (sq_moe_add's two halves). The caller's router
    scores go where the reference's router writes them: the grouped-input scratch, a row of the shape's router width
    per row (a block with router rows overwrites them); they are read back between the halves, before the routed
    work overwrites the grouped input with the input rows. Returns the plan, the scratch tensors and the bf16
    output."""
    t = torch()
    rows = x.shape[0]
    shape = block.shape(top_k)
    plan = make_plan(shape, rows, phase)
    scratch = {}
    for name in sq._MOE_WORKSPACE:
        nbytes = getattr(plan.workspace, name)
        scratch[name] = t.zeros(max(nbytes, 4) // 4 + 1, dtype=t.int32, device="cuda")
    width = sq.lib().sq_moe_router_width(sq.byref(shape))
    assert plan.workspace.grouped_input == max(rows * width * 4, rows * block.h * 2)
    padded = np.full(plan.workspace.grouped_input // 4, np.nan, np.float32)   # slots past the experts: unread
    padded[:rows * width].reshape(rows, width)[:, :block.e] = scores
    scratch["grouped_input"] = t.from_numpy(padded).cuda()
    ms = sq.MoeScratch(*[sq.view(scratch[n]) for n in sq._MOE_WORKSPACE])
    xin = to_device(x)
    res = to_device(residual) if residual is not None else None
    out = t.full((rows, block.h), -1, dtype=t.int16, device="cuda")
    vr = to_device(np.asarray(verify, np.uint32)) if verify is not None else None
    buffers = sq.MoeBuffers(sq.view(xin), sq.view(res), sq.view(out), ms, sq.view(vr))
    weights = block.weights()
    sq.call("sq_moe_add_routing", sq.stream_handle(), sq.byref(buffers), sq.byref(weights), sq.byref(plan))
    t.cuda.synchronize()
    scratch["scores"] = scratch["grouped_input"].cpu().numpy().view(np.float32)[:rows * width].reshape(
        rows, width)[:, :block.e].copy()
    sq.call("sq_moe_add_routed", sq.stream_handle(), sq.byref(buffers), sq.byref(weights), sq.byref(plan))
    t.cuda.synchronize()
    # The routed work leaves the input rows in the tiles' read order in the grouped input.
    table = to_host(scratch["grouped_input"], np.uint16)[:rows * block.h].reshape(rows, block.h // 32, 4, 2, 4)
    assert np.array_equal(table.transpose(0, 1, 3, 2, 4).reshape(rows, block.h), np.asarray(x, np.uint16))
    return plan, scratch, to_host(out, np.uint16)


def live_routes(rows, per_row, top_k, verify):
    """[rows][per_row] bool: the routes the grouping keeps (a verify step leaves the routed routes of rows past their
    lane's count out; the shared slices' routes always stay)."""
    live = np.ones((rows, per_row), bool)
    if verify is not None:
        dead = np.array([r % 8 >= verify[r // 8] for r in range(rows)])
        live[dead, :top_k] = False
    return live


def expected(block, x, selected, weights, residual, top_k=None, verify=None, staged=False):
    """The block's output from the routes' expert FFNs, expert by expert: fp64 products and sums (or, staged, the
    reference's staged numerics emulated: fp16 weights, fp32 products and sums) with the kernels' bf16 rounding
    points (gate and up, the SwiGLU intermediate, the expert output), then the residual plus the routing-weighted
    sum of the live routes."""
    dtype = np.float32 if staged else np.float64
    xf = synthetic.bf16_to_f32(x).astype(dtype)
    rows, per_row = selected.shape
    live = live_routes(rows, per_row, top_k if top_k is not None else per_row - block.shared, verify)
    out = np.zeros((rows, block.h))
    if residual is not None:
        out += synthetic.bf16_to_f32(residual)
    rb = lambda v: synthetic.bf16_to_f32(synthetic.bf16_bits(v.astype(np.float32))).astype(dtype)
    for e in np.unique(selected[live]):
        r_idx, s_idx = np.nonzero((selected == e) & live)
        w = lambda name: block.weights_of(name, e, staged).astype(dtype)
        g, u = rb(xf[r_idx] @ w("gate").T), rb(xf[r_idx] @ w("up").T)
        h = rb(u * (g / (1 + np.exp(-g.astype(np.float64))).astype(dtype)))
        y = rb(h @ w("down").T).astype(np.float64)
        np.add.at(out, r_idx, weights[r_idx, s_idx].astype(np.float64)[:, None] * y)
    return out


def errors(got, want):
    gotf = synthetic.bf16_to_f32(got).astype(np.float64)
    err = gotf - want
    return np.linalg.norm(err) / np.linalg.norm(want), err


@pytest.mark.parametrize("rows,experts,top_k", [(64, 32, 4), (6, 32, 4), (300, 16, 2), (1100, 32, 8), (1200, 32, 16)])
def test_moe_routed_experts(rows, experts, top_k):
    """Routing, grouping, expert passes and combine against the oracle: one chunk of rows, and past it the grouping's
    512-row chunks (1100 rows at top 8: three, the last ragged, its routes staged in LDS; 1200 rows at top 16: more
    routes than the LDS stage holds, read from the selection each chunk)."""
    rng = np.random.default_rng(rows + experts)
    hidden, intermediate = 512, 256
    block = Block(rng, experts, hidden, intermediate)
    x = synthetic.activations(rng, rows, hidden)
    scores = synthetic.router_logits(rng, rows, experts)
    scores[0, 3] = scores[0, 5] = scores[0].max() + 1   # a tie: the lower id ranks first
    residual = synthetic.bf16_bits(rng.uniform(-4, 4, (rows, hidden)).astype(np.float32))
    selected, _, _ = check_block(block, x, scores, top_k, residual)
    assert selected[0, 0] == 3 and selected[0, 1] == 5


def check_block(block, x, scores, top_k, residual, phase="prefill", weight_rtol=2e-6, verify=None, staged_check=False):
    """Runs the block and checks selection, weights, grouping and output against the oracle; returns the selection
    and the tile descriptors."""
    rows = x.shape[0]
    plan, scratch, got = run_moe(block, x, scores, top_k, residual, phase, verify)
    per_row = top_k + block.shared
    routes = rows * per_row
    sel_gpu = to_host(scratch["selected_experts"], np.uint32)[:routes].reshape(rows, per_row)
    w_gpu = scratch["routing_weights"].cpu().numpy().view(np.float32)[:routes].reshape(rows, per_row)
    selected, weights = block.route(x, scores, top_k)
    assert np.array_equal(sel_gpu, selected)
    finite = np.isfinite(weights)
    assert np.array_equal(np.isfinite(w_gpu), finite)
    assert np.allclose(w_gpu[finite], weights[finite], rtol=weight_rtol, atol=1e-7)
    tiles, grouped, route_rows = oracle.group_routes(selected, block.e, plan.tile_rows, block.shared, verify)
    count = to_host(scratch["tile_count"], np.uint32)
    assert count[0] == tiles.shape[0] <= plan.maximum_tiles
    gpu_tiles = to_host(scratch["tile_descriptors"], np.uint32)[: 2 * count[0]].reshape(-1, 2)
    assert np.array_equal(gpu_tiles, tiles)
    assert np.array_equal(to_host(scratch["grouped_routes"], np.uint32)[: grouped.size], grouped)
    assert np.array_equal(to_host(scratch["route_rows"], np.uint32)[:routes], route_rows)
    # rows whose routing weights are all finite (an all-NaN score row has none)
    ok = finite.all(axis=1)
    want = expected(block, x, selected, weights, residual, top_k, verify)[ok]
    rel, err = errors(got[ok], want)
    assert rel <= 1e-2, rel
    assert np.all(np.abs(err) <= np.ldexp(np.abs(want).max(axis=1, keepdims=True), -6))
    if staged_check:
        # no worse than the reference's staged expert tile (fp16 weights, fp32 sums), emulated on the CPU
        ref = expected(block, x, selected, weights, residual, top_k, verify, staged=True)[ok]
        ref_rel = np.linalg.norm(synthetic.bf16_to_f32(synthetic.bf16_bits(ref.astype(np.float32))) - want) / \
            np.linalg.norm(want)
        assert rel <= 1.10 * ref_rel + 1e-6, (rel, ref_rel)
    return sel_gpu, gpu_tiles, got


@pytest.mark.parametrize("fmt", [oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80,
                                 oracle.FMT_AF8G64])
@pytest.mark.parametrize("rows", [40, 6])
def test_moe_routed_formats(fmt, rows):
    """Every format through both expert-pass register budgets (tiles of 32 and of 16 rows)."""
    rng = np.random.default_rng(900 + fmt + rows)
    block = Block(rng, 16, 512, 256, fmt=fmt)
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 16)
    check_block(block, x, scores, 4, None, "prefill" if rows > 32 else "decode")


@pytest.mark.parametrize("rows,phase", [(48, "prefill"), (5, "decode")])
def test_moe_projections_in_formats_of_their_own(rows, phase):
    """Every projection in its own format (MoE.cpp:27-62): a routed gate and up of different formats (a gate pass and
    an up pass whose epilogue reads the gate), a shared pair likewise, and downs in others."""
    rng = np.random.default_rng(970 + rows)
    formats = {"gate": oracle.FMT_Q4K, "up": oracle.FMT_Q5K, "down": oracle.FMT_Q6K,
               "shared_gate": oracle.FMT_Q80, "shared_up": oracle.FMT_AF8G64, "shared_down": oracle.FMT_AF4G64}
    block = Block(rng, 16, 512, 256, fmt=oracle.FMT_Q4K, shared=1, gated=True, formats=formats)
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 16)
    residual = synthetic.bf16_bits(rng.uniform(-2, 2, (rows, 512)).astype(np.float32))
    check_block(block, x, scores, 4, residual, phase)


def test_moe_35b_formats():
    """The reference benchmark's 35B mix at a small width: Q4_K gate/up and Q5_K down experts, a gated Q8_0 shared
    expert, top 8 (gguf_moe_benchmark.mm:1-6; its F32 router is test_moe_router_projection's)."""
    rng = np.random.default_rng(990)
    block = Block(rng, 32, 512, 256, fmt=oracle.FMT_Q4K, shared=1, gated=True, shared_fmt=oracle.FMT_Q80,
                  formats={"down": oracle.FMT_Q5K})
    x = synthetic.activations(rng, 70, 512)
    scores = synthetic.router_logits(rng, 70, 32)
    check_block(block, x, scores, 8, None)


def test_moe_rows_independent_of_the_block():
    """A row's output is bitwise the same in any block: the 35B mix (its gated Q8_0 shared slice in launches of its
    own, whose few tiles run as 16-row halves) over 70 rows and over their first 24 (other expert tiles, other
    halves)."""
    rng = np.random.default_rng(991)
    block = Block(rng, 32, 512, 256, fmt=oracle.FMT_Q4K, shared=1, gated=True, shared_fmt=oracle.FMT_Q80,
                  formats={"down": oracle.FMT_Q5K})
    x = synthetic.activations(rng, 70, 512)
    scores = synthetic.router_logits(rng, 70, 32)
    _, _, whole = run_moe(block, x, scores, 8)
    _, _, first = run_moe(block, x[:24], scores[:24], 8)
    assert np.array_equal(whole[:24], first)


def test_moe_k_quant_experts_with_q8_0_shared_slice():
    """The mix the 4-bit MoE checkpoints ship: Q5_K routed experts with a gated Q8_0 shared slice (its own launches)."""
    rng = np.random.default_rng(950)
    block = Block(rng, 16, 512, 256, fmt=oracle.FMT_Q5K, shared=1, gated=True, shared_fmt=oracle.FMT_Q80)
    x = synthetic.activations(rng, 48, 512)
    scores = synthetic.router_logits(rng, 48, 16)
    residual = synthetic.bf16_bits(rng.uniform(-2, 2, (48, 512)).astype(np.float32))
    check_block(block, x, scores, 4, residual)


@pytest.mark.parametrize("rows,phase", [(48, "prefill"), (5, "decode")])
def test_moe_gated_shared_slice(rows, phase):
    """The reference's default routing: softmax over the top 4, one shared slice weighted sigmoid(x . g)."""
    rng = np.random.default_rng(500 + rows)
    block = Block(rng, 32, 512, 128, shared=1, gated=True)
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 32)
    residual = synthetic.bf16_bits(rng.uniform(-2, 2, (rows, 512)).astype(np.float32))
    check_block(block, x, scores, 4, residual, phase)


def test_moe_sigmoid_router_two_ungated_slices():
    """A sigmoid-normalised router with two ungated shared slices (weight 1 each), the second compiled routing."""
    rng = np.random.default_rng(600)
    block = Block(rng, 64, 512, 128, shared=2, router=oracle.ROUTER_SIGMOID_NORMALIZED)
    x = synthetic.activations(rng, 40, 512)
    scores = synthetic.router_logits(rng, 40, 64)
    check_block(block, x, scores, 6, None)


@pytest.mark.parametrize("shared_fmt,down_fmt", [(oracle.FMT_Q4K, oracle.FMT_Q4K), (oracle.FMT_AF4G128, oracle.FMT_AF4G32)])
def test_moe_shared_slices_in_their_own_formats(shared_fmt, down_fmt):
    """Shared gate/up and down in formats other than the routed experts' take launches of their own."""
    rng = np.random.default_rng(700 + shared_fmt + down_fmt)
    block = Block(rng, 16, 512, 256, shared=1, gated=True, shared_fmt=shared_fmt, down_fmt=down_fmt)
    x = synthetic.activations(rng, 70, 512)
    scores = synthetic.router_logits(rng, 70, 16)
    check_block(block, x, scores, 2, None)


def test_moe_decode_lane():
    """One decode lane through MoE::decodePlan(shape, 1 lane): 8 rows on 8-row tiles."""
    rng = np.random.default_rng(77)
    block = Block(rng, 64, 512, 128)
    x = synthetic.activations(rng, 8, 512)
    scores = synthetic.router_logits(rng, 8, 64)
    plan, _, got = run_moe(block, x, scores, 8, None, phase="lanes")
    assert plan.tile_rows == 8 and plan.rows == 8
    selected, weights = oracle.route_select(scores, 8)
    want = expected(block, x, selected, weights, None)
    err = synthetic.bf16_to_f32(got) - want
    assert np.linalg.norm(err) / np.linalg.norm(want) <= 1e-2


def test_moe_router_projection():
    """A block that carries its router's F32 rows projects the input onto them first (MoE::addRoutes): the scores
    lie within the fp32 accumulation bound of fp64, the selection and grouping follow from them as the oracle says,
    and the output is the one the same scores give when the caller supplies them."""
    rng = np.random.default_rng(808)
    block = Block(rng, 32, 512, 128, shared=1, gated=True)
    block.router_rows = rng.normal(0, 0.05, (32, 512)).astype(np.float32)
    rows = 44
    x = synthetic.activations(rng, rows, 512)
    plan, scratch, got = run_moe(block, x, np.zeros((rows, 32), np.float32), 4)
    scores = scratch["scores"].copy()
    exact, magnitude = oracle.float_rows_f64(x, block.router_rows)
    assert np.all(np.abs(scores - exact) <= (512 / 64 + 8) * 2.0 ** -24 * magnitude)
    per_row = 4 + 1
    sel_gpu = to_host(scratch["selected_experts"], np.uint32)[:rows * per_row].reshape(rows, per_row)
    selected, weights = block.route(x, scores, 4)
    assert np.array_equal(sel_gpu, selected)
    block.router_rows = None
    _, _, again = run_moe(block, x, scores, 4)
    assert np.array_equal(got, again)
    want = expected(block, x, selected, weights, None)
    err = synthetic.bf16_to_f32(got).astype(np.float64) - want
    assert np.linalg.norm(err) / np.linalg.norm(want) <= 1e-2


@pytest.mark.parametrize("router_rows,tile", [(False, sq.FLOAT_TILE_SIMDGROUP), (True, sq.FLOAT_TILE_SIMDGROUP),
                                              (True, sq.FLOAT_TILE_NEURAL_ACCELERATOR)])
def test_moe_add_routes(router_rows, tile):
    """MoE::addRoutes on its own (no plan, no grouping): with router rows it projects the input into the caller's
    scores (within the fp32 accumulation bound of fp64, on either float tile), then writes each row's top-k experts
    and its gated shared slice into the caller's selected and weight buffers: the selection bit for bit the oracle's
    on those scores, the weights within fp32 rounding; without router rows it routes the scores the caller wrote."""
    t = torch()
    rng = np.random.default_rng(909 + 2 * router_rows + tile)
    experts, hidden, top_k, rows = 64, 512, 6, 70
    block = Block(rng, experts, hidden, 128, shared=1, gated=True)
    shape = block.shape(top_k)
    width = sq.lib().sq_moe_router_width(sq.byref(shape))
    x = synthetic.activations(rng, rows, hidden)
    scores = np.full((rows, width), np.nan, np.float32)
    scores[:, :experts] = synthetic.router_logits(rng, rows, experts)
    scores_dev = to_device(scores)
    per_row = top_k + 1
    selected_dev = t.full((rows * per_row,), -1, dtype=t.int32, device="cuda")
    weights_dev = t.full((rows * per_row,), float("nan"), dtype=t.float32, device="cuda")
    gate_dev = to_device(block.scalar_gate)
    router = sq.Segment()
    if router_rows:
        rr = rng.normal(0, 0.05, (experts, hidden)).astype(np.float32)
        rr_dev = to_device(rr)
        router = sq.Segment(sq.view(rr_dev), sq.view(None), sq.view(None), experts, hidden, 0, sq.FLOAT32_ROWS)
    x_dev = to_device(x)
    sq.call("sq_moe_add_routes", sq.stream_handle(), sq.view(x_dev), sq.byref(router), sq.view(gate_dev),
            sq.view(scores_dev), sq.view(selected_dev), sq.view(weights_dev), rows, sq.byref(shape), tile)
    t.cuda.synchronize()
    got_scores = scores_dev.cpu().numpy()[:, :experts]
    if router_rows:
        exact, magnitude = oracle.float_rows_f64(x, rr)
        assert np.all(np.abs(got_scores - exact) <= (hidden / 64 + 8) * 2.0 ** -24 * magnitude)
    else:
        assert np.array_equal(got_scores, scores[:, :experts])
    selected, weights = block.route(x, got_scores, top_k)
    assert np.array_equal(to_host(selected_dev, np.uint32).reshape(rows, per_row), selected)
    np.testing.assert_allclose(weights_dev.cpu().numpy().reshape(rows, per_row), weights, rtol=2e-6, atol=1e-7)


def test_moe_nan_score_rows():
    """Rows of NaN router scores (an upstream NaN through the router projection): a NaN never wins, an all-NaN row
    selects expert 0 at every rank as the reference's kernel does, every selected id stays a valid expert, and the
    grouping and the other rows' outputs are the oracle's."""
    rng = np.random.default_rng(4242)
    block = Block(rng, 32, 512, 128)
    rows = 40
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 32)
    scores[3] = np.nan
    scores[7, ::2] = np.nan
    scores[11, :20] = -np.inf
    selected, _, got = check_block(block, x, scores, 4, None)
    assert selected[3].tolist() == [0, 0, 0, 0]
    assert np.all(selected < 32)
    assert np.all(selected[7] % 2 == 1)


@pytest.mark.parametrize("shared", [0, 1])
def test_moe_verify_rows(shared):
    """A verify step (MoeBuffers::verifyRows, MoE.cpp:467-475): two lanes of 8 rows with 3 and 8 live rows. The
    grouping is the oracle's verified grouping bit for bit (the dead rows' routed routes in no tile, their route rows
    ~0u), and a dead row's output is its residual plus its shared slices' routes only: without a shared expert,
    exactly its residual."""
    rng = np.random.default_rng(31 + shared)
    block = Block(rng, 16, 512, 256, shared=shared, gated=bool(shared))
    rows = 16
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 16)
    residual = synthetic.bf16_bits(rng.uniform(-2, 2, (rows, 512)).astype(np.float32))
    verify = [3, 8]
    _, tiles, got = check_block(block, x, scores, 4, residual, "lanes", verify=verify)
    assert tiles[:, 1].sum() == (3 + 8) * 4 + shared * rows
    dead = got[3:8]
    if not shared:
        assert np.array_equal(dead, residual[3:8])
    else:
        assert not np.array_equal(dead, residual[3:8])
    # every row live: the plain grouping
    check_block(block, x, scores, 4, residual, "lanes", verify=[8, 8])


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_AF4G32, oracle.FMT_AF4G128, oracle.FMT_Q4K,
                                 oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64])
def test_moe_tall_tiles_every_format(fmt):
    """Router scores skewed towards four experts give them tiles of more than 16 rows (the two-row-block body of the
    expert passes), in every format, in the one-pass gate/up pair (two tensors a wave) and the down pass (one)."""
    rng = np.random.default_rng(1300 + fmt)
    block = Block(rng, 16, 512, 256, fmt=fmt)
    rows = 64
    x = synthetic.activations(rng, rows, 512)
    scores = synthetic.router_logits(rng, rows, 16)
    scores[:, :4] += 4.0
    _, tiles, _ = check_block(block, x, scores, 4, None)
    assert tiles[:, 1].max() > 16 and np.count_nonzero(tiles[:, 1] > 16) >= 4


def test_moe_config4_block():
    """BASELINE config 4 at full size: 128 experts, top 8 of softmax(N(0,1) logits), hidden 2048, intermediate 768,
    512 tokens, MLX affine 4-bit group 64, on the prefill plan (32-row tiles, about 250 of them, dispatched longest
    first). Every row of the output against fp64 within BASELINE's tolerances, and no worse than the reference's
    staged expert numerics emulated on the CPU."""
    rng = np.random.default_rng(4096)
    block = Block(rng, 128, 2048, 768, device_repack=True)
    rows = 512
    x = synthetic.activations(rng, rows, 2048)
    scores = synthetic.router_logits(rng, rows, 128)
    _, tiles, _ = check_block(block, x, scores, 8, None, staged_check=True)
    assert tiles.shape[0] > 128 and tiles[:, 1].max() > 16
