"""MoE routed experts through the C ABI against the oracle (kernels/shared/moe.metal, moe_gguf.metal): the top-k
selection bit for bit (ties to the lower expert id), the renormalised softmax weights, the grouping (tiles in expert
order, each expert's routes in route order, padding marked ~0u), and the combined output against an fp64 SwiGLU of
every route with the kernels' bf16 rounding points, within BASELINE's tolerances."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import affine_native, to_device, to_host, torch
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


class Block:
    def __init__(self, rng, experts, hidden, intermediate, fmt=oracle.FMT_AF4G64):
        self.e, self.h, self.i, self.fmt = experts, hidden, intermediate, fmt
        self.parts = {}
        for name, n, k in (("gate", experts * intermediate, hidden), ("up", experts * intermediate, hidden),
                           ("down", experts * hidden, intermediate)):
            native = affine_native(rng, fmt, n, k)
            p0, meta, values = oracle.repack(fmt, native, n, k)
            self.parts[name] = (to_device(p0), to_device(meta), values, n, k)
        self.slots = to_device(np.arange(experts, dtype=np.uint32))

    def segment(self, name):
        p0, meta, _, n, k = self.parts[name]
        return sq.segment(self.fmt, n, k, p0, meta)

    def weights(self):
        return sq.MoeWeights(self.segment("gate"), self.segment("up"), self.segment("down"), sq.view(self.slots), self.e)

    def values(self, name, expert):
        _, _, v, n, k = self.parts[name]
        rows = self.i if name != "down" else self.h
        return v[expert * rows:(expert + 1) * rows]


def run_moe(block, x, scores, top_k, residual=None, phase="prefill"):
    t = torch()
    rows = x.shape[0]
    shape = sq.MoeShape(block.h, block.e, top_k, block.i, block.fmt)
    plan = sq.MoePlan()
    sq.call("sq_moe_prefill_plan" if phase == "prefill" else "sq_moe_decode_plan", sq.byref(shape), rows, sq.byref(plan))
    scratch = {}
    for name in sq._MOE_WORKSPACE:
        nbytes = getattr(plan.workspace, name)
        scratch[name] = t.zeros(max(nbytes, 4) // 4 + 1, dtype=t.int32, device="cuda")
    ms = sq.MoeScratch(*[sq.view(scratch[n]) if getattr(plan.workspace, n) else sq.Buffer(None, 0)
                         for n in sq._MOE_WORKSPACE])
    xin, sc = to_device(x), t.from_numpy(np.ascontiguousarray(scores)).cuda()
    res = to_device(residual) if residual is not None else None
    out = t.full((rows, block.h), -1, dtype=t.int16, device="cuda")
    buffers = sq.MoeBuffers(sq.view(xin), sq.view(sc), sq.view(res), sq.view(out), 0, ms)
    sq.call("sq_moe_add", sq.stream_handle(), sq.byref(buffers), sq.byref(block.weights()), sq.byref(plan))
    t.cuda.synchronize()
    return plan, scratch, to_host(out, np.uint16)


def expected(block, x, selected, weights, residual):
    xf = synthetic.bf16_to_f32(x).astype(np.float64)
    rows = x.shape[0]
    out = np.zeros((rows, block.h))
    if residual is not None:
        out += synthetic.bf16_to_f32(residual)
    for r in range(rows):
        for s, e in enumerate(selected[r]):
            g = block.values("gate", e).astype(np.float64) @ xf[r]
            u = block.values("up", e).astype(np.float64) @ xf[r]
            gb, ub = synthetic.bf16_to_f32(synthetic.bf16_bits(g)), synthetic.bf16_to_f32(synthetic.bf16_bits(u))
            h = synthetic.bf16_to_f32(synthetic.bf16_bits(ub * (gb / (1 + np.exp(-gb.astype(np.float64))))))
            y = block.values("down", e).astype(np.float64) @ h.astype(np.float64)
            out[r] += weights[r, s] * synthetic.bf16_to_f32(synthetic.bf16_bits(y))
    return out


@pytest.mark.parametrize("rows,experts,top_k", [(64, 32, 4), (6, 32, 4), (300, 16, 2)])
def test_moe_routed_experts(rows, experts, top_k):
    rng = np.random.default_rng(rows + experts)
    hidden, intermediate = 512, 256
    block = Block(rng, experts, hidden, intermediate)
    x = synthetic.activations(rng, rows, hidden)
    scores = synthetic.router_logits(rng, rows, experts)
    scores[0, 3] = scores[0, 5] = scores[0].max() + 1   # a tie: the lower id ranks first
    residual = synthetic.bf16_bits(rng.uniform(-4, 4, (rows, hidden)).astype(np.float32))
    plan, scratch, got = run_moe(block, x, scores, top_k, residual)
    routes = rows * top_k
    sel_gpu = to_host(scratch["selected_experts"], np.uint32)[:routes].reshape(rows, top_k)
    w_gpu = scratch["routing_weights"].cpu().numpy().view(np.float32)[:routes].reshape(rows, top_k)
    selected, weights = oracle.route_select(scores, top_k)
    assert np.array_equal(sel_gpu, selected)
    assert sel_gpu[0, 0] == 3 and sel_gpu[0, 1] == 5
    assert np.allclose(w_gpu, weights, rtol=2e-6, atol=1e-7)
    tiles, grouped, route_rows = oracle.group_routes(selected, experts, plan.tile_rows)
    count = to_host(scratch["tile_count"], np.uint32)
    assert count[0] == tiles.shape[0]
    assert np.array_equal(to_host(scratch["tile_descriptors"], np.uint32)[: 2 * count[0]].reshape(-1, 2), tiles)
    assert np.array_equal(to_host(scratch["grouped_routes"], np.uint32)[: grouped.size], grouped)
    assert np.array_equal(to_host(scratch["route_rows"], np.uint32)[:routes], route_rows)
    want = expected(block, x, selected, weights, residual)
    gotf = synthetic.bf16_to_f32(got).astype(np.float64)
    err = gotf - want
    assert np.linalg.norm(err) / np.linalg.norm(want) <= 1e-2
    assert np.all(np.abs(err) <= np.ldexp(np.abs(want).max(axis=1, keepdims=True), -6))


def test_moe_decode_rows():
    rng = np.random.default_rng(77)
    block = Block(rng, 64, 512, 128)
    x = synthetic.activations(rng, 8, 512)
    scores = synthetic.router_logits(rng, 8, 64)
    plan, _, got = run_moe(block, x, scores, 8, None, phase="decode")
    assert plan.tile_rows == 8
    selected, weights = oracle.route_select(scores, 8)
    want = expected(block, x, selected, weights, None)
    err = synthetic.bf16_to_f32(got) - want
    assert np.linalg.norm(err) / np.linalg.norm(want) <= 1e-2
