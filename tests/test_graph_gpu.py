"""Captured HIP graphs replay what eager dispatches compute. Each path that keeps state on the device between its
dispatches is captured once and replayed several times, with other eager work on the same scratch and a
synchronisation between replays, and every replay's output is compared bitwise with the eager one:
  - a decode plan's K-split partials and counters (the last workgroup of a tile returns its counter to zero);
  - a halved-K prefill's partials and close dispatch;
  - a stream prefill's partial slots and counters (the last piece of a tile returns its counter to zero);
  - the MoE block, router projection to combine (routes, tiles and their counts written and read on the device);
  - the static entry point, whose counters a fill kernel clears (a kernel node, not a memset node, in the graph)."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import Run, dense_inputs, make_weights, to_device, torch
from splash_q4 import synthetic
from test_moe_gpu import Block, make_plan

pytestmark = pytest.mark.gpu


def current_stream():
    return torch().cuda.current_stream().cuda_stream


def replays_match(launch, out, disturb, replays=4):
    """launch(stream) issues one call's dispatches on the stream of handle `stream`, writing `out`. Runs it eagerly,
    captures it in a graph on a side stream, then replays the graph `replays` times: before each replay `out` is
    poisoned and `disturb()` runs other eager work (which leaves the shared scratch as every call leaves it), and
    after each the output must equal the eager one bit for bit."""
    t = torch()
    launch(current_stream())
    t.cuda.synchronize()
    want = out.clone()
    side = t.cuda.Stream()
    graph = t.cuda.CUDAGraph()
    with t.cuda.graph(graph, stream=side):
        launch(current_stream())
    for i in range(replays):
        out.fill_(-1)
        disturb()
        t.cuda.synchronize()
        graph.replay()
        t.cuda.synchronize()
        assert t.equal(out, want), f"replay {i} differs from the eager call"
    del graph


def linear_case(plan, proj, n, rows, k, rng, static=False):
    """A projection call and a disturbing call of the same plan on other inputs, both on one scratch."""
    t = torch()
    main, other = Run(plan, n, dense_inputs(rng, rows, k)), Run(plan, n, dense_inputs(rng, rows, k))
    scratch = main.scratch.struct()

    def call(run, stream):
        if static:
            buffers = sq.LinearBuffers(sq.view(run.x), sq.view(run.out), sq.view(None), sq.view(None),
                                       sq.LinearScratch())
            sq.call("sq_linear_add_static", sq.c_void_p(stream), sq.byref(buffers), sq.byref(proj), sq.byref(plan),
                    None)
        else:
            sq.linear_add(plan, proj, run.x, run.out, scratch=scratch, stream=sq.c_void_p(stream))

    replays_match(lambda s: call(main, s), main.out, lambda: call(other, current_stream()))
    assert t.any(main.out != -1)


def test_graph_split_decode():
    rng = np.random.default_rng(90)
    w = make_weights(rng, oracle.FMT_AF4G64, 1024, 8192)
    plan = sq.plan_config(sq.decode_workload(1024, 8192, 16), sq.LinearConfig(sq.TILE_STAGED, 8, 0, 0, 0))
    linear_case(plan, sq.projection(w.segment()), 1024, 16, 8192, rng)


def test_graph_static_split_decode():
    rng = np.random.default_rng(91)
    w = make_weights(rng, oracle.FMT_AF4G64, 1024, 8192)
    plan = sq.plan_config(sq.decode_workload(1024, 8192, 16), sq.LinearConfig(sq.TILE_STAGED, 8, 0, 0, 0))
    linear_case(plan, sq.projection(w.segment()), 1024, 16, 8192, rng, static=True)


def test_graph_halved_prefill():
    rng = np.random.default_rng(92)
    n, k, rows = 4096, 4096, 1800
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.prefill_workload(n, k, rows), proj)
    size, _ = sq.scratch_size(plan)
    assert size.partials == 2 * rows * n * 4 and size.counters == 0, "the plan halves K"
    linear_case(plan, proj, n, rows, k, rng)


def test_graph_stream_prefill():
    rng = np.random.default_rng(93)
    n, k, rows = 24576, 1280, 1024
    w = make_weights(rng, oracle.FMT_Q4K, n, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.prefill_workload(n, k, rows), proj)
    size, _ = sq.scratch_size(plan)
    assert size.partials > 0 and size.counters > 0, "the plan runs stream pieces"
    linear_case(plan, proj, n, rows, k, rng)


def test_graph_moe_block():
    """sq_moe_add with the block's own F32 router: 16 experts, top 4 of 160 rows (tiles of more and fewer than 16
    rows), a gated shared slice."""
    t = torch()
    rng = np.random.default_rng(94)
    block = Block(rng, 16, 512, 128, shared=1, gated=True)
    block.router_rows = rng.normal(0, 0.05, (16, 512)).astype(np.float32)
    rows, top_k = 160, 4
    shape = block.shape(top_k)
    plan = make_plan(shape, rows, "prefill")
    weights = block.weights()
    scratch = {name: t.zeros(max(getattr(plan.workspace, name), 4) // 4 + 1, dtype=t.int32, device="cuda")
               for name in sq._MOE_WORKSPACE}
    ms = sq.MoeScratch(*[sq.view(scratch[name]) for name in sq._MOE_WORKSPACE])

    def buffers(x):
        out = t.full((rows, block.h), -1, dtype=t.int16, device="cuda")
        return out, sq.MoeBuffers(sq.view(x), sq.view(None), sq.view(out), ms, sq.view(None))

    x_main = to_device(synthetic.activations(rng, rows, block.h))
    x_other = to_device(synthetic.activations(rng, rows, block.h))
    out, main = buffers(x_main)
    out_other, other = buffers(x_other)   # kept alive while `other` points at it
    call = lambda bufs, stream: sq.call("sq_moe_add", sq.c_void_p(stream), sq.byref(bufs), sq.byref(weights),
                                        sq.byref(plan))
    replays_match(lambda s: call(main, s), out, lambda: call(other, current_stream()))
    assert t.any(out != -1)
