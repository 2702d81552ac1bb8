"""sq_linear_add_static, the entry point that allocates nothing, through the C ABI: its outputs equal
sq_linear_add's bit for bit (the same plans and kernels; only the scratch differs) for split decode plans (partials
and counters), one- and two-pass gate/up pairs (doubled partials, the gate scratch) and a prefill plan (the fp16
table and row scales), on two calls in a row of which the second is smaller, so stale contents of the shared static
array from the first call must not matter."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import Run, dense_inputs, make_weights, to_device, torch

pytestmark = pytest.mark.gpu


def run_both(plan, proj, x, n, gate=None):
    """(sq_linear_add output, sq_linear_add_static output) of the same plan and inputs, bf16 bits."""
    t = torch()
    run = Run(plan, n, x)
    gs = run.scratch.gate
    sq.linear_add(plan, proj, run.x, run.out, gate_scratch=gs, scratch=run.scratch.struct(), gate=gate)
    t.cuda.synchronize()
    want = run.output()[: x.shape[0]].copy()
    out = t.full((run.rows, n), -1, dtype=t.int16, device="cuda")
    # The caller's own scratch views stay null: the static entry point needs none.
    buffers = sq.LinearBuffers(sq.view(run.x), sq.view(out), sq.view(None), sq.view(None), sq.LinearScratch())
    sq.call("sq_linear_add_static", sq.stream_handle(), sq.byref(buffers), sq.byref(proj), sq.byref(plan),
            sq.byref(gate) if gate else None)
    t.cuda.synchronize()
    return want, out.cpu().numpy().view(np.uint16)[: x.shape[0]]


def staged(n, k, rows, splits, epilogue=sq.EPILOGUE_NONE, one_pass=0):
    return sq.plan_config(sq.decode_workload(n, k, rows, epilogue),
                          sq.LinearConfig(sq.TILE_STAGED, splits, 0, one_pass, 0), sq.OUTPUT_BF16)


def test_static_split_decode_then_smaller():
    rng = np.random.default_rng(71)
    w = make_weights(rng, oracle.FMT_AF4G64, 1024, 8192)
    proj = sq.projection(w.segment())
    for rows, splits in ((16, 8), (2, 4)):    # the second call is smaller: fewer rows, fewer partials
        x = dense_inputs(rng, rows, 8192)
        want, got = run_both(staged(1024, 8192, rows, splits), proj, x, 1024)
        assert np.array_equal(got, want), (rows, splits)
    small = make_weights(rng, oracle.FMT_Q4K, 256, 2048)
    x = dense_inputs(rng, 3, 2048)
    want, got = run_both(staged(256, 2048, 3, 2), sq.projection(small.segment()), x, 256)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("one_pass", [1, 0])
def test_static_gate_up_pair(one_pass):
    rng = np.random.default_rng(72 + one_pass)
    n, k = 512, 4096
    wg, wu = make_weights(rng, oracle.FMT_AF4G64, n, k), make_weights(rng, oracle.FMT_AF4G64, n, k)
    gate, up = sq.projection(wg.segment()), sq.projection(wu.segment())
    for rows in (8, 1):
        x = dense_inputs(rng, rows, k)
        want, got = run_both(staged(n, k, rows, 4, sq.EPILOGUE_GATE_UP, one_pass), up, x, n, gate=gate)
        assert np.array_equal(got, want), rows


def test_static_prefill_then_smaller():
    rng = np.random.default_rng(74)
    w = make_weights(rng, oracle.FMT_AF4G64, 512, 2048)
    proj = sq.projection(w.segment())
    for rows in (300, 40):
        x = dense_inputs(rng, rows, 2048)
        plan = sq.plan_for(sq.prefill_workload(512, 2048, rows), proj)
        assert plan.config.tile == sq.TILE_PREFILL
        want, got = run_both(plan, proj, x, 512)
        assert np.array_equal(got, want), rows
