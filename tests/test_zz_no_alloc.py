"""sq_linear_add_static, the entry point that allocates nothing, through the C ABI: its outputs equal
sq_linear_add's bit for bit (the same plans and kernels; only the scratch differs) for split decode plans (partials
and counters), one- and two-pass gate/up pairs (doubled partials, the gate scratch), prefill plans (the fp16 table
and row scales; a halved-K plan's fp32 partials) and the epilogues that read a caller operand (the residual, and an
up-with-gate plan's gate, which stays the caller's buffer), on two calls in a row of which the second is smaller, so
stale contents of the shared static array from the first call must not matter."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import DeviceAffine, Run, dense_inputs, make_weights, to_device, torch
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


def run_both(plan, proj, x, n, gate=None, operand=None):
    """(sq_linear_add output, sq_linear_add_static output) of the same plan and inputs, bf16 bits. operand: the bf16
    [rows][n] residual of a RESIDUAL plan or gate of an UP_WITH_GATE plan, handed to both entry points."""
    t = torch()
    run = Run(plan, n, x)
    epilogue = plan.workload.epilogue
    aux = None
    if operand is not None:
        padded = np.zeros((run.rows, n), np.uint16)
        padded[: operand.shape[0]] = operand
        aux = to_device(padded)
    residual = aux if epilogue == sq.EPILOGUE_RESIDUAL else None
    gate_operand = aux if epilogue == sq.EPILOGUE_UP_WITH_GATE else run.scratch.gate
    sq.linear_add(plan, proj, run.x, run.out, residual=residual, gate_scratch=gate_operand,
                  scratch=run.scratch.struct(), gate=gate)
    t.cuda.synchronize()
    want = run.output()[: x.shape[0]].copy()
    out = t.full((run.rows, n), -1, dtype=t.int16, device="cuda")
    # The caller's own scratch views stay null: the static entry point needs none. Only an up-with-gate plan's gate
    # operand is the caller's.
    buffers = sq.LinearBuffers(sq.view(run.x), sq.view(out), sq.view(residual),
                               sq.view(aux if epilogue == sq.EPILOGUE_UP_WITH_GATE else None), sq.LinearScratch())
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


def test_static_epilogue_operands_then_smaller():
    """An up-with-gate prefill multiplies in the caller's gate operand (not a static region), and a residual decode
    and prefill add the caller's residual: bitwise sq_linear_add's, at 300 rows then 40 (the staged and prefill tiles
    of the up-with-gate plan), and at 16 then 3 rows for the residual decode."""
    rng = np.random.default_rng(75)
    n, k = 512, 2048
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    proj = sq.projection(w.segment())
    for rows in (300, 40, 20):
        x = dense_inputs(rng, rows, k)
        gate = synthetic.bf16_bits(rng.uniform(-4, 4, (rows, n)).astype(np.float32))
        plan = sq.plan_for(sq.prefill_workload(n, k, rows, sq.EPILOGUE_UP_WITH_GATE), proj)
        want, got = run_both(plan, proj, x, n, operand=gate)
        assert np.array_equal(got, want), ("up with gate", rows)
        residual = synthetic.bf16_bits(rng.uniform(-64, 64, (rows, n)).astype(np.float32))
        plan = sq.plan_for(sq.prefill_workload(n, k, rows, sq.EPILOGUE_RESIDUAL), proj)
        want, got = run_both(plan, proj, x, n, operand=residual)
        assert np.array_equal(got, want), ("prefill residual", rows)
    for rows in (16, 3):
        x = dense_inputs(rng, rows, k)
        residual = synthetic.bf16_bits(rng.uniform(-64, 64, (rows, n)).astype(np.float32))
        want, got = run_both(staged(n, k, rows, 4, sq.EPILOGUE_RESIDUAL), proj, x, n, operand=residual)
        assert np.array_equal(got, want), ("decode residual", rows)


def test_static_halved_prefill_then_smaller():
    """A prefill whose tiles' K is halved (16384 x 3072 at 40 rows, then 33: 64 tiles of 256 columns, each cut
    between two workgroups whose fp32 halves a close dispatch adds) takes its partials from the static array: bitwise
    sq_linear_add's."""
    rng = np.random.default_rng(76)
    n, k = 16384, 3072
    w = DeviceAffine(rng, n, k)
    proj = sq.projection(w.segment())
    for rows in (40, 33):
        plan = sq.plan_for(sq.prefill_workload(n, k, rows), proj)
        size, _ = sq.scratch_size(plan)
        assert plan.config.tile == sq.TILE_PREFILL and size.partials == 2 * rows * n * 4, "the plan halves K"
        x = dense_inputs(rng, rows, k)
        want, got = run_both(plan, proj, x, n)
        assert np.array_equal(got, want), rows
