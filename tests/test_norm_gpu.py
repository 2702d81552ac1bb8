"""The producers either side of the projections through the C ABI: the RMS norm (Normalization::addRms) against the
reference's own acceptance (every output the fp64 norm rounded once to bf16, dev/tests/engine/NormReference.hpp),
its prefill table bit for bit against the oracle's and as the prefill tile's prepared input, and the float
projection of F32 and BF16 rows (addGgufFloat, the MoE router's) against fp64 within its accumulation bound."""
import ctypes

import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import make_weights, to_device, to_host, torch
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


def norm_weights(rng, width, f32):
    values = rng.uniform(0.25, 2.0, width).astype(np.float32)
    if f32:
        return to_device(values), values.astype(np.float64)
    bits = synthetic.bf16_bits(values)
    return to_device(bits), synthetic.bf16_to_f32(bits).astype(np.float64)


def run_norm(x_bits, w_dev, f32, width, layout=sq.LINEAR_INPUT_PLAIN, storage_rows=None):
    """The norm of x_bits' rows into an output of storage_rows rows (a prefill plan's input holds its storage rows)."""
    t = torch()
    rows = x_bits.shape[0]
    x = to_device(x_bits)
    out = t.zeros((storage_rows or rows, width), dtype=t.int16, device="cuda")
    table = t.zeros((storage_rows or rows, width), dtype=t.int16, device="cuda")
    sums = t.zeros(storage_rows or rows, dtype=t.float32, device="cuda")
    scratch = sq.LinearScratch(sq.view(table), sq.view(sums), sq.view(None), sq.view(None), sq.view(None))
    prepared = sq.PreparedInput()
    sq.call("sq_norm_add_rms", sq.stream_handle(), sq.view(x), ctypes.byref(sq.NormWeights(sq.view(w_dev), int(f32))),
            sq.view(out), width, rows, ctypes.byref(scratch), layout, ctypes.byref(prepared))
    t.cuda.synchronize()
    return out, table, sums, prepared


@pytest.mark.parametrize("width,f32", [(2048, False), (5120, True), (4096, False), (17408, True)])
def test_rms_norm_rounded_once(width, f32):
    rng = np.random.default_rng(width + f32)
    rows = 9
    x = rng.standard_normal((rows, width)).astype(np.float32)
    x[1] *= 3e4                     # a row past half's range
    x[2] *= 1e-3                    # a small one
    x[3, ::7] = 0.0
    bits = synthetic.bf16_bits(x)
    w_dev, w = norm_weights(rng, width, f32)
    out, _, _, prepared = run_norm(bits, w_dev, f32, width)
    assert prepared.layout == sq.LINEAR_INPUT_PLAIN
    got = to_host(out, np.uint16)
    exact = oracle.rms_norm_f64(bits, w)
    ok = oracle.rounded_once_to_bf16(got, exact)
    assert ok.all(), f"{(~ok).sum()} outputs not the fp64 norm rounded once"


@pytest.mark.parametrize("width,rows", [(4096, 300), (2048, 5)])
def test_rms_norm_writes_prefill_table(width, rows):
    """With the half-rows layout the norm also writes the prefill table of its own output: the oracle's table of
    the output bits, bit for bit, and the row scales."""
    rng = np.random.default_rng(31 + rows)
    x = rng.standard_normal((rows, width)).astype(np.float32)
    x[0] *= 5e4
    bits = synthetic.bf16_bits(x)
    w_dev, _ = norm_weights(rng, width, False)
    out, table, sums, prepared = run_norm(bits, w_dev, False, width, sq.LINEAR_INPUT_HALF_ROWS)
    assert prepared.layout == sq.LINEAR_INPUT_HALF_ROWS and prepared.source.ptr == out.data_ptr()
    want_table, want_scale = oracle.half_rows(to_host(out, np.uint16))
    assert table.shape[0] == rows
    assert np.array_equal(to_host(table, np.uint16), want_table)
    assert np.array_equal(sums.cpu().numpy(), want_scale)


@pytest.mark.parametrize("scale", [1e-5, 1e-6, 1e-8])
def test_norm_table_of_small_rows(scale):
    """Norm weights of scale x U(0.25, 2) make output rows of that magnitude: the table the norm writes of them is the
    oracle's bit for bit (scaled up into half's normal range, not left as half subnormals), and a prefill that takes
    it keeps every output inside its fp64 interval, as good as the staged emulation."""
    t = torch()
    rng = np.random.default_rng(int(-np.log10(scale)))
    rows, k, n = 96, 2048, 256
    x = synthetic.activations(rng, rows, k)
    w_bits = synthetic.bf16_bits(rng.uniform(0.25, 2.0, k).astype(np.float32) * np.float32(scale))
    w = make_weights(rng, sq.FMT_AF4G64, n, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.prefill_workload(n, k, rows), proj)
    normalized, table, sums, prepared = run_norm(x, to_device(w_bits), False, k, sq.LINEAR_INPUT_HALF_ROWS,
                                                 plan.storage_rows)
    out_bits = to_host(normalized, np.uint16)[:rows]
    want_table, want_scale = oracle.half_rows(out_bits)
    assert np.array_equal(to_host(table, np.uint16)[:rows], want_table)
    assert np.array_equal(sums.cpu().numpy()[:rows], want_scale)
    assert np.all(want_scale < 2.0 ** -10), "small rows are scaled up"
    scratch = sq.LinearScratch(sq.view(table), sq.view(sums), sq.view(None), sq.view(None), sq.view(None))
    got = t.zeros((plan.storage_rows, n), dtype=t.int16, device="cuda")
    buffers = sq.LinearBuffers(sq.view(normalized), sq.view(got), sq.view(None), sq.view(None), scratch, prepared)
    sq.call("sq_linear_add", sq.stream_handle(), ctypes.byref(buffers), ctypes.byref(proj), ctypes.byref(plan), None)
    t.cuda.synchronize()
    from helpers import check_projection, staged_reference
    stats = check_projection(to_host(got, np.uint16)[:rows], out_bits, w, f"norm table x {scale}")
    value, *_ = oracle.project_f64(out_bits, w.values)
    ref = synthetic.bf16_to_f32(staged_reference(out_bits, w))
    assert stats["rel_l2"] <= 1.10 * np.linalg.norm(ref - value) / np.linalg.norm(value) + 1e-6


def test_prefill_takes_the_norm_table():
    """A prefill plan whose buffers say the scratch holds its input's table skips its own preparation: it gives the
    same bits as a prefill that prepares, even after the input rows are overwritten, and reports the table."""
    t = torch()
    rng = np.random.default_rng(41)
    rows, k, n = 300, 2048, 512
    w = make_weights(rng, sq.FMT_AF4G64, n, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.prefill_workload(n, k, rows), proj)
    layout = ctypes.c_uint32()
    sq.call("sq_linear_plan_input", ctypes.byref(plan), ctypes.byref(layout))
    assert layout.value == sq.LINEAR_INPUT_HALF_ROWS
    bits = synthetic.activations(rng, rows, k)
    w_dev, _ = norm_weights(rng, k, False)
    normalized, table, sums, prepared = run_norm(bits, w_dev, False, k, sq.LINEAR_INPUT_HALF_ROWS, plan.storage_rows)
    scratch = sq.LinearScratch(sq.view(table), sq.view(sums), sq.view(None), sq.view(None), sq.view(None))
    want = t.zeros((plan.storage_rows, n), dtype=t.int16, device="cuda")
    sq.linear_add(plan, proj, normalized, want, scratch=scratch)            # prepares its own table
    t.cuda.synchronize()
    normalized2, table, sums, prepared = run_norm(bits, w_dev, False, k, sq.LINEAR_INPUT_HALF_ROWS, plan.storage_rows)
    assert t.equal(normalized2, normalized)
    scratch = sq.LinearScratch(sq.view(table), sq.view(sums), sq.view(None), sq.view(None), sq.view(None))
    normalized2.fill_(0x7F00)       # the table still holds the rows; the rows themselves are gone
    got = t.zeros_like(want)
    after = sq.PreparedInput()
    buffers = sq.LinearBuffers(sq.view(normalized2), sq.view(got), sq.view(None), sq.view(None), scratch, prepared)
    sq.call("sq_linear_add_prepared", sq.stream_handle(), ctypes.byref(buffers), ctypes.byref(proj),
            ctypes.byref(plan), None, ctypes.byref(after))
    t.cuda.synchronize()
    assert t.equal(got[:rows], want[:rows])
    assert after.layout == sq.LINEAR_INPUT_HALF_ROWS and after.source.ptr == normalized2.data_ptr()


@pytest.mark.parametrize("f32_rows,f32_out,rows,n,tile", [
    (True, True, 37, 128, None), (False, True, 37, 128, None), (True, False, 37, 128, None),
    (True, True, 300, 128, None), (False, True, 2048, 128, None), (True, False, 97, 60, None),
    (True, True, 13, 60, sq.FLOAT_TILE_NEURAL_ACCELERATOR), (False, False, 300, 128, sq.FLOAT_TILE_SIMDGROUP)])
def test_float_rows(f32_rows, f32_out, rows, n, tile):
    """The policy's tile (sq_linear_float_tile): 37 rows run the lane chains, 64 and more the fp32 MFMA (32 x 32 tiles,
    ragged in rows and columns at 97 x 60); and each tile where the policy would take the other (the MFMA at 13 rows,
    the lane chains at 300); all within the lane chains' rounding bound."""
    t = torch()
    rng = np.random.default_rng(51 + 2 * f32_rows + f32_out + rows)
    k, stride, offset = 2048, 136, 5
    x = synthetic.activations(rng, rows, k)
    values = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    if f32_rows:
        w_dev, w = to_device(values), values
        seg = sq.Segment(sq.view(w_dev), sq.view(None), sq.view(None), n, k, 0, sq.FLOAT32_ROWS)
    else:
        wb = synthetic.bf16_bits(values)
        w_dev, w = to_device(wb), synthetic.bf16_to_f32(wb)
        seg = sq.Segment(sq.view(w_dev), sq.view(None), sq.view(None), n, k, 0, sq.FMT_BF16)
    out = t.zeros((rows, stride), dtype=t.float32 if f32_out else t.int16, device="cuda")
    x_dev = to_device(x)
    if tile is None:
        chosen = ctypes.c_uint32()
        sq.call("sq_linear_float_tile", ctypes.byref(sq.device()), rows, n, seg.format_id, ctypes.byref(chosen))
        tile = chosen.value
        assert tile == (sq.FLOAT_TILE_NEURAL_ACCELERATOR if rows >= 64 else sq.FLOAT_TILE_SIMDGROUP)
    sq.call("sq_float_add", sq.stream_handle(), sq.view(x_dev), ctypes.byref(seg), sq.view(out), rows, stride,
            offset, sq.OUTPUT_F32 if f32_out else sq.OUTPUT_BF16, tile)
    t.cuda.synchronize()
    exact, magnitude = oracle.float_rows_f64(x, w)
    host = out.cpu().numpy()
    got = host[:, offset:offset + n].astype(np.float64) if f32_out else \
        synthetic.bf16_to_f32(host.view(np.uint16)[:, offset:offset + n]).astype(np.float64)
    # Each lane sums k / 64 products in a chain, then a 6-level butterfly; the MFMA kernel's longest path is
    # 4 k / 256 + 2 + 4 + 1: (k / 64 + 8) roundings of sum |x w| at most, plus half a bf16 ulp of the result for a
    # bf16 destination.
    bound = (k / 64 + 8) * 2.0 ** -24 * magnitude
    if not f32_out:
        bound = bound + 0.5 * oracle.ulp_bf16(exact)
    assert np.all(np.abs(got - exact) <= bound)
    untouched = np.delete(host, np.s_[offset:offset + n], axis=1)
    assert not untouched.any()
