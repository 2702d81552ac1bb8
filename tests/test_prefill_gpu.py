"""Prefill tile (rows > 32) through the C ABI against the fp64 oracle: each output inside its fp64 interval
(projectionBound of the staged numerics, which the tile follows: fp16 weights, exact products, fp32 sums),
BASELINE's tolerances, ragged chunks and odd column-tile counts, sparse inputs past half's range (the
power-of-two row scale), and the residual and up-with-gate epilogues of the SwiGLU chain (Linear.cpp:244-250)."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import (DeviceAffine, Run, check_projection, dense_inputs, make_weights, sparse_inputs, staged_reference,
                     to_device, torch)
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


def no_worse_than_staged(got, x, w, stats, what):
    """rel-L2 against fp64 no worse than the reference's staged numerics (fp16 weights, exact products, fp32 sums),
    emulated on the CPU, beyond rounding-boundary noise."""
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(staged_reference(x, w))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6, f"{what}: {stats['rel_l2']} against the staged {ref_l2}"


def run_prefill(w_list, x, epilogue=sq.EPILOGUE_NONE, residual=None, gate_scratch=None, n=None):
    segs, offset = [], 0
    for w in w_list:
        segs.append(w.segment(offset))
        offset += w.n
    n = n or offset
    proj = sq.projection(segs, output_size=n)
    rows, k = x.shape
    plan = sq.plan_for(sq.prefill_workload(n, k, rows, epilogue), proj)
    assert plan.config.tile == (sq.TILE_PREFILL if rows > 32 else sq.TILE_STAGED)
    run = Run(plan, n, x)
    t = torch()
    res = None
    if residual is not None:
        r = np.zeros((run.rows, n), np.uint16)
        r[:rows] = residual
        res = to_device(r)
    gs = None
    if gate_scratch is not None:
        g = np.zeros((run.rows, n), np.uint16)
        g[:rows] = gate_scratch
        gs = to_device(g)
    sq.linear_add(plan, proj, run.x, run.out, residual=res, gate_scratch=gs, scratch=run.scratch.struct())
    t.cuda.synchronize()
    out = run.output()
    assert np.all(out[rows:] == 0xFFFF), "rows past the chunk written"
    return out[:rows]


NEW_FORMATS = [oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64]


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_AF4G128, oracle.FMT_AF4G32] + NEW_FORMATS)
@pytest.mark.parametrize("rows", [33, 128, 300])
def test_prefill_dense(fmt, rows):
    rng = np.random.default_rng(rows + fmt)
    n, k = 320, 1024   # five 64-column tiles: the last workgroup's second half lies past the projection
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    stats = check_projection(run_prefill([w], x), x, w, f"prefill fmt {fmt} rows {rows}")
    no_worse_than_staged(None, x, w, stats, f"prefill fmt {fmt} rows {rows}")


def test_prefill_sparse_inputs_past_half_range():
    rng = np.random.default_rng(3)
    n, k = 256, 2048
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = sparse_inputs(64, k)
    check_projection(run_prefill([w], x), x, w, "prefill sparse")
    # mixed rows: tiny values beside 1e5 in the same row stay exact after the row scale
    xm = synthetic.bf16_to_f32(dense_inputs(rng, 48, k)) * np.float32(1e-3)
    xm[:, ::300] = 1e5
    xb = synthetic.bf16_bits(xm)
    check_projection(run_prefill([w], xb), xb, w, "prefill mixed")


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K])
@pytest.mark.parametrize("scale", [1e-5, 1e-6, 1e-8, 1e-30])
def test_prefill_small_rows(fmt, scale):
    """Rows of N(0,1) x scale: the reference multiplies bf16 rows of any magnitude exactly (matmul2d takes them as
    they are, gguf_linear.metal:36-55), so the table's row scale brings small rows up into half's normal range and
    the outputs stay inside the fp64 interval, as good as the staged emulation's. Below ~6e-5 a row left unscaled
    would enter the fp16 MFMA as half subnormals (1e-6: about a quarter of the outputs outside the interval)."""
    rng = np.random.default_rng(80 + fmt)
    n, k, rows = 512, 4096, 96
    w = make_weights(rng, fmt, n, k)
    x = synthetic.bf16_bits(synthetic.bf16_to_f32(dense_inputs(rng, rows, k)) * np.float32(scale))
    what = f"prefill fmt {fmt} rows x {scale}"
    stats = check_projection(run_prefill([w], x), x, w, what)
    no_worse_than_staged(None, x, w, stats, what)


def test_prefill_rows_of_every_magnitude_in_one_chunk():
    """One chunk whose rows run from 1e-30 to 1e4 (a different row scale each, bf16 subnormals and a zero row
    included): every row inside its interval, no worse than the staged emulation."""
    rng = np.random.default_rng(85)
    n, k, rows = 256, 2048, 40
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = synthetic.bf16_to_f32(dense_inputs(rng, rows, k)).astype(np.float64)
    x *= np.logspace(-30, 4, rows)[:, None]
    xb = synthetic.bf16_bits(x.astype(np.float32))
    xb[0] = rng.integers(0, 128, k).astype(np.uint16)          # bf16 subnormals
    xb[1] = 0
    out = run_prefill([w], xb)
    assert not synthetic.bf16_to_f32(out[1]).any(), "a zero row projects to zeros"
    stats = check_projection(out, xb, w, "prefill rows of every magnitude")
    no_worse_than_staged(None, xb, w, stats, "prefill rows of every magnitude")


@pytest.mark.parametrize("fmt", NEW_FORMATS)
def test_prefill_new_formats_sparse_and_mixed(fmt):
    """Sparse +-1e5 inputs (past half's range: the row scale) through the format's prefill tile, and the format beside
    a Q4_K segment in one fused projection (one dispatch per format, each writing its own columns)."""
    rng = np.random.default_rng(40 + fmt)
    k = 2048
    w = make_weights(rng, fmt, 256, k)
    x = sparse_inputs(64, k)
    check_projection(run_prefill([w], x), x, w, f"prefill sparse fmt {fmt}")
    parts = [make_weights(rng, oracle.FMT_Q4K, 128, k), make_weights(rng, fmt, 192, k)]
    x = dense_inputs(rng, 100, k)
    check_projection(run_prefill(parts, x), x, parts, f"prefill mixed fmt {fmt}")


@pytest.mark.parametrize("fmt", [oracle.FMT_Q4K] + NEW_FORMATS)
def test_prefill_tall_tiles(fmt):
    """Enough rows and columns that the launcher takes 256-row tiles (fewer rounds over the compute units), ragged in
    the last tile: four step slots a wave, or three for the formats whose slots leave room for no more (Q6_K, Q8_0,
    af8g64)."""
    rng = np.random.default_rng(60 + fmt)
    n, k, rows = 32768, 1024, 520
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    stats = check_projection(run_prefill([w], x), x, w, f"prefill tall fmt {fmt}")
    no_worse_than_staged(None, x, w, stats, f"prefill tall fmt {fmt}")


def test_prefill_fused_segments():
    rng = np.random.default_rng(5)
    k = 1024
    parts = [make_weights(rng, oracle.FMT_AF4G64, n, k) for n in (192, 64, 128)]
    x = dense_inputs(rng, 200, k)
    check_projection(run_prefill(parts, x), x, parts, "prefill fused")


def test_prefill_swiglu_epilogues():
    rng = np.random.default_rng(7)
    n, k, rows = 256, 1024, 160
    wg, wu = make_weights(rng, oracle.FMT_AF4G64, n, k), make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, rows, k)
    gate = run_prefill([wg], x)
    check_projection(gate, x, wg, "prefill gate")
    up_gated = run_prefill([wu], x, sq.EPILOGUE_UP_WITH_GATE, gate_scratch=gate)
    up = run_prefill([wu], x)
    gf, uf = synthetic.bf16_to_f32(gate).astype(np.float64), synthetic.bf16_to_f32(up).astype(np.float64)
    want = uf * gf / (1 + np.exp(-gf))
    got = synthetic.bf16_to_f32(up_gated).astype(np.float64)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(want), 1e-30))).astype(int) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-30)
    residual = synthetic.bf16_bits(rng.uniform(-64, 64, (rows, n)).astype(np.float32))
    down = make_weights(rng, oracle.FMT_AF4G64, n, k)
    out = run_prefill([down], x, sq.EPILOGUE_RESIDUAL, residual=residual)
    check_projection(out, x, down, "prefill residual", residual=residual)


def test_short_prefill_runs_decode_tile():
    rng = np.random.default_rng(9)
    n, k = 256, 1024
    w = make_weights(rng, oracle.FMT_Q4K, n, k)
    for rows in (1, 17, 32):
        x = dense_inputs(rng, rows, k)
        check_projection(run_prefill([w], x), x, w, f"short prefill {rows}")


_SHAPE_CACHE = {}


def shape_weights(fmt, n, k, seed):
    """Weights of a BASELINE shape, built once per module: af4g64 through the library's MLX repack (DeviceAffine),
    Q4_K through the oracle."""
    key = (fmt, n, k, seed)
    if key not in _SHAPE_CACHE:
        _SHAPE_CACHE.clear()
        rng = np.random.default_rng(seed)
        _SHAPE_CACHE[key] = DeviceAffine(rng, n, k) if fmt == oracle.FMT_AF4G64 else make_weights(rng, fmt, n, k)
    return _SHAPE_CACHE[key]


def sampled_rows(rows, count, rng):
    """The first and last rows, the last row of each 256-row tile and random others: every row tile kind is seen."""
    pick = {0, rows - 1} | {min(rows - 1, t * 256 + 255) for t in range((rows + 255) // 256)}
    pick |= set(rng.choice(rows, size=max(0, count - len(pick)), replace=False).tolist())
    return np.array(sorted(pick))


def check_sampled(out, x, w, what, rng, count=48):
    """Every column of a sample of rows against fp64: the staged interval, BASELINE's tolerances and no worse than
    the staged emulation."""
    pick = sampled_rows(x.shape[0], count, rng)
    stats = check_projection(out[pick], x[pick], w, what)
    no_worse_than_staged(None, x[pick], w, stats, what)
    return stats


@pytest.mark.parametrize("n,k,rows", [(14336, 4096, 2048), (4096, 14336, 2048), (27648, 5120, 2048),
                                      (14336, 4096, 2047)])
def test_config2_prefill_shapes(n, k, rows):
    """BASELINE config 2 at full size through the library's plan (its 256- and 128-row tiles as the launcher picks
    them per shape), af4g64 with z = -8 s; 2047 rows leave the last row tile ragged."""
    w = shape_weights(oracle.FMT_AF4G64, n, k, n + k)
    rng = np.random.default_rng(n + rows)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, f"config 2 {k}x{n} rows {rows}", rng)


@pytest.mark.parametrize("fmt", NEW_FORMATS)
def test_adjacent_formats_prefill_full_size(fmt):
    """The adjacent formats at the bench's full prefill size (M = 2048, K = 4096, N = 14336: 448 tiles of the
    four-wave tile, two rounds over the compute units): sampled rows against fp64, the staged interval and no worse
    than the staged emulation."""
    n, k, rows = 14336, 4096, 2048
    w = shape_weights(fmt, n, k, 40 + fmt)
    rng = np.random.default_rng(4096 + fmt)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, f"fmt {fmt} at M 2048, 4096 x 14336", rng, count=24)


def test_config2_ragged_with_small_rows():
    """Config 2's 4096 x 14336 at 2047 rows with rows scaled by 1e-5, 1e-6 and 1e-8 mixed in (the last 256-row tile
    ragged): the sampled rows, the small ones among them, inside their fp64 intervals and no worse than staged."""
    n, k, rows = 14336, 4096, 2047
    w = shape_weights(oracle.FMT_AF4G64, n, k, n + k)
    rng = np.random.default_rng(2047 + 5)
    x = synthetic.bf16_to_f32(dense_inputs(rng, rows, k))
    small = np.arange(3, rows, 97)
    x[small] *= np.array([1e-5, 1e-6, 1e-8], np.float32)[np.arange(small.size) % 3][:, None]
    xb = synthetic.bf16_bits(x)
    out = run_prefill([w], xb)
    pick = np.union1d(sampled_rows(rows, 24, rng), small[:12])
    stats = check_projection(out[pick], xb[pick], w, "config 2 ragged with small rows")
    no_worse_than_staged(None, xb[pick], w, stats, "config 2 ragged with small rows")


def test_prefill_halving_depends_on_the_chunk_rows():
    """Whether the prefill halves its tiles' K depends on the chunk's rows as well as the shape (4096 x 14336 halves
    from 257 to 512 rows, not at 256), so a row's bits can differ between chunks of 256 and 257 rows; both lie
    inside the row's fp64 interval, and their difference within two fp32 accumulation bounds of it."""
    n, k = 14336, 4096
    w = shape_weights(oracle.FMT_AF4G64, n, k, n + k)
    proj = sq.projection(w.segment())
    halved = lambda r: sq.scratch_size(sq.plan_for(sq.prefill_workload(n, k, r), proj))[0].partials > 0
    assert not halved(256) and halved(257)
    rng = np.random.default_rng(257)
    x = dense_inputs(rng, 257, k)
    whole, cut = run_prefill([w], x[:256]), run_prefill([w], x)[:256]
    pick = np.arange(0, 256, 17)
    check_projection(whole[pick], x[pick], w, "256 rows, whole K")
    check_projection(cut[pick], x[pick], w, "257 rows, halved K")
    value, magnitude, inputs, largest = oracle.project_f64(x[pick], w.values)
    bound = 2 * oracle.projection_bound(magnitude, inputs, largest, True) + \
        oracle.ulp_bf16(np.maximum(np.abs(value), 1e-30))
    a = synthetic.bf16_to_f32(whole[pick]).astype(np.float64)
    b = synthetic.bf16_to_f32(cut[pick]).astype(np.float64)
    assert np.all(np.abs(a - b) <= bound)


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_Q6K, oracle.FMT_AF8G64])
def test_prefill_halved_k(fmt):
    """A projection whose 256-row tiles would fill at most half the compute units runs each tile as two halves of K
    (two workgroups, fp32 halves added in K order by a close dispatch): 1800 rows (the last row tile ragged) of
    4096 x 4096, each half starting on whole meta units of the format."""
    n, k, rows = 4096, 4096, 1800
    w = make_weights(np.random.default_rng(70 + fmt), fmt, n, k)
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(n, k, rows), sq.projection(w.segment())))
    assert size.partials == 2 * rows * n * 4, "the plan halves K"
    rng = np.random.default_rng(71 + fmt)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, f"halved K fmt {fmt}", rng)


def test_prefill_halved_k_across_segments():
    """A fused projection whose halved tiles span segment boundaries: 1024 rows (4 row blocks) by 32 column groups of
    segments of 4096, 1536 and 2560 columns; the close maps each plane tile back to its segment's columns."""
    rng = np.random.default_rng(73)
    k, rows = 4096, 1024
    parts = [make_weights(rng, oracle.FMT_AF4G64, n, k) for n in (4096, 1536, 2560)]
    n = sum(p.n for p in parts)
    segs, offset = [], 0
    for p in parts:
        segs.append(p.segment(offset))
        offset += p.n
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(n, k, rows), sq.projection(segs)))
    assert size.partials == 2 * rows * n * 4, "the plan halves K"
    x = dense_inputs(rng, rows, k)
    out = run_prefill(parts, x)
    pick = sampled_rows(rows, 24, rng)
    check_projection(out[pick], x[pick], parts, "halved K across segments")


def test_prefill_halved_k_mixed_formats():
    """A projection of two formats halves by its whole width: each format's dispatch cuts its own tiles' K and closes
    its own columns, one after the other through the same partials."""
    rng = np.random.default_rng(74)
    k, rows = 4096, 1024
    parts = [make_weights(rng, oracle.FMT_AF4G64, 4096, k), make_weights(rng, oracle.FMT_Q4K, 4096, k)]
    segs = [parts[0].segment(0), parts[1].segment(4096)]
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(8192, k, rows), sq.projection(segs)))
    assert size.partials == 2 * rows * 8192 * 4, "the plan halves K"
    x = dense_inputs(rng, rows, k)
    out = run_prefill(parts, x)
    pick = sampled_rows(rows, 24, rng)
    check_projection(out[pick], x[pick], parts, "halved K, two formats")


def test_prefill_halved_k_epilogues():
    """The close dispatch of a halved projection applies the residual and the up-with-gate epilogues."""
    rng = np.random.default_rng(72)
    n, k, rows = 4096, 4096, 2048
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, rows, k)
    pick = sampled_rows(rows, 24, rng)
    plain = run_prefill([w], x)
    residual = synthetic.bf16_bits(rng.uniform(-64, 64, (rows, n)).astype(np.float32))
    out = run_prefill([w], x, sq.EPILOGUE_RESIDUAL, residual=residual)
    check_projection(out[pick], x[pick], w, "halved residual", residual=residual[pick])
    gate = synthetic.bf16_bits(rng.uniform(-4, 4, (rows, n)).astype(np.float32))
    up_gated = run_prefill([w], x, sq.EPILOGUE_UP_WITH_GATE, gate_scratch=gate)
    gf = synthetic.bf16_to_f32(gate[pick]).astype(np.float64)
    uf = synthetic.bf16_to_f32(plain[pick]).astype(np.float64)
    want = uf * gf / (1 + np.exp(-gf))
    got = synthetic.bf16_to_f32(up_gated[pick]).astype(np.float64)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(want), 1e-30))).astype(int) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-30)


def accumulation_bound(x, w, pick):
    """Two fp32 accumulation bounds of each picked row's outputs plus a bf16 ulp: how far apart two correct results
    of one row may lie when their fp32 sums ran in different orders (whole K against pieces of it)."""
    value, magnitude, inputs, largest = oracle.project_f64(x[pick], w.values)
    return 2 * oracle.projection_bound(magnitude, inputs, largest, True) + \
        oracle.ulp_bf16(np.maximum(np.abs(value), 1e-30))


def test_q4k_projection_benchmark_shape():
    """The reference's gguf-projection-benchmark shape (Q4_K, K = 5120, N = 17408, M = 2048; 544 256-row tiles: one
    whole round over the compute units, then the other 288 as stream pieces): sampled rows against fp64. Against a
    300-row prefill of the same weights (128-row tiles, all whole): the columns of the whole round's tiles bitwise
    the same, the stream tiles' columns within two fp32 accumulation bounds."""
    n, k, rows = 17408, 5120, 2048
    w = shape_weights(oracle.FMT_Q4K, n, k, 4)
    rng = np.random.default_rng(2048)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, "Q4_K projection benchmark rows 2048", rng)
    short = run_prefill([w], x[:300])
    whole = 256 // 8 * 256    # the whole rounds' 256 tiles: 8 row blocks x 32 column groups of 256 columns
    assert np.array_equal(short[:, :whole], out[:300, :whole])
    pick = np.arange(0, 300, 23)
    a = synthetic.bf16_to_f32(short[pick]).astype(np.float64)
    b = synthetic.bf16_to_f32(out[pick]).astype(np.float64)
    assert np.all(np.abs(a - b) <= accumulation_bound(x, w, pick))


def stream_schedule(rows, n, k):
    """The stream schedule the library's launcher computes for a whole-K dispatch of more than one round of 256-row
    tiles: whole rounds of 256 tiles, then each row block's remaining tiles with their K steps laid end to end and cut
    into ranges of a multiple of four steps, 256 / row blocks ranges at most a row block, one a workgroup. Returns the
    whole tiles, the stream tiles and how many of them are cut in two and in three pieces."""
    steps, blocks = k // 64, (rows + 255) // 256
    tiles = blocks * ((n // 64 + 3) // 4)
    rounds, rest = divmod(tiles, 256)
    assert rounds >= 1 and rest and 256 % blocks == 0
    dp = rounds * 256 if 2 * rest >= 256 else (rounds - 1) * 256
    per_block, ranges = (tiles - dp) // blocks, 256 // blocks
    span = -(-per_block * steps // (4 * ranges)) * 4
    assert steps <= 2 * span
    cut = [(c * steps + steps - 1) // span - c * steps // span + 1 for c in range(per_block)] * blocks
    return dp, tiles - dp, cut.count(2), cut.count(3)


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G128])
def test_prefill_stream_pieces(fmt):
    """Past whole rounds of tiles, the rest run as stream pieces (ranges of K steps over every compute unit, the last
    piece of a tile to arrive adding the pieces' fp32 sums in K order) in the same dispatch: 1024 rows of
    1280 x 24576 run 256 whole tiles, then 128 in pieces, 84 of them cut in two and 44 in three. Sampled rows against
    fp64, a second run bitwise the same (the sum does not depend on the order the pieces arrive in), and a 128-row
    chunk of the rows (whole tiles) within two accumulation bounds. Every eight-wave format: a range is a multiple
    of four 64-input steps, whole scale groups of 4-bit affine g32, g64 and g128 and whole Q4_K super-blocks."""
    n, k, rows = 24576, 1280, 1024
    assert stream_schedule(rows, n, k) == (256, 128, 84, 44)
    w = make_weights(np.random.default_rng(80 + fmt), fmt, n, k)
    size, _ = sq.scratch_size(sq.plan_for(sq.prefill_workload(n, k, rows), sq.projection(w.segment())))
    assert size.partials > 0 and size.counters >= 128 * 4, "the plan reserves the stream partials and counters"
    rng = np.random.default_rng(81 + fmt)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, f"stream pieces fmt {fmt}", rng)
    assert np.array_equal(run_prefill([w], x), out)
    pick = np.arange(0, 128, 9)
    a = synthetic.bf16_to_f32(run_prefill([w], x[:128])[pick]).astype(np.float64)
    b = synthetic.bf16_to_f32(out[pick]).astype(np.float64)
    assert np.all(np.abs(a - b) <= accumulation_bound(x, w, pick))


@pytest.mark.parametrize("rows,n,k,fmt,want", [
    (512, 49152, 1280, oracle.FMT_AF4G64, (256, 128, 86, 42)),    # two row blocks
    (1900, 12288, 1280, oracle.FMT_Q4K, (256, 128, 88, 40)),      # eight, the last ragged
])
def test_prefill_stream_row_blocks(rows, n, k, fmt, want):
    """The stream schedule over other row-block counts: each row block's ranges cover its own tiles (workgroups of a
    row block run on the XCDs that hold its activations); the last row block's rows past the chunk are not written.
    Sampled rows against fp64 and a second run bitwise the same."""
    assert stream_schedule(rows, n, k) == want
    w = make_weights(np.random.default_rng(rows + fmt), fmt, n, k)
    rng = np.random.default_rng(rows + n)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, f"stream pieces, {rows} rows of {k} x {n}", rng, count=32)
    assert np.array_equal(run_prefill([w], x), out)


def test_prefill_stream_epilogues_and_segments():
    """Stream pieces under the residual and up-with-gate epilogues (applied once, by the tile's last piece), across
    a fused projection's segments (8192, 4096 and 12288 columns of af4g64), and beside a four-wave format's whole
    tiles (24576 columns of af4g64 and 2048 of Q6_K in one projection: each format's dispatch schedules its own
    tiles, the af4g64 ones in part as stream pieces)."""
    rng = np.random.default_rng(82)
    k, rows = 1280, 1024
    parts = [make_weights(rng, oracle.FMT_AF4G64, n, k) for n in (8192, 4096, 12288)]
    x = dense_inputs(rng, rows, k)
    pick = sampled_rows(rows, 24, rng)
    out = run_prefill(parts, x)
    check_projection(out[pick], x[pick], parts, "stream pieces across segments")
    w = make_weights(rng, oracle.FMT_AF4G64, 24576, k)
    n = w.n
    plain = run_prefill([w], x)
    residual = synthetic.bf16_bits(rng.uniform(-64, 64, (rows, n)).astype(np.float32))
    got = run_prefill([w], x, sq.EPILOGUE_RESIDUAL, residual=residual)
    check_projection(got[pick], x[pick], w, "stream residual", residual=residual[pick])
    gate = synthetic.bf16_bits(rng.uniform(-4, 4, (rows, n)).astype(np.float32))
    up_gated = run_prefill([w], x, sq.EPILOGUE_UP_WITH_GATE, gate_scratch=gate)
    gf = synthetic.bf16_to_f32(gate[pick]).astype(np.float64)
    uf = synthetic.bf16_to_f32(plain[pick]).astype(np.float64)
    want = uf * gf / (1 + np.exp(-gf))
    got = synthetic.bf16_to_f32(up_gated[pick]).astype(np.float64)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(want), 1e-30))).astype(int) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-30)
    mixed = [w, make_weights(rng, oracle.FMT_Q6K, 2048, k)]
    out = run_prefill(mixed, x)
    check_projection(out[pick], x[pick], mixed, "stream af4g64 beside whole Q6_K tiles")


def test_config3_q4k_prefill():
    """BASELINE config 3's prefill point: Q4_K, K = 5120, N = 27648, M = 512."""
    n, k, rows = 27648, 5120, 512
    w = shape_weights(oracle.FMT_Q4K, n, k, 3)
    rng = np.random.default_rng(512)
    x = dense_inputs(rng, rows, k)
    out = run_prefill([w], x)
    check_sampled(out, x, w, "config 3 Q4_K rows 512", rng)
