"""Decode tile (rows <= 32) through the C ABI against the fp64 oracle, with the reference's projection-test
properties (dev/tests/engine/gguf_projection_test.mm): every output inside its fp64 interval (projectionBound of the
register tile, the accumulation term alone: the decode tiles multiply exact code operands, GgufFormatReference.hpp:
787-797),
BASELINE's rel-L2 <= 1e-2 and max-abs <= 2^-6 max|row|, sparse inputs past half's range, a row's output bitwise
independent of the other rows of its tile kind (the column tile runs 1..4 rows, the row tile more), K-split
determinism with counters returned to zero, the epilogues (residual, gate/up in one pass bitwise equal to two
passes, fp32 destination), fused segments equal to segments alone, and untouched padding columns. Both tile kinds
run every case that has rows to choose."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import (DeviceAffine, Run, Weights, bf16, check_projection, dense_inputs, make_weights, sparse_inputs,
                     staged_reference, to_device, to_host, torch)
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu


def check_decode(*args, **kwargs):
    """check_projection with the register tile's bound (no fp16 weight rounding term)."""
    return check_projection(*args, staged=False, **kwargs)

FORMATS = [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G128]


def run_plan(plan, proj, x, n, out_dtype=np.uint16, residual=None, gate=None, gate_scratch_rows=0):
    run = Run(plan, n, x, out_dtype)
    t = torch()
    res = None
    if residual is not None:
        r = np.zeros((run.rows, n), np.uint16)
        r[: residual.shape[0]] = residual
        res = to_device(r)
    gs = run.scratch.gate
    sq.linear_add(plan, proj, run.x, run.out, residual=res, gate_scratch=gs, scratch=run.scratch.struct(), gate=gate)
    t.cuda.synchronize()
    counters = run.scratch.counters
    if counters is not None:
        assert int(counters.abs().sum().item()) == 0, "split counters not returned to zero"
    return run.output()[: x.shape[0]]


def staged(n, k, rows, splits, epilogue=sq.EPILOGUE_NONE, destination=sq.OUTPUT_BF16, one_pass=0):
    return sq.plan_config(sq.decode_workload(n, k, rows, epilogue), sq.LinearConfig(sq.TILE_STAGED, splits, 0, one_pass, 0),
                          destination)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows", [1, 2, 3, 8, 16, 24, 32])
@pytest.mark.parametrize("splits", [1, 4])
def test_decode_dense(fmt, rows, splits):
    rng = np.random.default_rng(1000 * fmt + 10 * rows + splits)
    n, k = 256, 2048
    w = make_weights(rng, fmt, n, k, centred=rows % 2 == 1)
    x = dense_inputs(rng, rows, k)
    got = run_plan(staged(n, k, rows, splits), sq.projection(w.segment()), x, n)
    stats = check_decode(got, x, w, f"fmt {fmt} rows {rows} splits {splits}")
    # no worse than the reference's staged numerics (fp16 weights, fp32 sums), beyond rounding-boundary noise
    ref = staged_reference(x, w)
    value, *_ = oracle.project_f64(x, w.values)
    ref_l2 = np.linalg.norm(synthetic.bf16_to_f32(ref) - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K])
@pytest.mark.parametrize("splits", [1, 2, 16])
def test_decode_sparse_inputs(fmt, splits):
    rng = np.random.default_rng(7 + fmt + splits)
    n, k = 192, 4096
    w = make_weights(rng, fmt, n, k)
    x = sparse_inputs(8, k)
    got = run_plan(staged(n, k, 8, splits), sq.projection(w.segment()), x, n)
    check_decode(got, x, w, "sparse")


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K])
@pytest.mark.parametrize("splits", [1, 8])
def test_rows_are_independent(fmt, splits):
    """A row's output is bitwise the same in any batch of its tile kind: alone (the one-row instance), in a pair (the
    two-row instance) or among four rows on the column tile, among 16 or 32 rows on the row tile; across the kinds
    both are inside the oracle's interval (check_projection)."""
    rng = np.random.default_rng(31 + splits)
    n, k = 128, 2048   # K partitions take whole meta units: Q4_K's 256-input super-blocks
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, 32, k)
    proj = sq.projection(w.segment())
    all32 = run_plan(staged(n, k, 32, splits), proj, x, n)
    first16 = run_plan(staged(n, k, 16, splits), proj, x[:16], n)
    assert np.array_equal(all32[:16], first16)
    four = run_plan(staged(n, k, 4, splits), proj, x[:4], n)
    for r in range(4):
        alone = run_plan(staged(n, k, 1, splits), proj, x[r:r + 1], n)
        assert np.array_equal(alone[0], four[r]), f"row {r}"
    for r in (0, 2):
        two = run_plan(staged(n, k, 2, splits), proj, x[r:r + 2], n)
        assert np.array_equal(two, four[r:r + 2]), f"rows {r}, {r + 1}"
    check_decode(four, x[:4], w, "column tile")
    check_decode(all32, x, w, "row tile")


def test_split_determinism_and_poisoned_partials():
    rng = np.random.default_rng(3)
    n, k = 512, 4096
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, 4, k)
    proj = sq.projection(w.segment())
    plan = staged(n, k, 4, 8)
    run = Run(plan, n, x)
    t = torch()
    outs = []
    for poison in (0x7FC00000, 0x7E800000):   # NaN, then a large finite value in every partial
        run.scratch.partials.fill_(poison)
        sq.linear_add(plan, proj, run.x, run.out, scratch=run.scratch.struct())
        t.cuda.synchronize()
        assert int(run.scratch.counters.abs().sum().item()) == 0
        outs.append(run.output().copy())
    assert np.array_equal(outs[0], outs[1])
    check_decode(outs[0][:4], x, w, "poisoned partials")


@pytest.mark.parametrize("rows", [2, 8])
def test_residual_epilogue(rows):
    rng = np.random.default_rng(5 + rows)
    n, k = 256, 2048
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, rows, k)
    residual = synthetic.bf16_bits(rng.uniform(-1, 1, (rows, n)).astype(np.float32) * 64)
    for splits in (2, 4):
        got = run_plan(staged(n, k, rows, splits, sq.EPILOGUE_RESIDUAL), sq.projection(w.segment()), x, n,
                       residual=residual)
        check_decode(got, x, w, "residual", residual=residual)


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K])
@pytest.mark.parametrize("rows,splits", [(8, 1), (8, 4), (2, 2), (2, 4), (1, 8)])
def test_gate_up_one_pass_equals_two_passes(fmt, rows, splits):
    rng = np.random.default_rng(11 + splits + rows)
    n, k = 256, 2048
    wg, wu = make_weights(rng, fmt, n, k), make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    gate, up = sq.projection(wg.segment()), sq.projection(wu.segment())
    two = run_plan(staged(n, k, rows, splits, sq.EPILOGUE_GATE_UP), up, x, n, gate=gate)
    one = run_plan(staged(n, k, rows, splits, sq.EPILOGUE_GATE_UP, one_pass=1), up, x, n, gate=gate)
    assert np.array_equal(one, two)
    g = run_plan(staged(n, k, rows, splits), gate, x, n)
    u = run_plan(staged(n, k, rows, splits), up, x, n)
    gf, uf = synthetic.bf16_to_f32(g).astype(np.float64), synthetic.bf16_to_f32(u).astype(np.float64)
    want = uf * gf / (1 + np.exp(-gf))
    got = synthetic.bf16_to_f32(one).astype(np.float64)
    # bf16(up) * silu(bf16(gate)) in fp32, rounded once to bf16: within one bf16 ulp of the exact product
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(want), 1e-30))).astype(int) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-30)


@pytest.mark.parametrize("rows", [1, 8])
def test_fp32_destination_rounds_to_the_bf16_output(rows):
    rng = np.random.default_rng(17 + rows)
    n, k = 256, 4096
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment(), destination=sq.OUTPUT_F32)
    for splits in (2, 8):
        f32 = run_plan(staged(n, k, rows, splits, destination=sq.OUTPUT_F32), proj, x, n, out_dtype=np.float32)
        b16 = run_plan(staged(n, k, rows, splits), sq.projection(w.segment()), x, n)
        assert np.array_equal(synthetic.bf16_bits(f32), b16)
        value, magnitude, inputs, largest = oracle.project_f64(x, w.values)
        bound = oracle.projection_bound(magnitude, inputs, largest, False)
        assert np.all(np.abs(f32.astype(np.float64) - value) <= bound)
        # no worse than the reference's staged fp32 sums on these rows (plus accumulation-order slack)
        ref = oracle.project_staged_f32(x, w.halves).astype(np.float64)
        assert np.linalg.norm(f32 - value) <= 2.0 * np.linalg.norm(ref - value) + 1e-9 * np.linalg.norm(value)


@pytest.mark.parametrize("rows", [3, 8])
def test_fused_segments_equal_segments_alone(rows):
    rng = np.random.default_rng(23 + rows)
    k = 2048
    parts = [make_weights(rng, oracle.FMT_AF4G64, n, k) for n in (256, 64, 128)]
    x = dense_inputs(rng, rows, k)
    total = sum(p.n for p in parts)
    segs, offset = [], 0
    for p in parts:
        segs.append(p.segment(offset))
        offset += p.n
    fused = run_plan(staged(total, k, rows, 2), sq.projection(segs), x, total)
    offset = 0
    for p in parts:
        alone = run_plan(staged(p.n, k, rows, 2), sq.projection(p.segment()), x, p.n)
        assert np.array_equal(fused[:, offset:offset + p.n], alone)
        offset += p.n
    check_decode(fused, x, parts, "fused")


MIXED = [(oracle.FMT_Q4K, oracle.FMT_Q4K, oracle.FMT_Q6K), (oracle.FMT_Q80, oracle.FMT_Q5K, oracle.FMT_AF4G32),
         (oracle.FMT_AF8G64, oracle.FMT_AF4G128, oracle.FMT_AF4G64)]


@pytest.mark.parametrize("formats", MIXED)
@pytest.mark.parametrize("rows", [1, 3, 8, 20])
@pytest.mark.parametrize("splits", [1, 4])
def test_mixed_format_segments_in_one_dispatch(formats, rows, splits):
    """Up to three segments of any formats run in one dispatch (the reference's fused decode takes a format per
    segment: GgufDecodeFusedParams.fmt[3], Gguf.h:97-106), a Q4_K q|k with a Q6_K v among them. Each tile computes
    what it does alone: the fused columns equal each segment run by itself at the same split."""
    rng = np.random.default_rng(37 + 100 * rows + splits + formats[0])
    k = 2048
    parts = [make_weights(rng, f, n, k) for f, n in zip(formats, (128, 64, 192))]
    x = dense_inputs(rng, rows, k)
    total = sum(p.n for p in parts)
    segs, offset = [], 0
    for p in parts:
        segs.append(p.segment(offset))
        offset += p.n
    fused = run_plan(staged(total, k, rows, splits), sq.projection(segs), x, total)
    offset = 0
    for p in parts:
        alone = run_plan(staged(p.n, k, rows, splits), sq.projection(p.segment()), x, p.n)
        assert np.array_equal(fused[:, offset:offset + p.n], alone), f"segment at {offset} ({p.fmt})"
        offset += p.n
    check_decode(fused, x, parts, f"mixed {formats} rows {rows} splits {splits}")


def test_padding_columns_untouched():
    rng = np.random.default_rng(29)
    n, k, pad = 256, 1024, 256
    w = make_weights(rng, oracle.FMT_AF4G64, n, k)
    x = dense_inputs(rng, 4, k)
    proj = sq.projection(w.segment(), output_size=n + pad)
    got = run_plan(staged(n + pad, k, 4, 4), proj, x, n + pad)
    assert np.all(got[:, n:] == 0xFFFF)
    check_decode(got[:, :n], x, w, "padded")


def widened(w, extra):
    """w's planes followed by `extra` zero columns (whole tiles): the planes are tile-major, so the first w.n columns
    of the wider tensor are w's bytes. Returns the segment and the device buffers it points at."""
    t = torch()
    groups, p1 = w.k // 32, sq.FORMATS[w.fmt][5]
    p0_bytes, meta_bytes = sq.plane_bytes(w.fmt, extra, w.k)
    zeros = lambda b: t.zeros(b, dtype=t.uint8, device="cuda")
    plane0 = t.cat([w.plane0, zeros(p0_bytes)])
    meta = t.cat([w.meta, zeros(meta_bytes)])
    plane1 = t.cat([w.plane1, zeros(extra * groups * p1)]) if p1 else None
    keep = (plane0, meta, plane1)
    return sq.segment(w.fmt, w.n + extra, w.k, plane0, meta, 0, plane1), keep


# The column tile runs 16-column workgroups (each wave four K slices) while four for each of a dispatch's 64-column
# tiles times its splits fit one a compute unit (256 for the default device), the row tile (one MFMA column block a
# wave) while they fit a few a compute unit, 64-column ones past that: zero columns past a projection's own widen
# its dispatch to 64-column workgroups. The widened dispatch holds exactly 256 tiles times splits: past that the
# row tile takes its longest slices (another summation order).
def device_fill(n, splits=1):
    """The zero columns that widen an n-column dispatch of `splits` K splits to 256 tiles times splits."""
    return 64 * (256 // splits) - n


NARROW = [(oracle.FMT_AF4G64, 1, 1, 2048), (oracle.FMT_AF4G64, 4, 2, 4096), (oracle.FMT_AF4G64, 1, 1, 14336),
          (oracle.FMT_Q4K, 1, 4, 4096), (oracle.FMT_Q4K, 3, 1, 2048), (oracle.FMT_Q4K, 1, 1, 8192),
          (oracle.FMT_Q5K, 2, 1, 2048), (oracle.FMT_Q6K, 1, 2, 4096), (oracle.FMT_Q6K, 4, 1, 2048),
          (oracle.FMT_Q80, 1, 1, 4096), (oracle.FMT_AF8G64, 4, 4, 4096), (oracle.FMT_AF4G32, 2, 1, 2048),
          (oracle.FMT_AF4G128, 1, 2, 8192),
          # the row tile (5..32 rows): one MFMA column block a workgroup
          (oracle.FMT_AF4G64, 8, 1, 4096), (oracle.FMT_AF4G64, 16, 2, 4096), (oracle.FMT_AF4G64, 32, 1, 2048),
          (oracle.FMT_Q4K, 12, 4, 4096), (oracle.FMT_Q5K, 24, 1, 2048), (oracle.FMT_Q6K, 8, 2, 2048),
          (oracle.FMT_Q6K, 20, 1, 4096), (oracle.FMT_Q80, 16, 1, 2048), (oracle.FMT_AF8G64, 9, 2, 2048),
          (oracle.FMT_AF4G32, 32, 4, 2048), (oracle.FMT_AF4G128, 16, 1, 8192)]


@pytest.mark.parametrize("fmt,rows,splits,k", NARROW)
def test_column_slices_equal_whole_tile_workgroups(fmt, rows, splits, k):
    """A projection of few tiles runs 16-column workgroups; the same weights widened past the compute units run one
    64-column workgroup per tile (and split). Both compute the same bits for the shared columns, and those are
    inside the oracle's interval with the register tile's bound (K 14336: 14 slices of 32 groups, two quarters of
    the last wave idle). Rows past 4 run the row tile's one-block workgroups."""
    rng = np.random.default_rng(41 + fmt + 10 * rows + 100 * splits + k)
    n = 128
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    narrow = run_plan(staged(n, k, rows, splits), sq.projection(w.segment()), x, n)
    seg, keep = widened(w, device_fill(n, splits))
    total = seg.output_size
    wide = run_plan(staged(total, k, rows, splits), sq.projection(seg), x, total)
    assert np.array_equal(wide[:, :n], narrow)
    assert np.all(wide[:, n:] == 0)
    check_decode(narrow, x, w, f"16-column workgroups fmt {fmt} rows {rows} splits {splits} k {k}")


def _random_narrow_cases(count=12, seed=4242):
    """Seeded draws of (format, columns, K, rows, splits) that the decode tiles run: K a multiple of the format's
    meta unit times the splits, every row count of both tile kinds."""
    rng = np.random.default_rng(seed)
    formats = [oracle.FMT_AF4G64, oracle.FMT_AF4G32, oracle.FMT_AF4G128, oracle.FMT_Q4K, oracle.FMT_Q5K,
               oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64]
    cases = []
    while len(cases) < count:
        fmt = formats[rng.integers(len(formats))]
        unit = sq.FORMATS[fmt][4] * 32
        splits = int(rng.choice([1, 2, 4]))
        k = int(unit * splits * rng.integers(1, 1 + 6144 // (unit * splits)))
        n = int(64 * rng.integers(1, 9))
        rows = int(rng.choice([1, 2, 3, 4, 5, 9, 16, 17, 31, 32]))
        cases.append((fmt, n, k, rows, splits))
    return cases


@pytest.mark.parametrize("fmt,n,k,rows,splits", _random_narrow_cases())
def test_column_slices_random_shapes(fmt, n, k, rows, splits):
    """Random shapes (slices of 8, 16 or 32 groups, whole or with a short last one, idle quarters, one to four
    splits): a projection's 16-column workgroups give the bits its widened dispatch's 64-column ones give."""
    rng = np.random.default_rng(fmt + n + k + rows + splits)
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    narrow = run_plan(staged(n, k, rows, splits), sq.projection(w.segment()), x, n)
    seg, keep = widened(w, device_fill(n, splits))
    wide = run_plan(staged(seg.output_size, k, rows, splits), sq.projection(seg), x, seg.output_size)
    assert np.array_equal(wide[:, :n], narrow)
    check_decode(narrow, x, w, f"random shape fmt {fmt} {n}x{k} rows {rows} splits {splits}")


@pytest.mark.parametrize("fmt,rows,splits", [(oracle.FMT_AF4G64, 1, 1), (oracle.FMT_Q4K, 4, 2),
                                             (oracle.FMT_Q80, 1, 1), (oracle.FMT_AF8G64, 2, 4),
                                             (oracle.FMT_AF4G64, 8, 1), (oracle.FMT_Q4K, 24, 2),
                                             (oracle.FMT_Q6K, 16, 1), (oracle.FMT_AF8G64, 32, 1)])
def test_column_slices_gate_up_pairs(fmt, rows, splits):
    """One-pass gate/up pairs: 16-column workgroups (few tiles) and 64-column ones (widened) give the same bits."""
    rng = np.random.default_rng(43 + fmt + rows + splits)
    n, k = 128, 2048
    wg, wu = make_weights(rng, fmt, n, k), make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    narrow = run_plan(staged(n, k, rows, splits, sq.EPILOGUE_GATE_UP, one_pass=1), sq.projection(wu.segment()), x,
                      n, gate=sq.projection(wg.segment()))
    (g, keep_g), (u, keep_u) = widened(wg, device_fill(n, splits)), widened(wu, device_fill(n, splits))
    total = g.output_size
    wide = run_plan(staged(total, k, rows, splits, sq.EPILOGUE_GATE_UP, one_pass=1), sq.projection(u), x, total,
                    gate=sq.projection(g))
    assert np.array_equal(wide[:, :n], narrow)


@pytest.mark.parametrize("rows", [1, 4, 8, 20])
def test_column_slices_mixed_formats(rows):
    """Mixed-format segments in one dispatch: 16-column workgroups alone, 64-column ones with a wide third segment."""
    rng = np.random.default_rng(47 + rows)
    k = 2048
    a, b = make_weights(rng, oracle.FMT_Q4K, 128, k), make_weights(rng, oracle.FMT_Q6K, 64, k)
    c = make_weights(rng, oracle.FMT_AF4G64, 64, k)
    x = dense_inputs(rng, rows, k)
    narrow = run_plan(staged(256, k, rows, 1), sq.projection([a.segment(), b.segment(128), c.segment(192)]), x, 256)
    wide_c, keep = widened(c, device_fill(256))
    total = 192 + wide_c.output_size
    wide_c.column_offset = 192
    wide = run_plan(staged(total, k, rows, 1), sq.projection([a.segment(), b.segment(128), wide_c]), x, total)
    assert np.array_equal(wide[:, :256], narrow)


_SHAPE_CACHE = {}


def shape_weights(fmt, n, k, seed):
    """Weights of a BASELINE shape, built once per module (the largest take seconds on the CPU)."""
    key = (fmt, n, k, seed)
    if key not in _SHAPE_CACHE:
        _SHAPE_CACHE.clear()
        rng = np.random.default_rng(seed)
        _SHAPE_CACHE[key] = DeviceAffine(rng, n, k) if fmt == oracle.FMT_AF4G64 else make_weights(rng, fmt, n, k)
    return _SHAPE_CACHE[key]


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (2048, 5120)])
@pytest.mark.parametrize("rows", [1, 2, 4, 8, 16, 32])
def test_config1_sweep_policy_plans(n, k, rows):
    """BASELINE config 1's decode sweep (and config 0, the 4096 x 4096 shape at M = 1): every shape at every M under
    the library's own plan, every output against fp64 with the register tile's bound, and no worse than the
    reference's staged numerics. 2048 x 5120 adds the split law's two splits in 16-column workgroups."""
    w = shape_weights(oracle.FMT_AF4G64, n, k, n + k)
    rng = np.random.default_rng(n + k + rows)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    got = run_plan(plan, proj, x, n)
    stats = check_decode(got, x, w, f"{n}x{k} rows {rows}")
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(synthetic.bf16_bits(oracle.project_staged_f32(x, w.halves)))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


@pytest.mark.parametrize("n,k,want", [(512, 4096, 4), (1024, 4096, 4), (2048, 5120, 2), (1024, 2048, 1)])
@pytest.mark.parametrize("rows", [8, 16, 32])
def test_row_tile_split_law_plans(n, k, want, rows):
    """The row tile's split law at few tiles: a split doubled while its 16-column workgroups fit the device (N 512
    and 1024 at K 4096: four splits), four splits in 64-column workgroups narrowed to two in 16-column ones (2048 x
    5120), an unsplit tile kept unsplit (1024 x 2048). Each plan's outputs against fp64 with the register tile's
    bound, and no worse than the reference's staged numerics."""
    w = shape_weights(oracle.FMT_AF4G64, n, k, 17 + n + k)
    rng = np.random.default_rng(500 + rows + n)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    assert plan.config.splits == want
    got = run_plan(plan, proj, x, n)
    stats = check_decode(got, x, w, f"{n}x{k} rows {rows} splits {want}")
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(synthetic.bf16_bits(oracle.project_staged_f32(x, w.halves)))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


@pytest.mark.parametrize("n", [3072, 4096])
@pytest.mark.parametrize("rows", [5, 16])
def test_row_tile_unsplit_plans(n, rows):
    """K 4096 at 48 or 64 tiles: the split law leaves the row tile of up to 16 rows unsplit in 16-column workgroups
    (a split would leave it in 64-column ones). Every output against fp64 with the register tile's bound, and the
    same bits as the unsplit 64-column workgroups of the same weights widened past the compute units."""
    k = 4096
    w = shape_weights(oracle.FMT_AF4G64, n, k, 7 + n)
    rng = np.random.default_rng(n + rows)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    assert plan.config.splits == 1
    got = run_plan(plan, proj, x, n)
    check_decode(got, x, w, f"unsplit row tile {n}x{k} rows {rows}")
    seg, keep = widened(w, device_fill(n))
    wide = run_plan(staged(seg.output_size, k, rows, 1), sq.projection(seg), x, seg.output_size)
    assert np.array_equal(wide[:, :n], got)


@pytest.mark.parametrize("rows", [1, 16])
def test_config3_q4k_decode(rows):
    """BASELINE config 3's decode points: Q4_K, K = 5120, N = 27648, M = 1 and 16 under the library's plan, every
    output against fp64 (register tile bound) and no worse than the reference's staged numerics."""
    n, k = 27648, 5120
    w = shape_weights(oracle.FMT_Q4K, n, k, 3)
    rng = np.random.default_rng(300 + rows)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    got = run_plan(plan, proj, x, n)
    stats = check_decode(got, x, w, f"Q4_K {n}x{k} rows {rows}")
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(staged_reference(x, w))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_AF4G32, oracle.FMT_AF4G128, oracle.FMT_Q4K,
                                 oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80])
@pytest.mark.parametrize("rows,k", [(8, 2048), (16, 2048), (12, 2560)])
def test_row_tile_long_slices(fmt, rows, k):
    """A row tile of more 64-column workgroups than compute units (257 tiles) takes 32-group slices in the
    16-byte-code formats (8-bit codes keep the shortest): K 2048 in two whole slices, K 2560 (80 groups) with a last
    slice of 16, whose loads past it repeat its last group. Every output against fp64 with the register tile's bound,
    and no worse than the reference's staged numerics."""
    n = 64 * 257
    w = shape_weights(fmt, n, k, 11 + fmt)
    rng = np.random.default_rng(400 + rows + fmt + k)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    assert plan.config.splits == 1
    got = run_plan(plan, proj, x, n)
    stats = check_decode(got, x, w, f"fmt {fmt} {n}x{k} rows {rows}")
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(staged_reference(x, w))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


NEW_FORMATS = [oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64]


@pytest.mark.parametrize("fmt", NEW_FORMATS)
@pytest.mark.parametrize("rows", [1, 2, 4, 5, 16, 17, 32])
@pytest.mark.parametrize("splits", [1, 4])
def test_decode_new_formats(fmt, rows, splits):
    """Q5_K, Q6_K, Q8_0 and af8g64 through the decode column tile (rows <= 4) and row tile (5 to 32 rows): every
    output inside its fp64 interval, the BASELINE tolerances, and no worse than the reference's staged numerics."""
    rng = np.random.default_rng(2000 * fmt + 10 * rows + splits)
    n, k = 256, 2048
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    got = run_plan(staged(n, k, rows, splits), sq.projection(w.segment()), x, n)
    stats = check_decode(got, x, w, f"fmt {fmt} rows {rows} splits {splits}")
    ref = staged_reference(x, w)
    value, *_ = oracle.project_f64(x, w.values)
    ref_l2 = np.linalg.norm(synthetic.bf16_to_f32(ref) - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6


@pytest.mark.parametrize("fmt", NEW_FORMATS)
@pytest.mark.parametrize("rows", [3, 9])
def test_decode_new_formats_fixture_and_pairs(fmt, rows):
    """The reference's fixture weights (every byte random, finite half scales) through the column and row tiles,
    sparse +-1e5 inputs, and one-pass gate/up pairs (column tile, both row-tile register budgets) bitwise equal to
    two passes."""
    rng = np.random.default_rng(77 + fmt + rows)
    n, k = 128, 1024
    native = oracle.fixture(fmt, n, k, 9)
    if fmt == oracle.FMT_AF8G64:
        native = make_weights(rng, fmt, n, k).native
    w = Weights(fmt, n, k, native)
    if np.isfinite(w.values).all() and np.abs(w.values).max() < 1e30:
        x = sparse_inputs(rows, k, 1.0)
        got = run_plan(staged(n, k, rows, 1), sq.projection(w.segment()), x, n)
        check_decode(got, x, w, f"fixture fmt {fmt} rows {rows}")
    wg, wu = make_weights(rng, fmt, 256, 2048), make_weights(rng, fmt, 256, 2048)
    gate, up = sq.projection(wg.segment()), sq.projection(wu.segment())
    for pair_rows in ([2] if rows < 5 else [rows, 32]):
        x = dense_inputs(rng, pair_rows, 2048)
        two = run_plan(staged(256, 2048, pair_rows, 2, sq.EPILOGUE_GATE_UP), up, x, 256, gate=gate)
        one = run_plan(staged(256, 2048, pair_rows, 2, sq.EPILOGUE_GATE_UP, one_pass=1), up, x, 256, gate=gate)
        assert np.array_equal(one, two), pair_rows


@pytest.mark.parametrize("fmt", NEW_FORMATS)
@pytest.mark.parametrize("rows", [8, 24])
def test_decode_new_formats_longest_slices(fmt, rows):
    """One K partition of the row tile's longest slices (32 groups a wave: sixteen waves, 512 groups, at up to 16
    rows, where the K-quants keep fewer groups in flight; eight waves, 256 groups, past 16)."""
    rng = np.random.default_rng(300 + fmt + rows)
    n, k = 64, 16384 if rows <= 16 else 8192
    w = make_weights(rng, fmt, n, k)
    x = dense_inputs(rng, rows, k)
    got = run_plan(staged(n, k, rows, 1), sq.projection(w.segment()), x, n)
    check_decode(got, x, w, f"fmt {fmt} rows {rows} k {k}")



@pytest.mark.parametrize("fmt", NEW_FORMATS)
@pytest.mark.parametrize("rows", [1, 16])
def test_adjacent_formats_decode_full_size(fmt, rows):
    """The adjacent formats at the bench's full decode size (K = 4096, N = 14336, M = 1 and 16) under the library's
    own plan: every output against fp64 with the register tile's bound, and no worse than the reference's staged
    numerics."""
    n, k = 14336, 4096
    w = shape_weights(fmt, n, k, 50 + fmt)
    rng = np.random.default_rng(60 + fmt + rows)
    x = dense_inputs(rng, rows, k)
    proj = sq.projection(w.segment())
    plan = sq.plan_for(sq.decode_workload(n, k, rows), proj)
    got = run_plan(plan, proj, x, n)
    stats = check_decode(got, x, w, f"fmt {fmt} {n}x{k} rows {rows}")
    value, *_ = oracle.project_f64(x, w.values)
    ref = synthetic.bf16_to_f32(staged_reference(x, w))
    ref_l2 = np.linalg.norm(ref - value) / np.linalg.norm(value)
    assert stats["rel_l2"] <= ref_l2 * 1.10 + 1e-6
