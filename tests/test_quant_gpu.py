"""Weight preparation and dequantisation on the GPU, bit for bit against the oracle: the dequantised weights (fp32
fma(q, s, z) and the staged tiles' fp16 rounding of it, as gguf_dequant_test.mm:38-86 checks the staged dequant),
the load-time repack of native rows (gguf_repack.metal) and the MLX-tensor repack."""
import numpy as np
import pytest

import splash_q4 as sq
import sq_oracle as oracle
from helpers import Weights, affine_native, make_weights, to_device, to_host, torch
from splash_q4 import synthetic

pytestmark = pytest.mark.gpu

FORMATS = [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G128]


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.asarray(a).view(np.uint32 if a.dtype == np.float32 else a.dtype),
                          np.asarray(b).view(np.uint32 if b.dtype == np.float32 else b.dtype))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("source", ["fixture", "synthetic"])
def test_dequant_bit_exact(fmt, source):
    """N = 256, K = 1024; the fixture is the reference's (every byte random, seed 42, gguf_dequant_test.mm)."""
    n, k = 256, 1024
    if source == "fixture":
        w = Weights(fmt, n, k, oracle.fixture(fmt, n, k, 42))
    else:
        w = make_weights(np.random.default_rng(fmt), fmt, n, k)
    t = torch()
    values = t.zeros((n, k), dtype=t.float32, device="cuda")
    halves = t.zeros((n, k), dtype=t.int16, device="cuda")
    sq.dequant(w.segment(), values, halves)
    t.cuda.synchronize()
    got_v, got_h = values.cpu().numpy(), to_host(halves, np.uint16)
    nan = np.isnan(w.values)
    assert np.array_equal(np.isnan(got_v), nan)
    assert same_bits(got_v[~nan], w.values[~nan])
    want_h = oracle.f16_bits(w.values) if source == "synthetic" else w.halves
    assert np.array_equal(got_h[~nan], want_h[~nan])


@pytest.mark.parametrize("fmt", FORMATS)
def test_gguf_repack_matches_oracle(fmt):
    n, k = 192, 1024
    native = oracle.fixture(fmt, n, k, 5)
    plane0, meta, _ = oracle.repack(fmt, native, n, k)
    t = torch()
    src = to_device(native)
    dst = t.zeros(plane0.size + meta.size, dtype=t.uint8, device="cuda")
    sq.gguf_repack(src, dst, n, k, fmt, oracle.row_bytes(fmt, k), plane0.size)
    t.cuda.synchronize()
    out = dst.cpu().numpy()
    assert np.array_equal(out[: plane0.size], plane0)
    assert np.array_equal(out[plane0.size:], meta)


@pytest.mark.parametrize("group,fmt", [(32, oracle.FMT_AF4G32), (64, oracle.FMT_AF4G64), (128, oracle.FMT_AF4G128)])
def test_mlx_repack_matches_oracle(group, fmt):
    rng = np.random.default_rng(group)
    n, k = 128, 2048
    codes, weight, scales, biases = synthetic.mlx_affine(rng, n, k, group)
    native = oracle.mlx_native(fmt, weight, scales, biases, n, k)
    plane0, meta, _ = oracle.repack(fmt, native, n, k)
    t = torch()
    p0 = t.zeros(plane0.size, dtype=t.uint8, device="cuda")
    m = t.zeros(meta.size, dtype=t.uint8, device="cuda")
    sq.mlx_repack(fmt, n, k, to_device(weight), to_device(scales), to_device(biases), p0, m)
    t.cuda.synchronize()
    assert np.array_equal(p0.cpu().numpy(), plane0)
    assert np.array_equal(m.cpu().numpy(), meta)


def test_repack_rejects_bad_chunks():
    t = torch()
    src = t.zeros(1024, dtype=t.uint8, device="cuda")
    with pytest.raises(sq.InvalidArgument, match="whole plane tiles"):
        sq.gguf_repack(src, src, 10, 256, oracle.FMT_AF4G64, 144, 0)
    with pytest.raises(sq.InvalidArgument, match="repack source"):
        sq.gguf_repack(src, src, 64, 256, oracle.FMT_AF4G64, 144, 64 * 8 * 16)


def test_stream_read_folds_every_word():
    """The measurement stream reads every 16-byte vector of its share: thread g of the grid folds vectors g, g + S,
    g + 2S, ... (S the launch width; pairs, then a last single), and records itself in its workgroup's sink word only
    when they fold to the marker word. Chosen threads get vectors that fold to it only if every one is read, the
    others zeros (4 workgroups of 256 threads over 5000 vectors, not a multiple of the width; thread 5 ends on a
    single, thread 1023 on a pair)."""
    t = torch()
    rng = np.random.default_rng(21)
    grid, threads, n, marker = 4, 256, 5000, 0x9E3779B9
    stride = grid * threads
    words = np.zeros((n, 4), np.uint32)
    picks = [5, 256 + 200, 1023]
    for g in picks:
        share = np.arange(g, n, stride)
        words[share] = rng.integers(0, 2**32, size=(len(share), 4), dtype=np.uint32)
        words[share[-1], 0] ^= np.bitwise_xor.reduce(words[share].ravel()) ^ np.uint32(marker)
        assert np.bitwise_xor.reduce(words[share].ravel()) == marker
        assert np.bitwise_xor.reduce(words[share[:-1]].ravel()) != marker
    src = to_device(words.reshape(-1).view(np.uint8))
    sink = t.zeros(grid, dtype=t.int32, device="cuda")
    sq.stream_read(src, sink, grid, threads)
    want = [0] * grid
    for g in picks:
        want[g // threads] = g % threads + 1
    assert to_host(sink, np.int32).tolist() == want


NEW_FORMATS = [oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64]


@pytest.mark.parametrize("fmt", NEW_FORMATS)
@pytest.mark.parametrize("source", ["fixture", "synthetic"])
def test_dequant_bit_exact_new_formats(fmt, source):
    """Q5_K, Q6_K, Q8_0 and af8g64 dequantised on the GPU: fp32 values and fp16 bits equal the oracle's (signed
    zeros included: Q6_K multiplies the exact q - 32, Q8_0 its signed byte, as the reference's staged tile does)."""
    n, k = 128, 1024
    if source == "fixture":
        native = oracle.fixture(fmt, n, k, 42)
        if fmt == oracle.FMT_AF8G64:
            native = np.random.default_rng(42).integers(0, 256, size=native.size, dtype=np.uint8)
            native = native.reshape(-1, 68)
            native[:, 1] &= 0x3F   # finite scales and biases
            native[:, 3] &= 0x3F
            native = native.ravel()
        w = Weights(fmt, n, k, native)
    else:
        w = make_weights(np.random.default_rng(fmt), fmt, n, k)
    t = torch()
    values = t.zeros((n, k), dtype=t.float32, device="cuda")
    halves = t.zeros((n, k), dtype=t.int16, device="cuda")
    sq.dequant(w.segment(), values, halves)
    t.cuda.synchronize()
    got_v, got_h = values.cpu().numpy(), to_host(halves, np.uint16)
    nan = np.isnan(w.values)
    assert np.array_equal(np.isnan(got_v), nan)
    assert same_bits(got_v[~nan], w.values[~nan])
    assert np.array_equal(got_h[~nan], w.halves[~nan])


@pytest.mark.parametrize("fmt", NEW_FORMATS)
def test_gguf_repack_new_formats(fmt):
    """The load-time repack of native rows into plane0, plane1 and meta equals the oracle's (and so the reference
    CPU oracle's) bytes."""
    n, k = 192, 1024
    native = oracle.fixture(fmt, n, k, 5)
    plane0, plane1, meta, _ = oracle.repack_planes(fmt, native, n, k)
    t = torch()
    src = to_device(native)
    p1 = plane1.size if plane1 is not None else 0
    dst = t.zeros(plane0.size + p1 + meta.size, dtype=t.uint8, device="cuda")
    sq.gguf_repack(src, dst, n, k, fmt, oracle.row_bytes(fmt, k), plane0.size + p1, dst_plane1=plane0.size)
    t.cuda.synchronize()
    out = dst.cpu().numpy()
    assert np.array_equal(out[: plane0.size], plane0)
    if plane1 is not None:
        assert np.array_equal(out[plane0.size:plane0.size + p1], plane1)
    assert np.array_equal(out[plane0.size + p1:], meta)


def test_mlx_repack_8bit():
    rng = np.random.default_rng(8)
    n, k, fmt = 128, 2048, oracle.FMT_AF8G64
    codes, weight, scales, biases = synthetic.mlx_affine(rng, n, k, 64, bits=8)
    native = oracle.mlx_native(fmt, weight, scales, biases, n, k)
    plane0, plane1, meta, _ = oracle.repack_planes(fmt, native, n, k)
    assert plane1 is None
    t = torch()
    p0 = t.zeros(plane0.size, dtype=t.uint8, device="cuda")
    m = t.zeros(meta.size, dtype=t.uint8, device="cuda")
    sq.mlx_repack(fmt, n, k, to_device(weight), to_device(scales), to_device(biases), p0, m)
    t.cuda.synchronize()
    assert np.array_equal(p0.cpu().numpy(), plane0)
    assert np.array_equal(m.cpu().numpy(), meta)


def _expert_load_layout(projections, slots):
    """ExpertLoadParams for projections [(fmt, rows, columns)] with `slots` slots each: each plane of each projection
    a run of slots in the arena, slot_bytes its plane's bytes rounded up to 256. Returns (params, arena bytes)."""
    params, at = sq.ExpertLoadParams(), 0
    for z, (fmt, rows, columns) in enumerate(projections):
        q = params.projections[z]
        q.format_id, q.rows, q.columns, q.row_bytes = fmt, rows, columns, oracle.row_bytes(fmt, columns)
        p0, m = oracle.plane_sizes(fmt, rows, columns)
        for i, need in enumerate((p0, oracle.plane1_size(fmt, rows, columns), m)):
            q.slot_bytes[i] = -(-need // 256) * 256
            q.planes[i] = at
            at += slots * q.slot_bytes[i]
    return params, at


def _expert_load(staging, arena, slots, sources, params, jobs, grid):
    sq.call("sq_moe_expert_load", sq.stream_handle(), sq.view(staging), sq.view(arena), sq.view(slots),
            sq.view(sources), sq.byref(params), jobs, sq.view(grid))


def test_moe_expert_load_matches_repack():
    """MoE::addExpertLoad (moe_expert_load, gguf_repack.metal:239-257): jobs' gate (Q4_K), up (Q5_K, with plane1)
    and down (Q6_K) native rows, staged at their sources, land in their slots' planes as the oracle's repack writes
    them; the slots of jobs past the grid's live count, the other slots and the padding keep their bytes."""
    projections = [(oracle.FMT_Q4K, 128, 512), (oracle.FMT_Q5K, 128, 512), (oracle.FMT_Q6K, 256, 256)]
    params, arena_bytes = _expert_load_layout(projections, 8)
    assert sq.lib().sq_moe_expert_load_groups(sq.byref(params)) == max(
        -(-r * (c // 32) // 256) for _, r, c in projections)
    jobs, live, slot_of = 4, 3, [5, 2, 7, 0]
    natives, sources, staged = {}, [], []
    at = 0
    for j in range(jobs):
        for z, (fmt, rows, columns) in enumerate(projections):
            natives[j, z] = oracle.fixture(fmt, rows, columns, 100 + 3 * j + z)
            at += 48   # a gap between sources
            sources.append(at)
            staged.append((at, natives[j, z]))
            at += natives[j, z].size
    staging = np.zeros(at + 64, np.uint8)
    for off, native in staged:
        staging[off: off + native.size] = native
    t = torch()
    arena = t.full((arena_bytes,), 0xAB, dtype=t.uint8, device="cuda")
    grid = to_device(np.array([sq.lib().sq_moe_expert_load_groups(sq.byref(params)), live, 3], np.uint32))
    _expert_load(to_device(staging), arena, to_device(np.array(slot_of, np.uint32)),
                 t.from_numpy(np.array(sources, np.int64)).cuda(), params, jobs, grid)
    t.cuda.synchronize()
    got = arena.cpu().numpy()
    want = np.full(arena_bytes, 0xAB, np.uint8)
    for j in range(live):
        for z, (fmt, rows, columns) in enumerate(projections):
            plane0, plane1, meta, _ = oracle.repack_planes(fmt, natives[j, z], rows, columns)
            q = params.projections[z]
            for i, plane in enumerate((plane0, plane1, meta)):
                if plane is None:
                    continue
                start = q.planes[i] + slot_of[j] * q.slot_bytes[i]
                want[start: start + plane.size] = plane
    assert np.array_equal(got, want)


def test_moe_expert_load_skips_jobs_outside_its_buffers():
    """A job whose staged rows would run past the staging buffer, or whose slot's planes would run past the arena,
    writes nothing; a projection of no rows is skipped; the other jobs land as the oracle repacks them."""
    projections = [(oracle.FMT_AF4G64, 64, 256), (oracle.FMT_AF4G64, 0, 256), (oracle.FMT_Q80, 64, 256)]
    params, arena_bytes = _expert_load_layout(projections, 2)
    natives = [oracle.fixture(fmt, max(rows, 64), columns, 7 + z) for z, (fmt, rows, columns) in enumerate(projections)]
    staging = np.concatenate(natives)
    offsets = np.cumsum([0] + [n.size for n in natives[:-1]])
    t = torch()
    arena = t.full((arena_bytes,), 0x5A, dtype=t.uint8, device="cuda")
    # Job 0: slot 1, every source in range. Job 1: the gate's source past the staging, the down's in range but into
    # slot 9, past the arena. Job 2: slot 0, the down's source one byte short of its rows.
    sources = np.array([offsets[0], 0, offsets[2],
                        staging.size - 16, 0, offsets[2],
                        offsets[0], 0, staging.size - natives[2].size + 1], np.int64)
    slot_of = np.array([1, 9, 0], np.uint32)
    grid = to_device(np.array([sq.lib().sq_moe_expert_load_groups(sq.byref(params)), 3, 3], np.uint32))
    _expert_load(to_device(staging), arena, to_device(slot_of), t.from_numpy(sources).cuda(), params, 3, grid)
    t.cuda.synchronize()
    got = arena.cpu().numpy()
    want = np.full(arena_bytes, 0x5A, np.uint8)
    for j, z in ((0, 0), (0, 2), (2, 0)):
        fmt, rows, columns = projections[z]
        plane0, _, meta, _ = oracle.repack_planes(fmt, natives[z], rows, columns)
        q = params.projections[z]
        for i, plane in ((0, plane0), (2, meta)):
            start = q.planes[i] + int(slot_of[j]) * q.slot_bytes[i]
            want[start: start + plane.size] = plane
    assert np.array_equal(got, want)
