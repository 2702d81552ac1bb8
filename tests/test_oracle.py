"""The CPU oracle pinned before it is trusted: against the reference's golden vectors (MLX's own fp32 values of its
4-bit affine quantization; llama.cpp's Q4_K dequantisation hash), against the reference's own CPU oracle compiled
from its sources (oracle/_ref, when the reference checkout was present at build time), and against closed forms
and invariants (slot permutation, tile index, repack round trip, one-hot and constant inputs)."""
import hashlib
import json
import pathlib

import numpy as np
import pytest

import sq_oracle as oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
AF4 = {32: oracle.FMT_AF4G32, 64: oracle.FMT_AF4G64, 128: oracle.FMT_AF4G128}


def _hex(s: str, dtype) -> np.ndarray:
    return np.frombuffer(bytes.fromhex(s), dtype=dtype)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_mlx_fixture_values_bit_exact(group):
    """MLX 0.32.3's reading of its own 4-bit affine quantization: codes and fp32 values fma(code, s, z), bit for
    bit (the reference's gguf_reference_test.mm:84-112 over the same fixture entries)."""
    entry = next(f for f in json.loads((GOLDEN / "mlx_affine4.json").read_text())["formats"] if f["group"] == group)
    rows, k, fmt = entry["rows"], entry["columns"], AF4[group]
    weight, scales, biases = _hex(entry["weight"], np.uint8), _hex(entry["scales"], np.uint16), _hex(entry["biases"], np.uint16)
    codes, values = _hex(entry["codes"], np.uint8).reshape(rows, k), _hex(entry["values"], np.uint32).reshape(rows, k)
    native = oracle.mlx_native(fmt, weight, scales, biases, rows, k)
    n = 64   # planes hold whole 64-row tiles: pad the two rows with zero rows
    padded = np.zeros(n * oracle.row_bytes(fmt, k), np.uint8)
    padded[: native.size] = native
    plane0, meta, got = oracle.repack(fmt, padded, n, k)
    assert np.array_equal(got[:rows].view(np.uint32), values)
    decoded, _ = oracle.plane_values(fmt, plane0, meta, n, k)
    assert np.array_equal(decoded[:rows].view(np.uint32), values)
    # the codes the native blocks hold are MLX's
    unpacked = oracle.unpack(fmt, plane0, meta, n, k)
    assert np.array_equal(unpacked[: native.size], native)
    ref = oracle.reference()
    if ref is not None:
        import ctypes
        out = np.zeros_like(native)
        ref.sqref_mlx_native(fmt, rows, k, weight.ctypes.data_as(ctypes.c_void_p), scales.ctypes.data_as(ctypes.c_void_p),
                             biases.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p))
        assert np.array_equal(out, native)
    f = oracle.format_info(fmt)
    for r in range(rows):
        for b in range(k // group):
            blk = native[(r * (k // group) + b) * f["block_bytes"]:][: f["block_bytes"]]
            nibbles = np.stack([blk[4:] & 15, blk[4:] >> 4], axis=1).ravel()
            assert np.array_equal(nibbles, codes[r, b * group:(b + 1) * group])


def test_q4k_golden_hash():
    """llama.cpp's fp32 dequantisation of the reference's Q4_K fixture (256 x 1024, seed 7): SHA-256 equal
    (gguf_reference_test.mm:21-41; goldens.json gguf_dequantization.q4k)."""
    golden = json.loads((GOLDEN / "weight_goldens.json").read_text())
    fx = golden["fixture"]
    native = oracle.fixture(oracle.FMT_Q4K, fx["rows"], fx["columns"], fx["seed"])
    _, _, values = oracle.repack(oracle.FMT_Q4K, native, fx["rows"], fx["columns"])
    assert hashlib.sha256(values.tobytes()).hexdigest() == golden["q4k"]


def _q4k_values_numpy(native: np.ndarray, min_sign: float = -1.0, swap_scale_min: bool = False,
                      high_nibble_first: bool = False) -> np.ndarray:
    """GGML's dequantize_row_q4_K restated in numpy, block by block from the native bytes (d, dmin, the 12 packed
    6-bit scale/min bytes of get_scale_min_k4, then 4 chunks of 64 values: 32 low nibbles, 32 high nibbles), value =
    d sc q - dmin mn. The arguments plant the mistakes the golden hash must catch."""
    blocks = native.reshape(-1, 144)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    sc, qs = blocks[:, 4:16].astype(np.int32), blocks[:, 16:].astype(np.int32)

    def scale_min(j):
        if j < 4:
            return sc[:, j] & 63, sc[:, j + 4] & 63
        return (sc[:, j + 4] & 15) | ((sc[:, j - 4] >> 6) << 4), (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)

    out = np.zeros((blocks.shape[0], 256), np.float32)
    for chunk in range(4):
        q = qs[:, 32 * chunk:32 * chunk + 32]
        for half in range(2):
            s, m = scale_min(2 * chunk + half)
            if swap_scale_min:
                s, m = m, s
            d1, m1 = d * s.astype(np.float32), dmin * m.astype(np.float32)
            nibble = (q >> 4) if (half == 1) != high_nibble_first else (q & 15)
            out[:, 64 * chunk + 32 * half:][:, :32] = d1[:, None] * nibble.astype(np.float32) + np.float32(min_sign) * m1[:, None]
    return out


def test_q4k_planted_error_fails_golden():
    """A second, independent restatement of the Q4_K values (numpy, from the native bytes) reproduces the golden
    hash; the same restatement with a plausible mistake planted (the min term added rather than subtracted, the
    6-bit scale and min swapped, the two nibbles of a byte swapped) does not, so the hash pins each of them."""
    golden = json.loads((GOLDEN / "weight_goldens.json").read_text())
    fx = golden["fixture"]
    native = oracle.fixture(oracle.FMT_Q4K, fx["rows"], fx["columns"], fx["seed"])
    digest = lambda v: hashlib.sha256(v.reshape(fx["rows"], fx["columns"]).tobytes()).hexdigest()
    assert digest(_q4k_values_numpy(native)) == golden["q4k"]
    _, _, values = oracle.repack(oracle.FMT_Q4K, native, fx["rows"], fx["columns"])
    assert np.array_equal(values.ravel().view(np.uint32), _q4k_values_numpy(native).ravel().view(np.uint32))
    for planted in ({"min_sign": 1.0}, {"swap_scale_min": True}, {"high_nibble_first": True}):
        assert digest(_q4k_values_numpy(native, **planted)) != golden["q4k"], planted


@pytest.mark.parametrize("fmt", [oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G64, oracle.FMT_AF4G128])
def test_fixture_and_repack_match_reference_oracle(fmt):
    """The C restatement's fixture bytes, planes and values equal the reference's own CPU oracle's on the same
    inputs (GgufFormatReference.hpp repack/makeNative, built from the reference sources into oracle/_ref)."""
    ref = oracle.reference()
    if ref is None:
        pytest.skip("oracle/_ref not built (no reference checkout when the oracle was built)")
    import ctypes
    n, k = 128, 1024
    for seed in (1, 7, 42):
        native = oracle.fixture(fmt, n, k, seed)
        theirs = np.zeros_like(native)
        assert ref.sqref_fixture(fmt, n, k, seed, theirs.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(native, theirs)
        plane0, meta, values = oracle.repack(fmt, native, n, k)
        p0, m = np.zeros_like(plane0), np.zeros_like(meta)
        v = np.zeros_like(values)
        assert ref.sqref_repack(fmt, native.ctypes.data_as(ctypes.c_void_p), n, k, p0.ctypes.data_as(ctypes.c_void_p),
                                m.ctypes.data_as(ctypes.c_void_p), v.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(plane0, p0) and np.array_equal(meta, m)
        assert np.array_equal(values.view(np.uint32), v.view(np.uint32))


@pytest.mark.parametrize("fmt", [oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G64, oracle.FMT_AF4G128])
def test_repack_round_trip_and_plane_values(fmt):
    rng = np.random.default_rng(fmt)
    n, k = 192, 512
    native = rng.integers(0, 256, size=n * oracle.row_bytes(fmt, k), dtype=np.uint8)
    plane0, meta, values = oracle.repack(fmt, native, n, k)
    assert np.array_equal(oracle.unpack(fmt, plane0, meta, n, k), native)
    decoded, halves = oracle.plane_values(fmt, plane0, meta, n, k)
    assert np.array_equal(np.isnan(decoded), np.isnan(values))
    finite = ~np.isnan(values)
    assert np.array_equal(decoded[finite].view(np.uint32), values[finite].view(np.uint32))


def test_slots_and_tile_index():
    slots = [oracle.lib().sqo_quant_slot(e) for e in range(32)]
    assert sorted(slots) == list(range(32))
    # QuantFormat.h:18-26: element e0 = 16 (p >> 1) + 4c + 2 (p & 1) of pair p in chunk c sits at slot 8c + 2p.
    for c in range(4):
        for p in range(4):
            e0 = 16 * (p >> 1) + 4 * c + 2 * (p & 1)
            assert slots[e0] == 8 * c + 2 * p and slots[e0 + 1] == 8 * c + 2 * p + 1
    rng = np.random.default_rng(3)
    ref = oracle.reference()
    for _ in range(200):
        row, blocks = int(rng.integers(0, 100000)), int(rng.integers(1, 500))
        block = int(rng.integers(0, blocks))
        want = (row // 64 * blocks + block) * 64 + row % 64
        assert oracle.lib().sqo_tile_index(row, block, blocks) == want
        if ref is not None:
            assert ref.sqref_tile_index(row, block, blocks) == want
    if ref is not None:
        assert slots == [ref.sqref_quant_slot(e) for e in range(32)]
        for fmt in (0, 25, 26, 27):
            import ctypes
            row = (ctypes.c_uint32 * 7)()
            assert ref.sqref_format_row(fmt, row) == 0
            assert list(row) == list(oracle.format_info(fmt).values())


def test_f16_conversion():
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000),
                        np.float32([0.0, -0.0, 65504.0, 65520.0, 65519.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10])])
    got = oracle.f16_bits(v)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, v.astype(np.float16).view(np.uint16))
    ref = oracle.reference()
    if ref is not None:
        assert np.array_equal(got, np.array([ref.sqref_f2h(float(x)) for x in v], np.uint16))


def test_projection_closed_forms():
    rng = np.random.default_rng(11)
    n, k = 64, 256
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = np.zeros((k, k), np.uint16)
    x[np.arange(k), np.arange(k)] = 0x3F80   # bf16 1.0: row i is e_i
    value, magnitude, inputs, largest = oracle.project_f64(x, w)
    assert np.array_equal(value, w.T.astype(np.float64))   # e_k extracts column k exactly
    assert np.allclose(inputs, 1.0) and np.allclose(largest, np.abs(w).max(axis=1)[None, :])
    ones = np.full((1, k), 0x3F80, np.uint16)
    v1, *_ = oracle.project_f64(ones, w)
    assert np.allclose(v1[0], w.astype(np.float64).sum(axis=1), rtol=0, atol=1e-12)


def test_projection_bound_matches_reference():
    ref = oracle.reference()
    rng = np.random.default_rng(2)
    for _ in range(50):
        mag, inp, big = (float(x) for x in rng.uniform(0, 1e4, 3))
        for staged in (0, 1):
            mine = float(oracle.projection_bound(np.float64(mag), np.float64(inp), np.float64(big), bool(staged)))
            assert mine == oracle.lib().sqo_projection_bound(mag, inp, big, staged)
            if ref is not None:
                assert mine == ref.sqref_projection_bound(mag, inp, big, staged)


def test_staged_emulation_within_bound():
    """The reference's staged numerics (fp16 weights, exact products, fp32 sums) lie inside projectionBound."""
    rng = np.random.default_rng(9)
    n, k, m = 128, 1024, 4
    native = oracle.fixture(oracle.FMT_AF4G64, n, k, 3)
    # realistic scales: s small, z centring the codes (makeAffineNative)
    blocks = native.reshape(-1, 36)
    s = np.abs(rng.standard_normal(blocks.shape[0])).astype(np.float32) * np.float32(0.004)
    sb = (s.view(np.uint32) >> 16).astype(np.uint16)
    zb = (((-8 * (sb.astype(np.uint32) << 16).view(np.float32)).view(np.uint32)) >> 16).astype(np.uint16)
    blocks[:, 0:2] = sb.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = zb.view(np.uint8).reshape(-1, 2)
    plane0, meta, values = oracle.repack(oracle.FMT_AF4G64, native, n, k)
    _, halves = oracle.plane_values(oracle.FMT_AF4G64, plane0, meta, n, k)
    x = (rng.standard_normal((m, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    value, magnitude, inputs, largest = oracle.project_f64(x, values)
    staged = oracle.project_staged_f32(x, halves)
    bound = oracle.projection_bound(magnitude, inputs, largest, True)
    assert np.all(np.abs(staged.astype(np.float64) - value) <= bound)


def test_route_select_ties_and_weights():
    scores = np.array([[1.0, 3.0, 3.0, 2.0, -1.0, 3.0],
                       [0.5, 0.5, 0.5, 0.5, 0.5, 0.5]], np.float32)
    selected, weights = oracle.route_select(scores, 3)
    assert selected.tolist() == [[1, 2, 5], [0, 1, 2]]
    assert np.allclose(weights.sum(axis=1), 1.0)
    assert np.allclose(weights[1], 1 / 3)


def _route_select_lanes(scores: np.ndarray, top_k: int, lanes: int = 32) -> np.ndarray:
    """The reference kernel's selection simulated lane by lane (moe.metal:77-93): lane l holds experts l, l + lanes,
    ...; each rank every lane takes its best by strict `>` from -inf (its first slot when none beats -inf), the
    wave maximum of those, and the lowest expert id among the lanes whose best equals it; the winner's score
    becomes -inf. A different formulation from the oracle's flat scan, and run at two lane counts."""
    rows, experts = scores.shape
    slots = -(-experts // lanes)
    out = np.zeros((rows, top_k), np.uint32)
    for r in range(rows):
        table = np.full((lanes, slots), -np.inf, np.float32)
        for e in range(experts):
            table[e % lanes, e // lanes] = scores[r, e]
        for rank in range(top_k):
            best = np.full(lanes, -np.inf, np.float32)
            slot = np.zeros(lanes, np.int64)
            for lane in range(lanes):
                for i in range(slots):
                    if table[lane, i] > best[lane]:
                        best[lane], slot[lane] = table[lane, i], i
            top = best.max()
            candidates = [lane + lanes * slot[lane] for lane in range(lanes) if best[lane] == top]
            winner = min(candidates)
            table[winner % lanes, winner // lanes] = -np.inf
            out[r, rank] = winner
    return out


def test_route_select_nan_and_exhausted_scores():
    """NaN scores never win; with no score above -inf left expert 0 wins (so an all-NaN row selects expert 0 every
    rank), matching the reference's lane algorithm, simulated at 32 and 64 lanes over rows with NaNs, -inf, ties and
    fewer finite scores than top_k."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    scores = np.array([[nan, 1.0, nan, 2.0, 0.5],
                       [nan, nan, nan, nan, nan],
                       [nan, 5.0, 4.0, -inf, -inf],
                       [-inf, -inf, -inf, 3.0, 3.0],
                       [1.0, 1.0, 1.0, 1.0, 1.0]], np.float32)
    selected, weights = oracle.route_select(scores, 3)
    assert selected.tolist() == [[3, 1, 4], [0, 0, 0], [1, 2, 0], [3, 4, 0], [0, 1, 2]]
    assert np.allclose(weights[0].sum(), 1.0) and np.allclose(weights[4], 1 / 3)
    rng = np.random.default_rng(12)
    for experts, top_k in ((40, 8), (70, 6), (8, 8)):
        s = rng.choice(np.array([0.0, 1.0, 2.0, -1.0, nan, -inf, inf], np.float32), size=(24, experts))
        s[::3] = rng.standard_normal((8, experts)).astype(np.float32)
        s[5] = nan
        want, _ = oracle.route_select(s, top_k)
        for lanes in (32, 64):
            assert np.array_equal(_route_select_lanes(s, top_k, lanes), want), (experts, lanes)


def test_group_routes_verified():
    """The verified grouping (moe.metal:164-173): routed routes of rows past their lane's verify count take no grouped
    row and their route row is ~0u; the live ones are grouped as if the dead ones were absent; the shared slices hold
    every row; a full count per lane is the plain grouping."""
    rng = np.random.default_rng(21)
    rows, experts, top_k, shared, tile_rows = 24, 16, 4, 1, 8
    scores = rng.standard_normal((rows, experts)).astype(np.float32)
    selected, _ = oracle.route_select(scores, top_k, oracle.ROUTER_SOFTMAX, shared)
    plain = oracle.group_routes(selected, experts, tile_rows, shared)
    full = oracle.group_routes(selected, experts, tile_rows, shared, verify_rows=[8, 8, 8])
    for a, b in zip(plain, full):
        assert np.array_equal(a, b)
    verify = np.array([3, 0, 8], np.uint32)
    tiles, grouped, route_rows = oracle.group_routes(selected, experts, tile_rows, shared, verify_rows=verify)
    per_row = top_k + shared
    live_row = np.array([r % 8 < verify[r // 8] for r in range(rows)])
    for r in range(rows):
        for k in range(per_row):
            route = r * per_row + k
            if k < top_k and not live_row[r]:
                assert route_rows[route] == 0xFFFFFFFF
            else:
                assert grouped[route_rows[route]] == route
                assert tiles[route_rows[route] // tile_rows, 0] == selected[r, k]
    # the live routes alone, grouped plainly, give the same routed tiles
    live = selected[live_row][:, :top_k]
    counts = np.bincount(live.ravel(), minlength=experts)
    routed_tiles = sum((c + tile_rows - 1) // tile_rows for c in counts)
    assert tiles.shape[0] == routed_tiles + shared * 3
    assert tiles[:routed_tiles, 1].sum() == live.size


def test_group_routes_invariants():
    rng = np.random.default_rng(4)
    rows, experts, top_k, tile_rows = 96, 16, 4, 8
    scores = rng.standard_normal((rows, experts)).astype(np.float32)
    selected, _ = oracle.route_select(scores, top_k)
    tiles, grouped, route_rows = oracle.group_routes(selected, experts, tile_rows)
    counts = np.bincount(selected.ravel(), minlength=experts)
    assert tiles.shape[0] == sum((c + tile_rows - 1) // tile_rows for c in counts)
    assert list(tiles[:, 0]) == sorted(tiles[:, 0])   # expert order
    for r, g in enumerate(route_rows):
        assert grouped[g] == r
        assert tiles[g // tile_rows, 0] == selected.ravel()[r]
    assert np.count_nonzero(grouped == 0xFFFFFFFF) == tiles.shape[0] * tile_rows - rows * top_k


def test_route_weights_closed_form():
    """Scores ln 4, ln 2, 0 (and losers) give weights 4/7, 2/7, 1/7 in rank order: a sign or index slip in the
    renormalised softmax moves them."""
    scores = np.array([[0.0, np.log(2.0), -5.0, np.log(4.0), -6.0]], np.float32)
    selected, weights = oracle.route_select(scores, 3)
    assert selected.tolist() == [[3, 1, 0]]
    assert np.allclose(weights[0], [4 / 7, 2 / 7, 1 / 7], rtol=1e-6)


def test_sigmoid_router_closed_form():
    """SigmoidNormalized: scores ln 3, 0, -ln 3 have sigmoids 3/4, 1/2, 1/4, so weights 1/2, 1/3, 1/6 in rank order;
    equal scores give 1/k each."""
    scores = np.array([[-np.log(3.0), -9.0, np.log(3.0), 0.0],
                       [0.7, 0.7, 0.7, 0.7]], np.float32)
    selected, weights = oracle.route_select(scores, 3, oracle.ROUTER_SIGMOID_NORMALIZED)
    assert selected.tolist() == [[2, 3, 0], [0, 1, 2]]
    assert np.allclose(weights[0], [1 / 2, 1 / 3, 1 / 6], rtol=1e-6)
    assert np.allclose(weights[1], 1 / 3, rtol=1e-12)


def test_shared_slice_weights():
    """Shared slices follow the routed routes with ids experts.. and weight sigmoid(x . g): x . g = 0 gives 1/2 and
    x . g = ln 3 gives 3/4; ungated slices weigh 1."""
    scores = np.array([[0.0, 1.0, 2.0], [2.0, 1.0, 0.0]], np.float32)
    x = (np.array([[1.0, -1.0, 0.0, 0.0], [0.5, 0.0, 0.0, 0.0]], np.float32).view(np.uint32) >> 16).astype(np.uint16)
    g = np.array([2.0, 2.0, 0.0, 0.0], np.float32)
    g[0] = np.float32(2 * np.log(3.0))   # row 1: 0.5 * 2 ln 3 = ln 3
    g[1] = g[0]                           # row 0: 1 * g0 - 1 * g1 = 0
    selected, weights = oracle.route_select(scores, 2, oracle.ROUTER_SOFTMAX, 1, x, g)
    assert selected.tolist() == [[2, 1, 3], [0, 1, 3]]
    assert np.allclose(weights[:, 2], [0.5, 0.75], rtol=1e-6)
    assert np.allclose(weights[:, :2].sum(axis=1), 1.0)
    selected, weights = oracle.route_select(scores, 1, oracle.ROUTER_SIGMOID_NORMALIZED, 2)
    assert selected.tolist() == [[2, 3, 4], [0, 3, 4]]
    assert np.all(weights[:, 1:] == 1.0)


def test_group_routes_with_shared_slices():
    """The shared slices' tiles follow the routed tiles, slice after slice, each of every row in order; every route
    (routed and shared) owns exactly one grouped row."""
    rng = np.random.default_rng(9)
    rows, experts, top_k, shared, tile_rows = 21, 8, 2, 2, 8
    scores = rng.standard_normal((rows, experts)).astype(np.float32)
    selected, _ = oracle.route_select(scores, top_k, oracle.ROUTER_SIGMOID_NORMALIZED, shared)
    tiles, grouped, route_rows = oracle.group_routes(selected, experts, tile_rows, shared)
    routed = sum((c + tile_rows - 1) // tile_rows
                 for c in np.bincount(selected[:, :top_k].ravel(), minlength=experts))
    shared_tiles = -(-rows // tile_rows)
    assert tiles.shape[0] == routed + shared * shared_tiles
    assert tiles[routed:, 0].tolist() == [experts + s for s in range(shared) for _ in range(shared_tiles)]
    assert tiles[routed:, 1].tolist() == [8, 8, 5] * shared
    for r, g in enumerate(route_rows):
        assert grouped[g] == r
        assert tiles[g // tile_rows, 0] == selected.ravel()[r]
    for s in range(shared):
        base = (routed + s * shared_tiles) * tile_rows
        assert grouped[base:base + rows].tolist() == [row * (top_k + shared) + top_k + s for row in range(rows)]
    assert np.count_nonzero(grouped == 0xFFFFFFFF) == tiles.shape[0] * tile_rows - rows * (top_k + shared)


@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K])
def test_cpu_baseline_matches_fp64(fmt):
    """The CPU baseline (threaded fp32 sums of the dequantised weights) agrees with the fp64 projection within the
    accumulation bound plus one bf16 rounding of the output."""
    rng = np.random.default_rng(13)
    n, k, m = 128, 1024, 3
    native = oracle.fixture(fmt, n, k, 17)
    if fmt == oracle.FMT_AF4G64:   # the fixture's raw meta bytes span bf16's range: give the groups real scales
        blocks = native.reshape(-1, 36)
        sb = ((np.abs(rng.standard_normal(blocks.shape[0])).astype(np.float32) * np.float32(0.02)).view(np.uint32)
              >> 16).astype(np.uint16)
        zb = (((np.float32(-8) * (sb.astype(np.uint32) << 16).view(np.float32)).view(np.uint32)) >> 16).astype(np.uint16)
        blocks[:, 0:2] = sb.view(np.uint8).reshape(-1, 2)
        blocks[:, 2:4] = zb.view(np.uint8).reshape(-1, 2)
    plane0, meta, values = oracle.repack(fmt, native, n, k)
    x = (rng.standard_normal((m, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    out, secs = oracle.cpu_matmul(fmt, x, plane0, meta, n, 4)
    got = (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    value, magnitude, inputs, largest = oracle.project_f64(x, values)
    bound = oracle.projection_bound(magnitude, inputs, largest, False) + np.abs(value) * 2.0 ** -8
    assert secs > 0 and np.all(np.abs(got - value) <= bound)


def _bf16(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_rms_norm_oracle_invariants():
    """rms_norm_f64 is scale-free (a missing square root or mean breaks it) and, with unit weights, leaves each row
    with mean square ms / (ms + eps) (a dropped epsilon or a sum in place of the mean breaks that)."""
    rng = np.random.default_rng(21)
    x = _bf16(rng.standard_normal((4, 256)))
    x4 = _bf16(4 * oracle.bf16_values(x))          # exact: a power of two
    ones = np.ones(256)
    a, b = oracle.rms_norm_f64(x, ones), oracle.rms_norm_f64(x4, ones)
    assert np.allclose(a, b, rtol=1e-6)
    ms = (oracle.bf16_values(x) ** 2).mean(axis=1)
    assert np.allclose((a * a).mean(axis=1), ms / (ms + oracle.RMS_EPSILON), rtol=1e-12)
    w = rng.uniform(0.5, 2.0, 256)
    assert np.allclose(oracle.rms_norm_f64(x, w), a * w[None, :], rtol=1e-15)


def test_rounded_once_to_bf16():
    """The reference's acceptance of a norm output: the exact value rounded once to bf16 passes, one ulp off fails."""
    exact = np.array([1.0 + 2 ** -9 + 2 ** -12, -3.3, 1e-3, 65.0])
    rounded = _bf16(exact)
    assert oracle.rounded_once_to_bf16(rounded, exact).all()
    assert not oracle.rounded_once_to_bf16(rounded + 1, exact).any()


def _undo_half_rows(table, scale):
    rows, k = table.shape
    back = np.empty((rows, k))
    for v in range(k // 8):
        g, c = divmod(v, 4)
        back[:, 32 * g + 4 * c:32 * g + 4 * c + 4] = table[:, 8 * v:8 * v + 4].view(np.float16)
        back[:, 32 * g + 16 + 4 * c:32 * g + 20 + 4 * c] = table[:, 8 * v + 4:8 * v + 8].view(np.float16)
    return back * scale.astype(np.float64)[:, None]


def test_half_rows_round_trip():
    """The prefill table holds each row exactly, at any magnitude: undoing the chunk order and the power of two gives
    the bf16 row back, for rows of N(0,1), a 1e5 spike, N(0,1) x 1e-5, 1e-6, 1e-8 and 1e-30, bf16 subnormals and
    zeros; each row's largest table value lies in [2^15, 2^16) (the zero and subnormal rows at the shift's floor,
    -126). A down-only shift (rows kept as they are unless past 2^16) loses the small rows, so this pins the
    direction."""
    rng = np.random.default_rng(22)
    x = rng.standard_normal((9, 128)).astype(np.float32)
    x[2, 5] = 1.0e5
    for r, s in ((3, 1e-5), (4, 1e-6), (5, 1e-8), (6, 1e-30)):
        x[r] *= np.float32(s)
    bits = _bf16(x)
    bits[7] = rng.integers(0, 128, 128).astype(np.uint16) | (rng.integers(0, 2, 128).astype(np.uint16) << 15)
    bits[8] = 0
    table, scale = oracle.half_rows(bits)
    assert np.array_equal(_undo_half_rows(table, scale), oracle.bf16_values(bits))
    largest = np.abs(table.view(np.float16).astype(np.float64)).max(axis=1)
    assert np.all((largest[:7] >= 2.0 ** 15) & (largest[:7] < 2.0 ** 16)), largest
    assert np.all(scale[7:] == np.float32(2.0 ** -126))
    assert scale[2] == np.float32(2.0 ** (16 - 15))          # 1e5 = 1.53 * 2^16
    exponent = np.floor(np.log2(np.abs(oracle.bf16_values(bits[:2])).max(axis=1)))
    assert np.array_equal(scale[:2], np.ldexp(1.0, (exponent - 15).astype(int)).astype(np.float32))
    # The planted mistake: rows kept unscaled below 2^16 do not come back for the small rows.
    values = oracle.bf16_values(bits[3:6])
    assert not np.array_equal(values.astype(np.float16).astype(np.float64), values)


def test_float_rows_exact_on_integers():
    """Small integers multiply and sum exactly: the projection equals integer arithmetic, its magnitude too."""
    rng = np.random.default_rng(23)
    xi = rng.integers(-8, 9, (5, 64))
    wi = rng.integers(-8, 9, (7, 64))
    exact, magnitude = oracle.float_rows_f64(_bf16(xi), wi.astype(np.float32))
    assert np.array_equal(exact, (xi @ wi.T).astype(np.float64))
    assert np.array_equal(magnitude, (np.abs(xi) @ np.abs(wi).T).astype(np.float64))


NEW_FORMATS = [oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80, oracle.FMT_AF8G64]


@pytest.mark.parametrize("name", ["q4k", "q5k", "q6k", "q80"])
def test_gguf_golden_hashes(name):
    """llama.cpp 7ab4ee7's fp32 dequantisation of the reference's fixture of each GGUF format (256 x 1024, seed
    7 + format id): SHA-256 equal (gguf_reference_test.mm:20-41; goldens.json gguf_dequantization)."""
    entry = json.loads((GOLDEN / "weight_goldens.json").read_text())["formats"][name]
    native = oracle.fixture(entry["id"], 256, 1024, entry["seed"])
    _, _, _, values = oracle.repack_planes(entry["id"], native, 256, 1024)
    assert hashlib.sha256(values.tobytes()).hexdigest() == entry["sha256"]


@pytest.mark.parametrize("fmt", NEW_FORMATS)
def test_new_formats_match_reference_oracle(fmt):
    """Q5_K, Q6_K, Q8_0 and af8g64: the fixture bytes, plane0, plane1, meta and values equal the reference's own
    CPU oracle's (GgufFormatReference.hpp groupPack/metaPack/repack, built into oracle/_ref)."""
    ref = oracle.reference()
    if ref is None:
        pytest.skip("oracle/_ref not built (no reference checkout when the oracle was built)")
    import ctypes
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p) if a is not None else None
    n, k = 128, 1024
    for seed in (3, 7):
        native = oracle.fixture(fmt, n, k, seed)
        theirs = np.zeros_like(native)
        assert ref.sqref_fixture(fmt, n, k, seed, ptr(theirs)) == 0
        assert np.array_equal(native, theirs)
        plane0, plane1, meta, values = oracle.repack_planes(fmt, native, n, k)
        p0, m, v = np.zeros_like(plane0), np.zeros_like(meta), np.zeros_like(values)
        p1 = np.zeros_like(plane1) if plane1 is not None else None
        assert ref.sqref_repack_planes(fmt, ptr(native), n, k, ptr(p0), ptr(p1), ptr(m), ptr(v)) == 0
        assert np.array_equal(plane0, p0) and np.array_equal(meta, m)
        assert plane1 is None or np.array_equal(plane1, p1)
        assert np.array_equal(values.view(np.uint32), v.view(np.uint32))


@pytest.mark.parametrize("fmt", NEW_FORMATS)
def test_new_formats_round_trip_and_plane_values(fmt):
    """Planes and meta hold every byte of the native blocks, and the values decoded from the planes alone equal
    the native decode's bit for bit."""
    rng = np.random.default_rng(100 + fmt)
    n, k = 128, 512
    native = oracle.fixture(fmt, n, k, 5)
    if fmt == oracle.FMT_AF8G64:
        native = rng.integers(0, 256, size=native.size, dtype=np.uint8)
    plane0, plane1, meta, values = oracle.repack_planes(fmt, native, n, k)
    assert np.array_equal(oracle.unpack(fmt, plane0, meta, n, k, plane1), native)
    decoded, halves = oracle.plane_values(fmt, plane0, meta, n, k, plane1)
    finite = ~np.isnan(values)
    assert np.array_equal(np.isnan(decoded), ~finite)
    assert np.array_equal(decoded[finite].view(np.uint32), values[finite].view(np.uint32))
    with np.errstate(over="ignore"):   # fixture values past half's range round to infinity on both sides
        assert np.array_equal(halves[finite], values[finite].astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("group", [64])
def test_mlx_fixture_values_bit_exact_8bit(group):
    """MLX 0.32.3's reading of its own 8-bit affine quantization (group 64): fp32 values fma(code, s, z) bit for
    bit from the loader's native blocks and from the planes."""
    entry = next(f for f in json.loads((GOLDEN / "mlx_affine8.json").read_text())["formats"] if f["group"] == group)
    rows, k, fmt = entry["rows"], entry["columns"], oracle.FMT_AF8G64
    weight, scales, biases = _hex(entry["weight"], np.uint8), _hex(entry["scales"], np.uint16), _hex(entry["biases"], np.uint16)
    codes, values = _hex(entry["codes"], np.uint8).reshape(rows, k), _hex(entry["values"], np.uint32).reshape(rows, k)
    native = oracle.mlx_native(fmt, weight, scales, biases, rows, k)
    n = 64
    padded = np.zeros(n * oracle.row_bytes(fmt, k), np.uint8)
    padded[: native.size] = native
    plane0, plane1, meta, got = oracle.repack_planes(fmt, padded, n, k)
    assert plane1 is None
    assert np.array_equal(got[:rows].view(np.uint32), values)
    decoded, _ = oracle.plane_values(fmt, plane0, meta, n, k)
    assert np.array_equal(decoded[:rows].view(np.uint32), values)
    f = oracle.format_info(fmt)
    for r in range(rows):
        for b in range(k // group):
            blk = native[(r * (k // group) + b) * f["block_bytes"]:][: f["block_bytes"]]
            assert np.array_equal(blk[4:], codes[r, b * group:(b + 1) * group])


@pytest.mark.parametrize("isa", ["avx512bf16", "avx512f", "avx2+fma", "scalar"])
@pytest.mark.parametrize("fmt", [oracle.FMT_AF4G64, oracle.FMT_Q4K, oracle.FMT_AF4G32, oracle.FMT_AF4G128])
@pytest.mark.parametrize("m", [1, 3, 19])
def test_cpu_pool_matches_fp64(fmt, m, isa):
    """Every kernel of the CPU baseline this host runs (thread pool; bf16 dot products, AVX-512, AVX2 or scalar)
    agrees with the fp64 projection within the accumulation bound plus one bf16 rounding of the output, for row
    counts around its eight-row blocks."""
    rng = np.random.default_rng(50 + fmt + m)
    n, k = 192, 1024
    if fmt == oracle.FMT_Q4K:
        native = oracle.fixture(fmt, n, k, 23)
    else:
        group = {oracle.FMT_AF4G32: 32, oracle.FMT_AF4G64: 64, oracle.FMT_AF4G128: 128}[fmt]
        codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
        w = np.bitwise_or.reduce(codes.reshape(n, k // 8, 8).astype(np.uint32)
                                 << (np.arange(8, dtype=np.uint32) * 4), axis=2).astype(np.uint32)
        s = (np.abs(rng.standard_normal((n, k // group))).astype(np.float32) * np.float32(0.02)).view(np.uint32) >> 16
        z = ((np.float32(-8) * (s << 16).view(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
        native = oracle.mlx_native(fmt, w, s.astype(np.uint16), z, n, k)
    plane0, meta, values = oracle.repack(fmt, native, n, k)
    x = (rng.standard_normal((m, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    pool = oracle.CpuPool(3)
    if not pool.set_isa(isa):
        pool.close()
        pytest.skip(f"this CPU has no {isa}")
    pool.reserve(m, k)
    out, secs = pool.matmul(fmt, x, plane0, meta, n)
    pool.close()
    assert secs > 0
    got = (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    value, magnitude, inputs, largest = oracle.project_f64(x, values)
    bound = oracle.projection_bound(magnitude, inputs, largest, False)
    lo, hi = value - bound, value + bound
    rb = lambda v: ((v.astype(np.float32).view(np.uint32) + 0x7FFF + ((v.astype(np.float32).view(np.uint32) >> 16) & 1))
                    >> 16 << 16).view(np.float32)
    assert np.all(got >= np.nextafter(rb(lo), -np.inf)) and np.all(got <= np.nextafter(rb(hi), np.inf))
