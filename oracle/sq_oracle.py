"""numpy binding of the CPU oracle (sq_oracle.c) and of the reference's own CPU oracle (_ref/libsqref.so, built
from the reference checkout by oracle/Makefile when it is present). TEST INFRASTRUCTURE ONLY: imported by tests/,
by __graft_entry__.smoke() as the checker and by bench.py's cpu_baseline leg, never by the product path.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
from ctypes import POINTER, c_double, c_float, c_int, c_uint8, c_uint16, c_uint32, c_uint64

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "libsq_oracle.so"
REFERENCE_LIBRARY = ORACLE_DIR / "_ref" / "libsqref.so"

FMT_Q4K, FMT_AF4G32, FMT_AF4G64, FMT_AF4G128 = 0, 25, 26, 27
FMT_Q5K, FMT_Q6K, FMT_Q80, FMT_AF8G64 = 3, 4, 6, 35

_lib = None
_ref = None


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(POINTER(ctype)) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is not built (make -C oracle)")
        _lib = ctypes.CDLL(str(LIBRARY))
        _lib.sqo_projection_bound.restype = c_double
        _lib.sqo_projection_bound.argtypes = [c_double, c_double, c_double, c_int]
        _lib.sqo_cpu_matmul.restype = c_double
        _lib.sqo_group_routes.restype = c_uint32
        _lib.sqo_tile_index.restype = c_uint64
        _lib.sqo_f32_to_f16.restype = c_uint16
        _lib.sqo_f32_to_f16.argtypes = [c_float]
    return _lib


def reference():
    """The reference's own CPU oracle, or None when it was not built (no reference checkout)."""
    global _ref
    if _ref is None and REFERENCE_LIBRARY.exists():
        _ref = ctypes.CDLL(str(REFERENCE_LIBRARY))
        _ref.sqref_projection_bound.restype = c_double
        _ref.sqref_projection_bound.argtypes = [c_double, c_double, c_double, c_int]
        _ref.sqref_tile_index.restype = c_uint64
        _ref.sqref_f2h.restype = c_uint16
        _ref.sqref_f2h.argtypes = [c_float]
    return _ref


def format_info(fmt: int) -> dict:
    out = (c_uint32 * 7)()
    if lib().sqo_format_info(fmt, out) != 0:
        raise ValueError(f"format {fmt} not in the oracle")
    keys = ("ggml_type", "block_elements", "block_bytes", "plane0_bytes", "plane1_bytes", "meta_bytes", "meta_groups")
    return dict(zip(keys, list(out)))


def row_bytes(fmt: int, k: int) -> int:
    f = format_info(fmt)
    return k // f["block_elements"] * f["block_bytes"]


def plane_sizes(fmt: int, n: int, k: int) -> tuple[int, int]:
    f = format_info(fmt)
    g = k // 32
    return n * g * f["plane0_bytes"], n * (g // f["meta_groups"]) * f["meta_bytes"]


def plane1_size(fmt: int, n: int, k: int) -> int:
    return n * (k // 32) * format_info(fmt)["plane1_bytes"]


def mlx_native(fmt: int, weight: np.ndarray, scales: np.ndarray, biases: np.ndarray, rows: int, k: int) -> np.ndarray:
    native = np.zeros(rows * row_bytes(fmt, k), dtype=np.uint8)
    w = np.ascontiguousarray(weight).view(np.uint8)
    rc = lib().sqo_mlx_native(fmt, rows, k, _ptr(w, c_uint8), _ptr(np.ascontiguousarray(scales, np.uint16), c_uint16),
                              _ptr(np.ascontiguousarray(biases, np.uint16), c_uint16), _ptr(native, c_uint8))
    assert rc == 0
    return native


def repack_planes(fmt: int, native: np.ndarray, n: int, k: int):
    """(plane0, plane1 (None for a format without one), meta, fp32 values [n][k]) of native rows."""
    p0, m = plane_sizes(fmt, n, k)
    plane0, meta = np.zeros(p0, np.uint8), np.zeros(m, np.uint8)
    p1 = plane1_size(fmt, n, k)
    plane1 = np.zeros(p1, np.uint8) if p1 else None
    values = np.zeros((n, k), np.float32)
    rc = lib().sqo_repack(fmt, _ptr(np.ascontiguousarray(native, np.uint8), c_uint8), n, k, _ptr(plane0, c_uint8),
                          _ptr(plane1, c_uint8) if p1 else None, _ptr(meta, c_uint8), _ptr(values, c_float))
    assert rc == 0
    return plane0, plane1, meta, values


def repack(fmt: int, native: np.ndarray, n: int, k: int):
    """(plane0, meta, fp32 values [n][k]) of native rows of a format without a plane1."""
    plane0, plane1, meta, values = repack_planes(fmt, native, n, k)
    assert plane1 is None, "this format has a plane1: use repack_planes"
    return plane0, meta, values


def unpack(fmt: int, plane0: np.ndarray, meta: np.ndarray, n: int, k: int, plane1: np.ndarray | None = None):
    native = np.zeros(n * row_bytes(fmt, k), np.uint8)
    rc = lib().sqo_unpack(fmt, _ptr(plane0, c_uint8), _ptr(plane1, c_uint8) if plane1 is not None else None,
                          _ptr(meta, c_uint8), n, k, _ptr(native, c_uint8))
    assert rc == 0
    return native


def plane_values(fmt: int, plane0: np.ndarray, meta: np.ndarray, n: int, k: int, plane1: np.ndarray | None = None):
    """(fp32 values, fp16 bits) [n][k] decoded from the planes."""
    values, halves = np.zeros((n, k), np.float32), np.zeros((n, k), np.uint16)
    rc = lib().sqo_plane_values(fmt, _ptr(plane0, c_uint8), _ptr(plane1, c_uint8) if plane1 is not None else None,
                                _ptr(meta, c_uint8), n, k, _ptr(values, c_float), _ptr(halves, c_uint16))
    assert rc == 0
    return values, halves


def fixture(fmt: int, rows: int, k: int, seed: int) -> np.ndarray:
    native = np.zeros(rows * row_bytes(fmt, k), np.uint8)
    assert lib().sqo_fixture(fmt, rows, k, seed, _ptr(native, c_uint8)) == 0
    return native


def project_f64(x_bf16: np.ndarray, w: np.ndarray, threads: int = 8):
    """(value, magnitude, inputs, largest) fp64 [M][N] of bf16 x [M][K] against fp32 w [N][K]."""
    m, k = x_bf16.shape
    n = w.shape[0]
    outs = [np.zeros((m, n), np.float64) for _ in range(4)]
    lib().sqo_project_f64(m, n, k, _ptr(np.ascontiguousarray(x_bf16, np.uint16), c_uint16),
                          _ptr(np.ascontiguousarray(w, np.float32), c_float), *[_ptr(o, c_double) for o in outs],
                          threads)
    return tuple(outs)


def projection_bound(magnitude, inputs, largest, staged: bool) -> np.ndarray:
    """projectionBound elementwise (GgufFormatReference.hpp:794-797)."""
    accumulation = np.ldexp(inputs * largest, -16)
    return accumulation + np.ldexp(magnitude, -11) + np.ldexp(inputs, -25) if staged else accumulation


def project_staged_f32(x_bf16: np.ndarray, halves: np.ndarray, threads: int = 8) -> np.ndarray:
    m, k = x_bf16.shape
    n = halves.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().sqo_project_staged_f32(m, n, k, _ptr(np.ascontiguousarray(x_bf16, np.uint16), c_uint16),
                                 _ptr(np.ascontiguousarray(halves, np.uint16), c_uint16), _ptr(out, c_float), threads)
    return out


def cpu_matmul(fmt: int, x_bf16: np.ndarray, plane0: np.ndarray, meta: np.ndarray, n: int, threads: int):
    """(bf16 bits [M][N], seconds) of the CPU baseline."""
    m, k = x_bf16.shape
    out = np.zeros((m, n), np.uint16)
    secs = lib().sqo_cpu_matmul(fmt, m, n, k, _ptr(np.ascontiguousarray(x_bf16, np.uint16), c_uint16),
                                _ptr(plane0, c_uint8), _ptr(meta, c_uint8), _ptr(out, c_uint16), threads)
    return out, secs


class CpuPool:
    """The CPU baseline's persistent thread pool (sq_cpu.c): started once, then matmul() runs y = x W^T on it and
    returns the call's wall seconds. Buffers are reserved outside any timed call (reserve)."""

    def __init__(self, threads: int):
        L = lib()
        L.sqo_pool_create.restype = ctypes.c_void_p
        L.sqo_pool_create.argtypes = [ctypes.c_int]
        L.sqo_pool_destroy.argtypes = [ctypes.c_void_p]
        L.sqo_pool_threads.argtypes = [ctypes.c_void_p]
        L.sqo_pool_isa.restype = ctypes.c_char_p
        L.sqo_pool_isa.argtypes = [ctypes.c_void_p]
        L.sqo_pool_set_isa.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        L.sqo_pool_reserve.argtypes = [ctypes.c_void_p, c_uint32, c_uint32]
        L.sqo_pool_matmul.restype = ctypes.c_double
        L.sqo_pool_matmul.argtypes = [ctypes.c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, POINTER(c_uint16),
                                      POINTER(c_uint8), POINTER(c_uint8), POINTER(c_uint16)]
        self._lib = L
        self._pool = L.sqo_pool_create(threads)
        self.threads = L.sqo_pool_threads(self._pool)
        self.isa = L.sqo_pool_isa(self._pool).decode()

    def set_isa(self, isa: str) -> bool:
        """Runs later calls on the kernel named isa ("avx512bf16", "avx512f", "avx2+fma", "scalar"); False when the CPU
        lacks it (the pool keeps its kernel)."""
        if self._lib.sqo_pool_set_isa(self._pool, isa.encode()) != 0:
            return False
        self.isa = isa
        return True

    def reserve(self, m: int, k: int) -> None:
        if self._lib.sqo_pool_reserve(self._pool, m, k) != 0:
            raise MemoryError("CPU baseline buffer")

    def matmul(self, fmt: int, x_bf16: np.ndarray, plane0: np.ndarray, meta: np.ndarray, n: int, out=None):
        """(bf16 bits [M][N], seconds); x must be reserved for (see reserve)."""
        m, k = x_bf16.shape
        out = np.zeros((m, n), np.uint16) if out is None else out
        secs = self._lib.sqo_pool_matmul(self._pool, fmt, m, n, k,
                                         _ptr(np.ascontiguousarray(x_bf16, np.uint16), c_uint16),
                                         _ptr(plane0, c_uint8), _ptr(meta, c_uint8), _ptr(out, c_uint16))
        if secs < 0:
            raise ValueError("the CPU baseline does not take this format or shape")
        return out, secs

    def close(self) -> None:
        if self._pool:
            self._lib.sqo_pool_destroy(self._pool)
            self._pool = None

    def __del__(self):
        self.close()


ROUTER_SOFTMAX, ROUTER_SIGMOID_NORMALIZED = 0, 1


def route_select(scores: np.ndarray, top_k: int, router: int = ROUTER_SOFTMAX, shared: int = 0,
                 x_bf16: np.ndarray | None = None, scalar_gate: np.ndarray | None = None):
    """moe_route_select (moe.metal:23-104): [rows][top_k + shared] experts and fp64 weights. The shared slices'
    routes (ids experts..experts + shared - 1) follow the routed ones, weighted sigmoid(x . g) of the fp32 scalar
    gate g when one is given (moe.metal:43-67), else 1."""
    rows, experts = scores.shape
    per_row = top_k + shared
    selected = np.zeros((rows, per_row), np.uint32)
    weights = np.zeros((rows, per_row), np.float64)
    lib().sqo_route_select(rows, experts, top_k, router, per_row,
                           _ptr(np.ascontiguousarray(scores, np.float32), c_float),
                           _ptr(selected, c_uint32), _ptr(weights, c_double))
    if shared:
        selected[:, top_k:] = experts + np.arange(shared, dtype=np.uint32)
        if scalar_gate is not None:
            x = (x_bf16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            gate = 1.0 / (1.0 + np.exp(-(x @ scalar_gate.astype(np.float64))))
            weights[:, top_k:] = gate[:, None]
        else:
            weights[:, top_k:] = 1.0
    return selected, weights


LANE_ROWS = 8


def group_routes(selected: np.ndarray, experts: int, tile_rows: int, shared: int = 0, verify_rows=None):
    """moe_group_routes_phase (moe.metal:184-278) over rows of top_k routed then `shared` shared routes; with
    verify_rows (a live-row count per lane of LANE_ROWS rows) the verified grouping, which leaves the routed routes of
    rows past their lane's count out (route row ~0u)."""
    rows, per_row = selected.shape
    top_k = per_row - shared
    routed = rows * top_k
    max_tiles = min(routed // tile_rows + experts, routed) + shared * (-(-rows // tile_rows))
    tiles = np.zeros((max_tiles, 2), np.uint32)
    grouped = np.zeros(max_tiles * tile_rows, np.uint32)
    route_rows = np.zeros(rows * per_row, np.uint32)
    verify = None if verify_rows is None else np.ascontiguousarray(verify_rows, np.uint32)
    count = lib().sqo_group_routes(rows, top_k, shared, experts, tile_rows,
                                   _ptr(np.ascontiguousarray(selected), c_uint32),
                                   None if verify is None else _ptr(verify, c_uint32), LANE_ROWS,
                                   _ptr(tiles, c_uint32), _ptr(grouped, c_uint32), _ptr(route_rows, c_uint32))
    return tiles[:count], grouped[:count * tile_rows], route_rows


def f16_bits(values: np.ndarray) -> np.ndarray:
    """The oracle's float32 -> float16 (round to nearest even) of every value."""
    v = np.ascontiguousarray(values, np.float32).ravel()
    return np.array([lib().sqo_f32_to_f16(float(x)) for x in v], np.uint16).reshape(np.shape(values))


# ---------------------------------------------------------------- producers either side of the path

RMS_EPSILON = 1e-6   # SPLASH_RMS_EPSILON (runtime/metal/abi/ExecutionGeometry.h:59)


def bf16_values(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns as fp64 values (exact)."""
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def rms_norm_f64(x_bf16: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """The fp64 RMS norm of bf16 rows with the kernels' epsilon, scaled by the weights as read (fp32 values of the
    stored bf16 or F32 weights): x / sqrt(mean(x^2) + eps) * w (dev/tests/engine/NormReference.hpp:44-57)."""
    x = bf16_values(x_bf16)
    inverse = 1.0 / np.sqrt((x * x).sum(axis=1, keepdims=True) / x.shape[1] + RMS_EPSILON)
    return x * inverse * np.asarray(weights, np.float64)[None, :]


def ulp_bf16(values: np.ndarray) -> np.ndarray:
    """The spacing of bf16 at each |value| (the smallest normal's for zero and subnormals)."""
    v = np.abs(np.asarray(values, np.float64))
    exponent = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return np.ldexp(1.0, (exponent - 7).astype(np.int64))


def rounded_once_to_bf16(got_bits: np.ndarray, exact: np.ndarray) -> np.ndarray:
    """Whether each bf16 result is the exact value rounded once to bf16, up to fp32 noise well below 2^-8 of half
    an ulp (dev/tests/engine/NormReference.hpp:59-66)."""
    return np.abs(bf16_values(got_bits) - exact) <= 0.5 * ulp_bf16(exact) * (1 + 1.0 / 256)


def half_rows(x_bf16: np.ndarray):
    """The prefill tile's prepared input of bf16 rows [rows][K] (K % 32 == 0): each row times 2^-shift, shift the one
    that puts its largest magnitude in [2^15, 2^16), but at least -126 (zero rows and rows of bf16 subnormals take
    -126; infinities and NaNs count as 2^128), as fp16 bits, chunk v = 4 g + c of a row holding inputs
    32 g + 4 c .. +3 then 32 g + 16 + 4 c .. +3; and the fp32 scales 2^shift."""
    bits = np.ascontiguousarray(x_bf16, np.uint16)
    rows, k = bits.shape
    largest = (bits & 0x7FFF).max(axis=1).astype(np.int64)
    exponent = (np.minimum(largest, 0x7F80) >> 7) - 127
    shift = np.maximum(exponent - 15, -126)
    scaled = bf16_values(bits) * np.ldexp(1.0, -shift)[:, None]
    half = scaled.astype(np.float32).astype(np.float16).view(np.uint16)   # exact in fp32; one rounding to fp16
    order = np.empty(k, np.int64)
    for v in range(k // 8):
        g, c = divmod(v, 4)
        base = 32 * g + 4 * c
        order[8 * v:8 * v + 4] = np.arange(base, base + 4)
        order[8 * v + 4:8 * v + 8] = np.arange(base + 16, base + 20)
    return half[:, order], np.ldexp(1.0, shift).astype(np.float32)


def float_rows_f64(x_bf16: np.ndarray, w: np.ndarray):
    """The fp64 projection of bf16 rows onto float rows w [N][K] as read (fp32 values), and sum_k |x w| per output
    (the scale of the fp32 accumulation bound)."""
    x = bf16_values(x_bf16)
    wf = np.asarray(w, np.float64)
    return x @ wf.T, np.abs(x) @ np.abs(wf).T
