"""Shared helpers of the GPU tests: weights built on the CPU oracle and uploaded, runs through the C ABI, and the
acceptance checks of the reference's projection tests (fp64 interval per element) plus the BASELINE tolerances."""
from __future__ import annotations

import numpy as np

import splash_q4 as sq
from splash_q4 import synthetic
import sq_oracle as oracle


def torch():
    import torch as t
    return t


def to_device(array: np.ndarray):
    t = torch()
    a = np.ascontiguousarray(array)
    if a.dtype == np.uint16:
        return t.from_numpy(a.view(np.int16)).cuda()
    if a.dtype == np.uint32:
        return t.from_numpy(a.view(np.int32)).cuda()
    if a.dtype == np.uint8:
        return t.from_numpy(a).cuda()
    return t.from_numpy(a).cuda()


def to_host(tensor, dtype) -> np.ndarray:
    return tensor.cpu().numpy().view(dtype)


class Weights:
    """An n x k tensor in `fmt`: native rows, planes on the device and the oracle's fp32 values and fp16 bits."""

    def __init__(self, fmt: int, n: int, k: int, native: np.ndarray):
        self.fmt, self.n, self.k, self.native = fmt, n, k, native
        self.plane0_h, self.plane1_h, self.meta_h, self.values = oracle.repack_planes(fmt, native, n, k)
        _, self.halves = oracle.plane_values(fmt, self.plane0_h, self.meta_h, n, k, self.plane1_h)
        self.plane0, self.meta = to_device(self.plane0_h), to_device(self.meta_h)
        self.plane1 = to_device(self.plane1_h) if self.plane1_h is not None else None

    def segment(self, column_offset: int = 0) -> sq.Segment:
        return sq.segment(self.fmt, self.n, self.k, self.plane0, self.meta, column_offset, self.plane1)


class DeviceAffine:
    """An n x k MLX affine 4-bit tensor (z = -8 s, the benchmark's) repacked into planes on the device by the
    library's own load path (sq_mlx_repack, bit-exact against the oracle in test_quant_gpu), with its fp32 values
    fma(q, s, z) and their fp16 bits computed in numpy: s q and s (q - 8) have at most 12 significant bits, so the
    fp32 products and sums are exact and equal the fma. For tensors too large for the CPU repack in a test's time
    (the MoE block's 100 M-weight projections)."""

    def __init__(self, rng: np.random.Generator, n: int, k: int, group: int = 64):
        self.fmt = {32: oracle.FMT_AF4G32, 64: oracle.FMT_AF4G64, 128: oracle.FMT_AF4G128}[group]
        self.n, self.k = n, k
        codes, weight, scales, biases = synthetic.mlx_affine(rng, n, k, group, scale_sigma=0.02)
        s, z = synthetic.bf16_to_f32(scales)[:, :, None], synthetic.bf16_to_f32(biases)[:, :, None]
        self.values = (codes.reshape(n, k // group, group).astype(np.float32) * s + z).reshape(n, k)
        self.halves = self.values.astype(np.float16).view(np.uint16)
        t = torch()
        p0_bytes, meta_bytes = sq.plane_bytes(self.fmt, n, k)
        self.plane0 = t.zeros(p0_bytes, dtype=t.uint8, device="cuda")
        self.meta = t.zeros(meta_bytes, dtype=t.uint8, device="cuda")
        self.plane1 = None
        sq.mlx_repack(self.fmt, n, k, to_device(weight), to_device(scales), to_device(biases), self.plane0, self.meta)
        t.cuda.synchronize()

    def segment(self, column_offset: int = 0) -> sq.Segment:
        return sq.segment(self.fmt, self.n, self.k, self.plane0, self.meta, column_offset, self.plane1)


def affine_native(rng: np.random.Generator, fmt: int, n: int, k: int, centred: bool = False) -> np.ndarray:
    """Native rows of an af4 format: z = -8 s (the benchmark's), or z centring the codes at a random point
    (the reference's makeAffineNative)."""
    group = {oracle.FMT_AF4G32: 32, oracle.FMT_AF4G64: 64, oracle.FMT_AF4G128: 128}[fmt]
    codes, weight, scales, biases = synthetic.mlx_affine(rng, n, k, group, scale_sigma=0.02)
    if centred:
        s = synthetic.bf16_to_f32(scales)
        biases = synthetic.bf16_bits(-s * 15 * rng.uniform(0.4, 0.6, size=s.shape).astype(np.float32))
    return oracle.mlx_native(fmt, weight, scales, biases, n, k)


def make_weights(rng, fmt: int, n: int, k: int, centred: bool = False) -> Weights:
    if fmt == oracle.FMT_Q4K:
        return Weights(fmt, n, k, synthetic.q4k_native(rng, n, k).ravel())
    if fmt in (oracle.FMT_Q5K, oracle.FMT_Q6K, oracle.FMT_Q80):
        return Weights(fmt, n, k, synthetic.gguf_native(rng, fmt, n, k).ravel())
    if fmt == oracle.FMT_AF8G64:
        codes, weight, scales, biases = synthetic.mlx_affine(rng, n, k, 64, scale_sigma=0.02 / 16, bits=8)
        return Weights(fmt, n, k, oracle.mlx_native(fmt, weight, scales, biases, n, k))
    return Weights(fmt, n, k, affine_native(rng, fmt, n, k, centred))


def dense_inputs(rng, rows: int, k: int) -> np.ndarray:
    return synthetic.activations(rng, rows, k)


def sparse_inputs(rows: int, k: int, magnitude: float = 1e5) -> np.ndarray:
    """One +-magnitude entry per 256 inputs, past half's range (gguf_projection_test.mm:156-169)."""
    x = np.zeros((rows, k), np.float32)
    for r in range(rows):
        for b in range(k // 256):
            x[r, b * 256 + (r * 31 + b * 97) % 256] = -magnitude if (r + b) % 2 else magnitude
    return synthetic.bf16_bits(x)


def bf16(values) -> np.ndarray:
    return synthetic.bf16_to_f32(synthetic.bf16_bits(np.asarray(values, np.float32)))


def check_projection(got_bf16: np.ndarray, x: np.ndarray, weights, what: str,
                     residual: np.ndarray | None = None, staged: bool = True, columns=None) -> dict:
    """Every output inside [bf16(v - e), bf16(v + e)] of its fp64 value v and projectionBound e, and the BASELINE
    tolerances: rel-L2 <= 1e-2 and max-abs <= 2^-6 max|row| against fp64. staged: the bound of the reference's staged
    tile (fp16 weights: the prefill tile); else the register tile's, accumulation alone (GgufFormatReference.hpp:
    787-797), which the decode tiles' exact operands meet. columns: the output columns `got_bf16` holds (all by
    default). Returns error statistics."""
    if not isinstance(weights, (list, tuple)):
        weights = [weights]
    w = np.concatenate([wt.values for wt in weights], axis=0)
    if columns is not None:
        w = w[columns]
    value, magnitude, inputs, largest = oracle.project_f64(x, w)
    bound = oracle.projection_bound(magnitude, inputs, largest, staged)
    lo, hi = value - bound, value + bound
    if residual is not None:
        res = synthetic.bf16_to_f32(residual).astype(np.float64)
        lo = (lo.astype(np.float32) + res.astype(np.float32)).astype(np.float64)
        hi = (hi.astype(np.float32) + res.astype(np.float32)).astype(np.float64)
        value = value + res
    got = synthetic.bf16_to_f32(got_bf16).astype(np.float64)
    inside = (got >= bf16(lo)) & (got <= bf16(hi)) & np.isfinite(got)
    assert inside.all(), f"{what}: {np.count_nonzero(~inside)} outputs outside their fp64 interval, first at " \
                         f"{np.argwhere(~inside)[:3].tolist()}"
    err = got - value
    rel_l2 = np.linalg.norm(err) / max(np.linalg.norm(value), 1e-300)
    row_inf = np.abs(value).max(axis=1, keepdims=True)
    assert rel_l2 <= 1e-2, f"{what}: relative L2 {rel_l2}"
    assert np.all(np.abs(err) <= np.ldexp(row_inf, -6)), f"{what}: max-abs error past 2^-6 |row|"
    return {"rel_l2": rel_l2, "max_abs": float(np.abs(err).max())}


def staged_reference(x: np.ndarray, weights: Weights) -> np.ndarray:
    """bf16 output of the reference's staged numerics (fp16 weights, exact products, fp32 sums)."""
    return synthetic.bf16_bits(oracle.project_staged_f32(x, weights.halves))


class Run:
    """Device buffers for a projection run through sq_linear_add."""

    def __init__(self, plan: sq.LinearPlan, n: int, x: np.ndarray, out_dtype=np.uint16):
        t = torch()
        self.plan = plan
        self.rows = plan.storage_rows
        k = x.shape[1]
        xin = np.zeros((self.rows, k), np.uint16)
        xin[: x.shape[0]] = x
        self.x = to_device(xin)
        self.n = n
        self.out_dtype = out_dtype
        # Every element starts as a NaN no kernel writes (bf16 0xFFFF), so untouched outputs show.
        self.out = (t.full((self.rows, n), -1, dtype=t.int16, device="cuda") if out_dtype == np.uint16
                    else t.full((self.rows, n), float("nan"), dtype=t.float32, device="cuda"))
        self.scratch = sq.Scratch(plan)

    def output(self) -> np.ndarray:
        return to_host(self.out, self.out_dtype)
