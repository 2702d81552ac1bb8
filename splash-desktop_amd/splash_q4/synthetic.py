"""Seeded synthetic inputs of the benchmark configurations (numpy; no device needed).

- Activations: bf16 (round to nearest even) of N(0, 1).
- MLX affine 4-bit weights (mlx.core.quantize layout): uint4 codes uniform in 0..15 packed 8 per uint32 along K
  (element j of a row at bits 4j of its little-endian bit string), one bf16 scale s = bf16(|N(0, 0.02)|) and bias
  z = -8 s (exact in bf16) per group, so w = s q + z.
- GGUF Q4_K native rows: random 12-byte scale fields and quants, d and dmin = fp16(|N(0, 0.01)|).
"""
from __future__ import annotations

import numpy as np


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    v = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    return ((v + np.uint32(0x7FFF) + ((v >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def activations(rng: np.random.Generator, rows: int, k: int) -> np.ndarray:
    return bf16_bits(rng.standard_normal((rows, k), dtype=np.float32))


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """uint8 codes [n][k] in 0..15 -> uint32 [n][k/8], element j at bits 4j."""
    n, k = codes.shape
    c = codes.reshape(n, k // 8, 8).astype(np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=2).astype(np.uint32)


def mlx_affine(rng: np.random.Generator, n: int, k: int, group: int = 64, scale_sigma: float = 0.02, bits: int = 4):
    """(codes uint8 [n][k], weight uint32 [n][k * bits / 32], scales bf16 bits [n][k/group], biases bf16 bits):
    bits 4 or 8, z = -2^(bits-1) s."""
    codes = rng.integers(0, 1 << bits, size=(n, k), dtype=np.uint8)
    scales = bf16_bits(np.abs(rng.standard_normal((n, k // group), dtype=np.float32)) * np.float32(scale_sigma))
    biases = bf16_bits(-float(1 << (bits - 1)) * bf16_to_f32(scales))
    weight = pack_codes(codes) if bits == 4 else np.ascontiguousarray(codes).view(np.uint32)
    return codes, weight, scales, biases


def fp16_bits(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def q4k_native(rng: np.random.Generator, n: int, k: int, sigma: float = 0.01) -> np.ndarray:
    """Native block_q4_K rows [n][k/256 * 144] bytes: d, dmin, 12 scale bytes, 128 quant bytes."""
    blocks = n * (k // 256)
    raw = rng.integers(0, 256, size=(blocks, 144), dtype=np.uint8)
    d = fp16_bits(np.abs(rng.standard_normal(blocks, dtype=np.float32)) * np.float32(sigma))
    dmin = fp16_bits(np.abs(rng.standard_normal(blocks, dtype=np.float32)) * np.float32(sigma))
    raw[:, 0:2] = d.view(np.uint8).reshape(blocks, 2)
    raw[:, 2:4] = dmin.view(np.uint8).reshape(blocks, 2)
    return raw.reshape(n, (k // 256) * 144)


# (block bytes, offset of d, offset of dmin or None) of the GGUF K-quant and Q8_0 blocks (llama.cpp's layouts).
_GGUF_BLOCKS = {3: (176, 0, 2), 4: (210, 208, None), 6: (34, 0, None)}
# The reference's realistic half scales per format (GgufFormatReference.hpp scaleRange).
_GGUF_SCALES = {3: (0.0005, 0.004), 4: (0.00002, 0.0001), 6: (0.0005, 0.004)}


def gguf_native(rng: np.random.Generator, fmt: int, n: int, k: int) -> np.ndarray:
    """Native rows of Q5_K (3), Q6_K (4) or Q8_0 (6): random bytes with half scales d (and Q5_K's dmin) drawn from
    the format's realistic range, as the reference's makeNative (GgufFormatReference.hpp:190-216) builds them."""
    size, d_at, m_at = _GGUF_BLOCKS[fmt]
    elements = 32 if fmt == 6 else 256
    blocks = n * (k // elements)
    raw = rng.integers(0, 256, size=(blocks, size), dtype=np.uint8)
    lo, hi = _GGUF_SCALES[fmt]
    raw[:, d_at:d_at + 2] = fp16_bits(rng.uniform(lo, hi, blocks).astype(np.float32)).view(np.uint8).reshape(blocks, 2)
    if m_at is not None:
        raw[:, m_at:m_at + 2] = fp16_bits(rng.uniform(lo, hi, blocks).astype(np.float32)).view(np.uint8).reshape(blocks, 2)
    return raw.reshape(n, (k // elements) * size)


def router_logits(rng: np.random.Generator, rows: int, experts: int) -> np.ndarray:
    return rng.standard_normal((rows, experts), dtype=np.float32)
