"""Affine n-bit weights in MLX layout, restated in numpy -- TEST INFRASTRUCTURE
ONLY (see oracle/__init__.py).

Layout (reference dsv4_kernels.py:26-29, 59-79, 241; dsv4_arena.py:169-171):
  weight  uint32 [N, K*bits/32]; value j of a row sits in word (j*bits)//32 at
          bit offset (j*bits)%32, least-significant bits first (2-bit: 16
          values per word, 4-bit: 8, 8-bit: 4). 3-bit rows are the same
          little-endian bit stream with values crossing word boundaries: 32
          values per 3 words, 8 per 3 bytes (MLX's 3-bit packing, used by the
          DSpark/MTP tier whose bit width dsv4_index.py:202-207 infers)
  scales  [N, K/group]   (bf16 or fp16)
  biases  [N, K/group]
  w[n, j] = scales[n, j//group] * q[n, j] + biases[n, j//group]

qmv is the exact (fp64) value of sum_j x_j * w[n, j]; it is what every
float path is compared against after rounding to the activation dtype.
"""

from __future__ import annotations

import numpy as np

SUPPORTED_BITS = (2, 3, 4, 8)


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """uint8 codes [..., K] -> uint32 words [..., K*bits/32]: the codes'
    bits concatenated least-significant first into one little-endian
    stream."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}")
    q = np.asarray(q, dtype=np.uint8)
    K = q.shape[-1]
    if (K * bits) % 32:
        raise ValueError("K * bits must be a multiple of 32")
    stream = np.unpackbits(q[..., None], axis=-1, bitorder="little")[..., :bits]
    stream = stream.reshape(*q.shape[:-1], K * bits)
    raw = np.packbits(stream, axis=-1, bitorder="little")
    return np.ascontiguousarray(raw).view("<u4").astype(np.uint32)


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words [..., W] -> uint8 codes [..., W*32/bits]."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.uint32).astype("<u4"))
    stream = np.unpackbits(w.view(np.uint8), axis=-1, bitorder="little")
    n = stream.shape[-1] // bits
    vals = stream[..., :n * bits].reshape(*stream.shape[:-1], n, bits)
    weights = (1 << np.arange(bits, dtype=np.uint32)).astype(np.uint32)
    return (vals.astype(np.uint32) * weights).sum(axis=-1).astype(np.uint8)


def dequant(w, scales, biases, bits: int, group: int) -> np.ndarray:
    """fp64 [N, K] dequantised matrix."""
    q = unpack(w, bits).astype(np.float64)
    s = np.repeat(np.asarray(scales, dtype=np.float64), group, axis=-1)
    b = np.repeat(np.asarray(biases, dtype=np.float64), group, axis=-1)
    return s * q + b


def qmv(x, w, scales, biases, bits: int, group: int) -> np.ndarray:
    """Exact x @ dequant(W)^T in fp64. x [..., K] -> [..., N]."""
    W = dequant(w, scales, biases, bits, group)
    return np.asarray(x, dtype=np.float64) @ W.T


# -- 16-bit float rounding --------------------------------------------------

def bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even float -> bfloat16 bit pattern (uint16)."""
    f = np.asarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out


def bf16_value(bits16) -> np.ndarray:
    return (np.asarray(bits16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(a, dtype: str) -> np.ndarray:
    """Round to bf16 / fp16 and return the value as float32 ('f32' keeps fp32;
    'f64' rounds nothing: the exact formula, for comparisons with float64
    references)."""
    if dtype == "f64":
        return np.asarray(a, dtype=np.float64)
    if dtype == "bf16":
        return bf16_value(bf16_bits(np.asarray(a, dtype=np.float64).astype(np.float32)))
    if dtype == "f16":
        return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32)
    raise ValueError(dtype)


def to_bits16(a, dtype: str) -> np.ndarray:
    """Float values (exactly representable) -> uint16 storage bits."""
    if dtype == "bf16":
        return bf16_bits(a)
    if dtype == "f16":
        return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)
    raise ValueError(dtype)


def from_bits16(u, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_value(u)
    if dtype == "f16":
        return np.asarray(u, dtype=np.uint16).view(np.float16).astype(np.float32)
    raise ValueError(dtype)
