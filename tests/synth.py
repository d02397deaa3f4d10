"""Seeded synthetic inputs for the quantized operators, laid out as ONNX stores them."""

from __future__ import annotations

import numpy as np


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Packs unsigned values < 2^bits along the last axis, lowest bits first (the layout of
    the reference's test/support/make_op_fixtures.py:136-141 and packed.ex:3)."""
    per = 8 // bits
    q = np.asarray(q).astype(np.uint8)
    q = q.reshape(*q.shape[:-1], -1, per)
    out = np.zeros(q.shape[:-1], dtype=np.uint8)
    for i in range(per):
        out |= (q[..., i] << (bits * i)).astype(np.uint8)
    return out


def nbits_weight(rng, k: int, n: int, bits: int, block_size: int, zp: str = "packed",
                 scale_dtype=np.float16, scale_mul: float = 0.01):
    """B [N, blocks, block_size*bits/8] of uniform values, scales |N(0,1)|*scale_mul + 1e-4,
    zero points none / packed uniform / float uniform in [0, 2^bits)."""
    blocks = -(-k // block_size)
    q = rng.integers(0, 2 ** bits, (n, blocks * block_size))
    b = pack(q, bits).reshape(n, blocks, block_size * bits // 8)
    scales = (np.abs(rng.standard_normal(n * blocks)) * scale_mul + 1e-4).astype(scale_dtype)
    if zp == "packed":
        per_row = -(-blocks * bits // 8)
        zq = rng.integers(0, 2 ** bits, (n, per_row * 8 // bits))
        zero = pack(zq, bits).reshape(-1)
    elif zp == "float":
        zero = (rng.random(n * blocks) * 2 ** bits).astype(np.float32)
    else:
        zero = None
    return b, scales, zero
