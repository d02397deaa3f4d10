"""A MatMulNBits model on disk for the loader tests: B (q4, K=512, N=48, block 32) in an external
data file, f16 scales and a float bias-like param inline, small zero points static."""

from __future__ import annotations

import os

import numpy as np

import onnx_writer as w
from synth import nbits_weight

K, N, BITS, BS = 512, 48, 4, 32


def write(directory: str, seed: int = 7):
    rng = np.random.default_rng(seed)
    b, s, z = nbits_weight(rng, K, N, BITS, BS, zp="packed")
    scales = s.astype(np.float16)
    extra = rng.standard_normal(64).astype(np.float32)  # a float param the move uploads
    data = os.path.join(directory, "weights.bin")
    with open(data, "wb") as f:
        f.write(b"\0" * 100)  # the data starts at an offset
        f.write(b.tobytes())
    inits = [w.tensor("B", b, external=("weights.bin", 100)), w.tensor("scales", scales), w.tensor("zp", z),
             w.tensor("extra", extra)]
    node = w.node("MatMulNBits", ["A", "B", "scales", "zp"], ["Y"],
                  [w.attribute_int("K", K), w.attribute_int("N", N), w.attribute_int("bits", BITS),
                   w.attribute_int("block_size", BS)], domain="com.microsoft")
    path = os.path.join(directory, "model.onnx")
    with open(path, "wb") as f:
        f.write(w.model([node], inits, ["A", "B", "scales", "zp", "extra"], ["Y"]))
    return path, {"B": b, "scales": scales, "zp": z, "extra": extra}
