"""transmuter_amd: Transmuter's quantized-weight operators on MI355X (gfx950).

The product is libtmhip.so (hand-written HIP kernels behind the C ABI of
include/transmuter_hip.h). This package is its host side: the ctypes binding (`_lib`), device
tensors (`device`), packed MatMulNBits weights (`packed`), the operator handlers that mirror
`Transmuter.Ops.Quantized` (`quantized`), the load-time hooks of `Transmuter.move/2` (`hip`),
and a reader of ONNX graphs (`onnx_wire`).
"""

from .device import Context, DeviceTensor  # noqa: F401
from .packed import PackedWeight  # noqa: F401

__all__ = ["Context", "DeviceTensor", "PackedWeight"]
