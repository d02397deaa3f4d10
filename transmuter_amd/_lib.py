"""ctypes binding of libtmhip.so (include/transmuter_hip.h).

The library is loaded from this package's directory only. There is no fallback: when the
library is missing, `lib()` raises, and every operator of this package fails with it.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmhip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "transmuter_hip.h")

# tmh_status
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_DEVICE, ERR_OOM, ERR_NO_DEVICE = 0, 1, 2, 3, 4, 5
# tmh_dtype: ONNX TensorProto.DataType codes
F32, U8, S8, U16, S16, S32, S64, F16, BF16 = 1, 2, 3, 4, 5, 6, 7, 10, 16
# tmh_zp_kind
ZP_NONE, ZP_PACKED, ZP_FLOAT = 0, 1, 2
# tmh_qparam_mode
QPARAM_TENSOR, QPARAM_AXIS, QPARAM_BLOCKED = 0, 1, 2
# QMoE activation_type
ACTIVATIONS = {"relu": 0, "gelu": 1, "silu": 2, "identity": 3, "swiglu": 4}
# Kernel ids of the launch timeline (TMH_TL_*)
TIMELINE_KERNELS = {1: "k_gemv_dot", 2: "k_gemv_dec", 3: "k_gemm_lds", 4: "k_splitk_reduce", 5: "k_moe_gemm_f16",
                    6: "k_floor_empty", 7: "k_floor_read", 8: "k_gather_bq_rows", 9: "k_floor_read_all",
                    10: "k_floor_write", 11: "k_moe_route", 12: "k_moe_plan", 13: "k_moe_combine"}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the declarations of include/transmuter_hip.h.
SIGNATURES = {
    "tmh_abi_version": (_i, []),
    "tmh_device_count": (_i, [ctypes.POINTER(_i)]),
    "tmh_ctx_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "tmh_ctx_destroy": (None, [_vp]),
    "tmh_last_error": (ctypes.c_char_p, [_vp]),
    "tmh_ctx_stream": (_vp, [_vp]),
    "tmh_alloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "tmh_free": (_i, [_vp, _vp]),
    "tmh_upload": (_i, [_vp, _vp, _vp, _sz]),
    "tmh_download": (_i, [_vp, _vp, _vp, _sz]),
    "tmh_synchronize": (_i, [_vp, _vp]),
    "tmh_copy_2d": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    "tmh_weight_concat_nbits": (_i, [_vp, ctypes.POINTER(_vp), _i, ctypes.POINTER(_vp)]),
    "tmh_event_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "tmh_event_destroy": (_i, [_vp, _vp]),
    "tmh_event_record": (_i, [_vp, _vp, _vp]),
    "tmh_event_query": (_i, [_vp, _vp, ctypes.POINTER(_i)]),
    "tmh_event_synchronize": (_i, [_vp, _vp]),
    "tmh_event_elapsed": (_i, [_vp, _vp, _vp, ctypes.POINTER(ctypes.c_float)]),
    "tmh_graph_begin": (_i, [_vp, _vp]),
    "tmh_graph_end": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "tmh_graph_launch": (_i, [_vp, _vp, _vp]),
    "tmh_graph_destroy": (_i, [_vp, _vp]),
    "tmh_weight_upload_nbits": (_i, [_vp, _vp, _sz, _vp, _i, _sz, _vp, _i, _i, _sz, _i64, _i64, _i, _i, _i,
                                     ctypes.POINTER(_vp)]),
    "tmh_weight_free": (None, [_vp]),
    "tmh_weight_pack_nbits": (_i, [_vp, _vp, _sz, _vp, _i, _sz, _vp, _i, _i, _sz, _i64, _i64, _i, _i, _i, _vp,
                                   ctypes.POINTER(_vp)]),
    "tmh_pack_nbits_host": (_i, [_vp, _sz, _vp, _i, _sz, _vp, _i, _i, _sz, _i64, _i64, _i, _i, _i,
                                 _vp, ctypes.POINTER(_sz), _vp, ctypes.POINTER(_sz), _vp, ctypes.POINTER(_sz)]),
    "tmh_weight_info": (_i, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i),
                             ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_sz)]),
    "tmh_dequantize_nbits": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmh_matmul_nbits": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _vp, _i, _vp, _i, _i64, _vp]),
    "tmh_matmul_nbits_noalloc": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _vp, _i, _vp, _i, _i64, _vp]),
    "tmh_gather_block_quantized": (_i, [_vp, _vp, _i, _i64, _i64, _vp, _i, _i64, _vp, _i, _i64, _vp, _i, _i,
                                        _vp, _vp]),
    "tmh_dequantize_linear": (_i, [_vp, _vp, _i, _i64, _i64, _i64, _vp, _i, _vp, _i, _i, _i64, _vp, _vp]),
    "tmh_matmul_integer": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i, _vp,
                                _vp]),
    "tmh_int8_weight_prepare": (_i, [_vp, _vp, _i, _vp, _i64, _i64, _i64, _vp, ctypes.POINTER(_vp)]),
    "tmh_int8_weight_free": (None, [_vp]),
    "tmh_int8_weight_info": (_i, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_sz)]),
    "tmh_matmul_integer_prepared": (_i, [_vp, _vp, _i, _vp, _i64, _i64, _i64, _vp, _vp, _vp]),
    "tmh_dynamic_quantize_linear": (_i, [_vp, _vp, _i, _i64, _vp, _vp, _vp, _vp]),
    "tmh_upload_file": (_i, [_vp, _vp, ctypes.c_char_p, _i64, _sz]),
    "tmh_floor_empty": (_i, [_vp, _i, _vp]),
    "tmh_floor_read": (_i, [_vp, _vp, _vp, _vp]),
    "tmh_floor_read_all": (_i, [_vp, _vp, _vp, _vp]),
    "tmh_floor_write": (_i, [_vp, _vp, _sz, _vp]),
    "tmh_timeline_begin": (_i, [_vp, _vp, _i64]),
    "tmh_timeline_end": (_i, [_vp, ctypes.POINTER(_i64), _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "tmh_weight_upload_qmoe": (_i, [_vp, _vp, _sz, _vp, _i, _sz, _vp, _sz, _i64, _i64, _i64, _i, _i64, _i,
                                    ctypes.POINTER(_vp)]),
    "tmh_qmoe": (_i, [_vp, _vp, _i, _i64, _i64, _vp, _i, _i64, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                      ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp, _vp]),
}

_lock = threading.Lock()
_lib = None


class TmhError(RuntimeError):
    """A failed library call: `status` is the tmh_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class TmhArgumentError(TmhError, ValueError):
    """TMH_ERR_INVALID / TMH_ERR_UNSUPPORTED: the cases the reference raises ArgumentError for."""


def lib() -> ctypes.CDLL:
    """The loaded library. Raises when libtmhip.so has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m transmuter_amd.build`; "
                    "the quantized operators have no other implementation")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(status: int, ctx=None) -> None:
    if status == OK:
        return
    msg = lib().tmh_last_error(ctx)
    text = msg.decode() if msg else "unknown error"
    if status in (ERR_INVALID, ERR_UNSUPPORTED):
        raise TmhArgumentError(status, text)
    raise TmhError(status, text)
