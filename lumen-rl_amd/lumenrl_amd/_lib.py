"""ctypes binding of liblrq.so (the C ABI declared in include/lrq.h).

The library is loaded lazily on first use.  There is no fallback: if the
library is missing or no HIP device is present, every quantize call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblrq.so")

DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_F64 = 0, 1, 2, 3
FLAG_POW2_SCALE, FLAG_NATIVE_ARITH, FLAG_SCALE_BF16, FLAG_OUT_BF16 = 1, 2, 4, 8
FMT_FP8_BLOCK, FMT_MXFP8, FMT_MXFP4, FMT_FP8_DEQUANT, FMT_TENSOR_SCALE, FMT_COPY = 0, 1, 2, 3, 4, 5
FMT_CAST_E4M3, FMT_MXFP8_DEQUANT, FMT_MXFP4_DEQUANT = 6, 7, 8
ERR_ARG, ERR_ALIGN, ERR_CAPACITY, ERR_TABLE = -1, -2, -3, -4
STATIC_WORKSPACE_BYTES = 4 << 20  # LRQ_STATIC_WORKSPACE_BYTES


class LrqError(RuntimeError):
    """A liblrq call failed (HIP runtime error or corrupt table)."""


class LrqTensor(ctypes.Structure):
    """Mirror of ``lrq_tensor`` in include/lrq.h."""

    _fields_ = [
        ("in_", ctypes.c_void_p),
        ("codes", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("ld", ctypes.c_int64),
        ("batch_stride", ctypes.c_int64),
    ]


# name -> (restype, argtypes); every symbol of include/lrq.h
_VP, _I64, _CI, _CU = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint
SIGNATURES = {
    "lrq_fp8_block_quant": (_CI, [_VP, _CI, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _VP, _CU, _VP]),
    "lrq_fp8_block_dequant": (_CI, [_VP, _VP, _CI, _I64, _I64, _I64, _I64, _I64, _VP, _CI, _VP]),
    "lrq_mxfp8_quant": (_CI, [_VP, _CI, _I64, _I64, _I64, _VP, _VP, _VP]),
    "lrq_mxfp4_quant": (_CI, [_VP, _CI, _I64, _I64, _I64, _VP, _VP, _VP]),
    "lrq_act_qdq": (_CI, [_VP, _CI, _I64, _I64, _I64, _I64, _CU, _VP, _VP]),
    "lrq_cast_e4m3": (_CI, [_VP, _CI, _I64, _VP, _VP]),
    "lrq_mx_dequant": (_CI, [_CI, _VP, _VP, _I64, _I64, _VP, _CI, _VP]),
    "lrq_group_table_bytes": (_I64, [_CI, ctypes.POINTER(LrqTensor), _I64, _CI, _I64, _I64, _CU]),
    "lrq_group_pack": (_CI, [_CI, ctypes.POINTER(LrqTensor), _I64, _CI, _I64, _I64, _CU, _VP, _I64]),
    "lrq_quant_grouped": (_CI, [_VP, _VP, _VP]),
    "lrq_group_units": (_I64, [_VP]),
    "lrq_group_kernel": (_CI, [_VP]),
    "lrq_group_device_bytes": (_I64, [_VP]),
    "lrq_group_build_map": (_CI, [_VP, _VP, _VP]),
    "lrq_group_workspace_bytes": (_I64, [_VP]),
    "lrq_tensor_scale_grouped": (_CI, [_VP, _VP, _VP, _I64, _VP]),
    "lrq_tensor_scale_grouped_static": (_CI, [_VP, _VP, _VP]),
    "lrq_version": (ctypes.c_char_p, []),
    "lrq_last_error": (ctypes.c_char_p, []),
    "lrq_diag_e4m3_bits": (_CI, [ctypes.c_uint32, _I64, _VP, _VP]),
    "lrq_diag_bf16_bits": (_CI, [ctypes.c_uint32, _I64, _VP, _VP]),
    "lrq_diag_mx_encode": (_CI, [_CI, _VP, _VP, _VP, _I64, _VP]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load liblrq.so once; raise if it was not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise LrqError(
                        f"{LIB_PATH} is missing: build it with `make -C lumen-rl_amd` "
                        "(hipcc, gfx950) -- lumenrl_amd has no non-HIP fallback"
                    )
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def last_error() -> str:
    return (lib().lrq_last_error() or b"").decode()


def check(rc: int, what: str) -> None:
    """Turn a liblrq return code into an exception."""
    if rc == 0:
        return
    msg = f"{what}: {last_error()} (code {rc})"
    if rc in (ERR_ARG, ERR_ALIGN, ERR_CAPACITY):
        raise ValueError(msg)
    raise LrqError(msg)


def version() -> str:
    return lib().lrq_version().decode()
