"""ctypes bindings for the C oracle (lrq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` as the checker.  The shipped package never
imports this module.

Arrays are numpy.  16-bit float inputs are passed as their bit patterns
(``np.uint16``) together with a dtype name, so bf16 needs no numpy support.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liblrq_oracle.so")
_LIB = None

DTYPES = {"bf16": 0, "f16": 1, "f32": 2}
ARITH = {"f32": 0, "native": 1}


def build() -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        i64, vp, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
        L.lrqo_fp8_block_quant.argtypes = [vp, ci, ci, i64, i64, i64, i64, i64, i64, i64, ci, vp, vp, ci]
        L.lrqo_fp8_block_dequant.argtypes = [vp, vp, ci, i64, i64, i64, i64, i64, vp, ci, ci]
        L.lrqo_mx_quant.argtypes = [vp, ci, i64, i64, i64, ci, vp, vp, ci]
        for name in ("lrqo_f32_to_e4m3_n", "lrqo_f32_to_e2m1_n"):
            getattr(L, name).argtypes = [vp, vp, i64]
        L.lrqo_f32_to_bf16_n.argtypes = [vp, vp, i64]
        L.lrqo_f32_to_f16_n.argtypes = [vp, vp, i64]
        L.lrqo_pow2_f32_n.argtypes = [vp, vp, i64]
        L.lrqo_pow2_f64_n.argtypes = [vp, vp, i64]
        L.lrqo_fp8_block_quant_f64.argtypes = [vp, i64, i64, i64, i64, i64, i64, i64, ci, vp, vp, ci]
        L.lrqo_f32_to_e4m3_bits_range.argtypes = [ctypes.c_uint32, i64, vp]
        L.lrqo_pow2_bf16.argtypes = [ctypes.c_uint16]
        L.lrqo_pow2_bf16.restype = ctypes.c_uint16
        L.lrqo_pow2_f16.argtypes = [ctypes.c_uint16]
        L.lrqo_pow2_f16.restype = ctypes.c_uint16
        L.lrqo_act_qdq.argtypes = [vp, ci, i64, i64, i64, ci, vp, ci]
        L.lrqo_tensor_scale.argtypes = [vp, ci, i64]
        L.lrqo_tensor_scale.restype = ctypes.c_uint32
        L.lrqo_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.lrqo_e4m3_to_f32.restype = ctypes.c_float
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _as_input(x: np.ndarray, dtype: str) -> np.ndarray:
    want = np.float32 if dtype == "f32" else np.uint16
    if dtype == "f16" and x.dtype == np.float16:
        x = x.view(np.uint16)
    x = np.ascontiguousarray(x)
    if x.dtype != want:
        raise TypeError(f"oracle input for {dtype} must be {want}, got {x.dtype}")
    return x


def fp8_block_quant(x: np.ndarray, dtype: str = "bf16", arith: str = "f32",
                    block: tuple[int, int] = (1, 128), pow2: bool = False,
                    nthreads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Blockwise e4m3 quantization of ``x`` shaped [..., rows, cols] (2-D or 3-D).

    Returns (codes uint8 [batch, rows, cols], scales [batch, ceil(rows/br), ceil(cols/bc)])
    with scales float32 for float32 arithmetic, else the 16-bit bit patterns.
    """
    if dtype == "f64":
        return _fp8_block_quant_f64(x, arith, block, pow2, nthreads)
    x = _as_input(x, dtype)
    if x.ndim == 2:
        x = x[None]
    batch, rows, cols = x.shape
    br, bc = block
    tr, tc = -(-rows // br), -(-cols // bc)
    codes = np.zeros((batch, rows, cols), np.uint8)
    cdt = "f32" if arith == "f32" else dtype
    scales = np.zeros((batch, tr, tc), np.float32 if cdt == "f32" else np.uint16)
    rc = lib().lrqo_fp8_block_quant(_ptr(x), DTYPES[dtype], ARITH[arith], batch, rows, cols,
                                    cols, rows * cols, br, bc, int(pow2), _ptr(codes),
                                    _ptr(scales), nthreads)
    if rc:
        raise ValueError("oracle rejected the arguments")
    return codes, scales


def _fp8_block_quant_f64(x, arith, block, pow2, nthreads):
    """float64 input: the reference computes in float64 (quantize_tensor on a
    float64 tensor); scales come back float64."""
    if arith != "native":
        raise ValueError("float64 input is quantized in float64 arithmetic (arith='native')")
    x = np.ascontiguousarray(x, dtype=np.float64)
    if x.ndim == 2:
        x = x[None]
    batch, rows, cols = x.shape
    br, bc = block
    tr, tc = -(-rows // br), -(-cols // bc)
    codes = np.zeros((batch, rows, cols), np.uint8)
    scales = np.zeros((batch, tr, tc), np.float64)
    rc = lib().lrqo_fp8_block_quant_f64(_ptr(x), batch, rows, cols, cols, rows * cols, br, bc,
                                        int(pow2), _ptr(codes), _ptr(scales), nthreads)
    if rc:
        raise ValueError("oracle rejected the arguments")
    return codes, scales


def pow2_f64(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty_like(x)
    lib().lrqo_pow2_f64_n(_ptr(x), _ptr(out), x.size)
    return out


def fp8_block_dequant(codes: np.ndarray, scales: np.ndarray, scale_dtype: str,
                      block: tuple[int, int] = (1, 128), out_dtype: str = "f32",
                      nthreads: int = 0) -> np.ndarray:
    codes = np.ascontiguousarray(codes)
    if codes.ndim == 2:
        codes = codes[None]
    batch, rows, cols = codes.shape
    scales = np.ascontiguousarray(scales)
    out = np.zeros((batch, rows, cols), np.float32 if out_dtype == "f32" else np.uint16)
    rc = lib().lrqo_fp8_block_dequant(_ptr(codes), _ptr(scales), DTYPES[scale_dtype], batch,
                                      rows, cols, block[0], block[1], _ptr(out),
                                      DTYPES[out_dtype], nthreads)
    if rc:
        raise ValueError("oracle rejected the arguments")
    return out


def mx_quant(x: np.ndarray, dtype: str = "bf16", fmt: int = 8,
             nthreads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """MXFP8 (fmt=8) or MXFP4 (fmt=4) of a 2-D [rows, cols] array."""
    x = _as_input(x, dtype)
    rows, cols = x.shape
    codes = np.zeros((rows, cols if fmt == 8 else cols // 2), np.uint8)
    scales = np.zeros((rows, cols // 32), np.uint8)
    rc = lib().lrqo_mx_quant(_ptr(x), DTYPES[dtype], rows, cols, cols, fmt, _ptr(codes),
                             _ptr(scales), nthreads)
    if rc:
        raise ValueError("oracle rejected the arguments")
    return codes, scales


def act_qdq(x: np.ndarray, dtype: str = "f32", block: int = 128, pow2: bool = False,
            nthreads: int = 0) -> np.ndarray:
    """_FP8W8A8Linear activation fake-quant of a 2-D [rows, cols] array -> float32."""
    x = _as_input(x, dtype)
    rows, cols = x.shape
    out = np.zeros((rows, cols), np.float32)
    rc = lib().lrqo_act_qdq(_ptr(x), DTYPES[dtype], rows, cols, block, int(pow2), _ptr(out), nthreads)
    if rc:
        raise ValueError("oracle rejected the arguments")
    return out


def tensor_scale(x: np.ndarray, dtype: str = "bf16") -> np.uint32:
    """FP8KVCacheQuantizer per-tensor scale of a whole tensor -> float32 bit pattern."""
    x = _as_input(x, dtype)
    return np.uint32(lib().lrqo_tensor_scale(_ptr(x), DTYPES[dtype], x.size))


def e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().lrqo_f32_to_e4m3_n(_ptr(x), _ptr(out), x.size)
    return out


def cast_e4m3(x: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Unscaled ``tensor.to(torch.float8_e4m3fn)`` of DynamicWeightLoader
    (lumenrl/engine/inference/weight_loader.py:19-43): widen to float32 (exact
    for bf16/fp16), then the e4m3fn encoder (RNE; past 448, inf, NaN -> 0x7F|sign)."""
    x = _as_input(x, dtype)
    if dtype == "bf16":
        f = bf16_bits_to_f32(x)
    elif dtype == "f16":
        f = x.view(np.float16).astype(np.float32)
    else:
        f = x
    return e4m3_from_f32(f)


def e4m3_from_f32_bits_range(start: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().lrqo_f32_to_e4m3_bits_range(start, n, _ptr(out))
    return out


def e2m1_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().lrqo_f32_to_e2m1_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().lrqo_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def f16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().lrqo_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def pow2_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.float32)
    lib().lrqo_pow2_f32_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
