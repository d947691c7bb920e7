"""Device quantization ops: thin torch wrappers over liblrq's C ABI.

Every function takes HIP device tensors (torch allocates inputs and outputs),
launches on the current torch stream of the tensor's device and returns
without synchronizing.  Formats:

* FP8 blockwise -- e4m3fn codes + one scale per ``(br, bc)`` block; (1, 128)
  is the reference's ``quantize_tensor`` layout
  (lumenrl/quantization/weight_quantizer.py:40-77), (128, 128) is the
  vLLM/ATOM ``weight_scale_inv`` layout.
* MXFP8 -- e4m3fn codes + one E8M0 byte per 1x32 group (OCP MX v1.0).
* MXFP4 -- E2M1 codes packed two per byte (element 2i in the low nibble) +
  one E8M0 byte per 1x32 group.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch
from torch import Tensor

from lumenrl_amd import _lib

_IN_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
              torch.float32: _lib.DTYPE_F32}
_ESIZE = {torch.bfloat16: 2, torch.float16: 2, torch.float32: 4}


def require_device() -> torch.device:
    """The current HIP device; raises if there is none (no CPU fallback)."""
    if not torch.cuda.is_available():
        raise RuntimeError(
            "lumenrl_amd quantization runs only on a HIP device (MI355X, gfx950); "
            "torch.cuda.is_available() is False"
        )
    return torch.device("cuda", torch.cuda.current_device())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _check_input(x: Tensor, what: str) -> None:
    if not isinstance(x, Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor, got {type(x)!r}")
    if not x.is_cuda:
        raise ValueError(f"{what}: expected a HIP device tensor, got device {x.device}")
    if x.dtype not in _IN_DTYPES:
        raise TypeError(f"{what}: unsupported input dtype {x.dtype} (bf16, fp16, fp32)")


def matrix_view(x: Tensor) -> tuple[Tensor, int, int, int, int, int]:
    """View ``x`` [..., rows, cols] as (xb, batch, rows, cols, ld, batch_stride).

    ``xb`` is a [batch, rows, cols] view sharing x's storage when x's leading
    dims collapse to one evenly spaced dim and its rows are unit-stride (so a
    slice of a larger matrix costs no copy); otherwise a contiguous copy made
    on the device.
    """
    if x.dim() == 1:
        x = x.reshape(1, -1)
    *lead, rows, cols = x.shape
    batch = 1
    for s in lead:
        batch *= int(s)
    try:
        xb = x.view(batch, rows, cols)
    except RuntimeError:
        xb = None
    if xb is not None:
        ld = xb.stride(1) if rows > 1 else cols
        bstride = xb.stride(0) if batch > 1 else rows * ld
        if ((cols == 1 or xb.stride(2) == 1) and (rows == 1 or ld >= cols)
                and (batch == 1 or bstride >= (rows - 1) * ld + cols)):
            return xb, batch, rows, cols, ld, bstride
    xb = x.contiguous().view(batch, rows, cols)
    return xb, batch, rows, cols, cols, rows * cols


def fp8_block_quant(x: Tensor, block: tuple[int, int], *, native_arith: bool = False,
                    pow2: bool = False, scale_dtype: Optional[torch.dtype] = None
                    ) -> tuple[Tensor, Tensor]:
    """Blockwise e4m3 of ``x`` [..., rows, cols]; scales [..., ceil(rows/br), ceil(cols/bc)].

    ``native_arith`` evaluates the reference's arithmetic in x's own dtype
    (quantize_tensor called on a bf16/fp16 tensor); otherwise float32
    (quantize_state_dict's upcast, weight_quantizer.py:109).  ``scale_dtype``
    torch.bfloat16 rounds float32 scales to bf16 in the kernel (the
    ``_fp8_scales`` sidecar, :111).
    """
    _check_input(x, "fp8_block_quant")
    br, bc = int(block[0]), int(block[1])
    if br < 1 or bc < 1:
        raise ValueError(f"block must be positive, got {block}")
    shape = x.shape if x.dim() >= 2 else (1,) + tuple(x.shape)
    xm, batch, rows, cols, ld, bstride = matrix_view(x)
    native = native_arith and x.dtype != torch.float32
    flags = 0
    if pow2:
        flags |= _lib.FLAG_POW2_SCALE
    if native:
        flags |= _lib.FLAG_NATIVE_ARITH
        sdt = x.dtype
    elif scale_dtype in (None, torch.float32):
        sdt = torch.float32
    elif scale_dtype == torch.bfloat16:
        flags |= _lib.FLAG_SCALE_BF16
        sdt = torch.bfloat16
    else:
        raise ValueError(f"scale_dtype must be float32 or bfloat16, got {scale_dtype}")
    codes = torch.empty(tuple(shape), dtype=torch.float8_e4m3fn, device=x.device)
    sshape = tuple(shape[:-2]) + (-(-rows // br), -(-cols // bc))
    scales = torch.empty(sshape, dtype=sdt, device=x.device)
    if codes.numel() == 0:
        return codes.reshape(x.shape), scales
    with torch.cuda.device(x.device):
        rc = _lib.lib().lrq_fp8_block_quant(
            xm.data_ptr(), _IN_DTYPES[x.dtype], batch, rows, cols, ld, bstride, br, bc,
            codes.data_ptr(), scales.data_ptr(), flags, _stream(x.device))
    _lib.check(rc, "lrq_fp8_block_quant")
    return codes.reshape(x.shape), scales


def fp8_block_dequant(codes: Tensor, scales: Tensor, block: tuple[int, int],
                      out_dtype: torch.dtype = torch.float32) -> Tensor:
    """fp32(code) * fp32(scale) per block; ``out_dtype`` float32 or bfloat16."""
    if codes.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"codes must be float8_e4m3fn, got {codes.dtype}")
    if not codes.is_cuda or not scales.is_cuda:
        raise ValueError("fp8_block_dequant expects HIP device tensors")
    if scales.dtype not in _IN_DTYPES:
        scales = scales.to(torch.float32)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
    c = codes.contiguous()
    s = scales.contiguous()
    shape = c.shape if c.dim() >= 2 else (1,) + tuple(c.shape)
    *lead, rows, cols = shape
    batch = 1
    for d in lead:
        batch *= int(d)
    br, bc = int(block[0]), int(block[1])
    need = batch * (-(-rows // br)) * (-(-cols // bc))
    if s.numel() != need:
        raise ValueError(f"scales have {s.numel()} elements, blocks need {need}")
    out = torch.empty(codes.shape, dtype=out_dtype, device=codes.device)
    if out.numel() == 0:
        return out
    with torch.cuda.device(codes.device):
        rc = _lib.lib().lrq_fp8_block_dequant(
            c.data_ptr(), s.data_ptr(), _IN_DTYPES[s.dtype], batch, rows, cols, br, bc,
            out.data_ptr(), _IN_DTYPES[out_dtype], _stream(codes.device))
    _lib.check(rc, "lrq_fp8_block_dequant")
    return out


def _mx(x: Tensor, fmt: int) -> tuple[Tensor, Tensor]:
    _check_input(x, "mx quantize")
    if x.dim() < 1 or x.shape[-1] % 32 != 0:
        raise ValueError(f"MX quantization needs the last dim to be a multiple of 32, got {tuple(x.shape)}")
    xm, batch, rows, cols, ld, bstride = matrix_view(x)
    if batch > 1 and bstride != rows * ld:
        xm, batch, rows, cols, ld, bstride = matrix_view(x.contiguous())
    rows_all = batch * rows
    lead = tuple(x.shape[:-1])
    if fmt == 8:
        codes = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    else:
        codes = torch.empty(lead + (x.shape[-1] // 2,), dtype=torch.uint8, device=x.device)
    scales = torch.empty(lead + (x.shape[-1] // 32,), dtype=torch.uint8, device=x.device)
    if x.numel() == 0:
        return codes, scales
    fn = _lib.lib().lrq_mxfp8_quant if fmt == 8 else _lib.lib().lrq_mxfp4_quant
    with torch.cuda.device(x.device):
        rc = fn(xm.data_ptr(), _IN_DTYPES[x.dtype], rows_all, cols, ld, codes.data_ptr(),
                scales.data_ptr(), _stream(x.device))
    _lib.check(rc, "lrq_mxfp8_quant" if fmt == 8 else "lrq_mxfp4_quant")
    return codes, scales


def quantize_mxfp8(x: Tensor) -> tuple[Tensor, Tensor]:
    """MXFP8: (e4m3fn codes, E8M0 uint8 scales [..., K/32])."""
    return _mx(x, 8)


def quantize_mxfp4(x: Tensor) -> tuple[Tensor, Tensor]:
    """MXFP4: (uint8 codes [..., K/2], two E2M1 per byte low nibble first; E8M0 scales)."""
    return _mx(x, 4)


def quantize_fp8_blockwise(x: Tensor, block_size: tuple[int, int] = (128, 128), *,
                           use_pow2_scale: bool = False,
                           scale_dtype: torch.dtype = torch.float32) -> tuple[Tensor, Tensor]:
    """128x128 (default) FP8 e4m3 with float32 arithmetic in the reference's op order.

    For [N, K] weights the scales are [ceil(N/128), ceil(K/128)] float32: the
    layout vLLM/ATOM per-block FP8 loaders take as ``weight_scale_inv``.  A
    [E, N, K] expert stack is quantized by one launch with scales [E, ...].
    """
    return fp8_block_quant(x, block_size, native_arith=False, pow2=use_pow2_scale,
                           scale_dtype=scale_dtype)


# ---------------------------------------------------------------------------
# grouped launches
# ---------------------------------------------------------------------------
_FMTS = {"fp8_block": _lib.FMT_FP8_BLOCK, "mxfp8": _lib.FMT_MXFP8, "mxfp4": _lib.FMT_MXFP4}


class QuantPlan:
    """One kernel launch that quantizes a whole list of weights.

    The plan allocates every output once and uploads a small descriptor table
    (tensor pointers and shapes plus a work-group -> tensor map).  ``run()``
    re-quantizes whatever the input tensors currently hold -- the RL weight-sync
    pattern, where the same parameter storage is refreshed every step.

    Inputs must be device tensors with 16-byte aligned rows (every torch
    allocation of a [N, K] weight with K % 8 == 0 qualifies).
    """

    def __init__(self, tensors: Sequence[Tensor], fmt: str = "fp8_block",
                 block_size: tuple[int, int] = (128, 128), *, use_pow2_scale: bool = False,
                 native_arith: bool = False, scale_dtype: torch.dtype = torch.float32) -> None:
        if fmt not in _FMTS:
            raise ValueError(f"fmt must be one of {sorted(_FMTS)}, got {fmt!r}")
        if not tensors:
            raise ValueError("QuantPlan needs at least one tensor")
        dt = tensors[0].dtype
        dev = tensors[0].device
        for t in tensors:
            _check_input(t, "QuantPlan")
            if t.dtype != dt or t.device != dev:
                raise ValueError("all tensors of a QuantPlan must share dtype and device")
        self.fmt = fmt
        self.device = dev
        self.inputs = list(tensors)
        self.outputs: list[tuple[Tensor, Tensor]] = []
        br, bc = (int(block_size[0]), int(block_size[1])) if fmt == "fp8_block" else (1, 32)
        flags = 0
        native = native_arith and dt != torch.float32
        if fmt == "fp8_block":
            if use_pow2_scale:
                flags |= _lib.FLAG_POW2_SCALE
            if native:
                flags |= _lib.FLAG_NATIVE_ARITH
            elif scale_dtype == torch.bfloat16:
                flags |= _lib.FLAG_SCALE_BF16
        descs = (_lib.LrqTensor * len(tensors))()
        self._views = []
        nbytes = 0
        for i, t in enumerate(tensors):
            xm, batch, rows, cols, ld, bstride = matrix_view(t)
            if xm.data_ptr() != t.data_ptr():
                raise ValueError(f"tensor {i} is not a strided matrix view; pass .contiguous()")
            self._views.append(xm)
            shape = tuple(t.shape) if t.dim() >= 2 else (1,) + tuple(t.shape)
            if fmt == "fp8_block":
                codes = torch.empty(shape, dtype=torch.float8_e4m3fn, device=dev)
                sdt = dt if native else (torch.bfloat16 if flags & _lib.FLAG_SCALE_BF16 else torch.float32)
                scales = torch.empty(shape[:-2] + (-(-rows // br), -(-cols // bc)), dtype=sdt, device=dev)
            else:
                if cols % 32:
                    raise ValueError(f"tensor {i}: last dim {cols} is not a multiple of 32")
                lead = shape[:-1]
                if fmt == "mxfp8":
                    codes = torch.empty(shape, dtype=torch.float8_e4m3fn, device=dev)
                else:
                    codes = torch.empty(lead + (cols // 2,), dtype=torch.uint8, device=dev)
                scales = torch.empty(lead + (cols // 32,), dtype=torch.uint8, device=dev)
            self.outputs.append((codes, scales))
            descs[i].in_ = xm.data_ptr()
            descs[i].codes = codes.data_ptr()
            descs[i].scales = scales.data_ptr()
            descs[i].batch, descs[i].rows, descs[i].cols = batch, rows, cols
            descs[i].ld, descs[i].batch_stride = ld, bstride
            nbytes += t.numel() * t.element_size() + codes.numel() * codes.element_size() + \
                scales.numel() * scales.element_size()
        self.algorithmic_bytes = nbytes
        L = _lib.lib()
        in_dt = _IN_DTYPES[dt]
        need = L.lrq_group_table_bytes(_FMTS[fmt], descs, len(tensors), in_dt, br, bc, flags)
        if need < 0:
            _lib.check(int(need), "lrq_group_table_bytes")
        self._host_table = torch.empty(int(need), dtype=torch.uint8, pin_memory=False)
        rc = L.lrq_group_pack(_FMTS[fmt], descs, len(tensors), in_dt, br, bc, flags,
                              self._host_table.data_ptr(), int(need))
        _lib.check(rc, "lrq_group_pack")
        self._dev_table = self._host_table.to(dev)
        self.units = int(L.lrq_group_units(self._host_table.data_ptr()))

    def run(self) -> list[tuple[Tensor, Tensor]]:
        """Enqueue the launch on the current stream; returns the (codes, scales) list."""
        with torch.cuda.device(self.device):
            rc = _lib.lib().lrq_quant_grouped(self._host_table.data_ptr(),
                                              self._dev_table.data_ptr(), _stream(self.device))
        _lib.check(rc, "lrq_quant_grouped")
        return self.outputs
