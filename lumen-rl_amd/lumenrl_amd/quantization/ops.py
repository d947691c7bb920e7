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

import contextlib
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


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> ctypes.c_void_p:
    """The current torch stream of ``device`` as a hipStream_t."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _on(device: torch.device):
    """Make ``device`` current for a launch; a no-op when it already is."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _check_input(x: Tensor, what: str, allow_f64: bool = False) -> None:
    if not isinstance(x, Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor, got {type(x)!r}")
    if not x.is_cuda:
        raise ValueError(f"{what}: expected a HIP device tensor, got device {x.device}")
    if x.dtype not in _IN_DTYPES and not (allow_f64 and x.dtype == torch.float64):
        raise TypeError(f"{what}: unsupported input dtype {x.dtype} (bf16, fp16, fp32"
                        f"{', fp64' if allow_f64 else ''})")


def matrix_view(x: Tensor) -> tuple[Tensor, int, int, int, int, int]:
    """View ``x`` [..., rows, cols] as (xb, batch, rows, cols, ld, batch_stride).

    ``xb`` is a [batch, rows, cols] view sharing x's storage when x's leading
    dims collapse to one evenly spaced dim and its rows are unit-stride (so a
    slice of a larger matrix costs no copy); otherwise a contiguous copy made
    on the device.
    """
    if x.dim() == 2 and x.is_contiguous():  # the common case, without building a view
        rows, cols = x.shape
        return x, 1, rows, cols, cols, rows * cols
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
    (quantize_tensor called on a bf16/fp16/fp64 tensor); otherwise float32
    (quantize_state_dict's upcast, weight_quantizer.py:109).  ``scale_dtype``
    torch.bfloat16 rounds float32 scales to bf16 in the kernel (the
    ``_fp8_scales`` sidecar, :111).  float64 input takes float64 arithmetic
    only (scales float64; the quotient rounded to float32 before the e4m3
    cast, :68-71).
    """
    _check_input(x, "fp8_block_quant", allow_f64=True)
    if x.dtype == torch.float64 and not native_arith:
        raise ValueError("fp8_block_quant: float64 input is quantized in float64 arithmetic "
                         "(native_arith=True); cast it to float32 for float32 arithmetic")
    if x.dim() < 1:
        raise ValueError("fp8_block_quant expects a tensor with at least one dimension")
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
    codes = torch.empty(shape, dtype=torch.float8_e4m3fn, device=x.device)
    sshape = tuple(shape[:-2]) + (-(-rows // br), -(-cols // bc))
    scales = torch.empty(sshape, dtype=sdt, device=x.device)
    if x.dim() < 2:
        codes = codes.reshape(x.shape)
    if batch * rows * cols == 0:
        return codes, scales
    with _on(x.device):
        rc = _lib.lib().lrq_fp8_block_quant(
            xm.data_ptr(), _IN_DTYPES.get(x.dtype, _lib.DTYPE_F64), batch, rows, cols, ld, bstride,
            br, bc, codes.data_ptr(), scales.data_ptr(), flags, _stream(x.device))
    _lib.check(rc, "lrq_fp8_block_quant")
    return codes, scales


def fp8_block_dequant(codes: Tensor, scales: Tensor, block: tuple[int, int],
                      out_dtype: torch.dtype = torch.float32) -> Tensor:
    """fp32(code) * fp32(scale) per block; ``out_dtype`` float32 or bfloat16."""
    if codes.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"codes must be float8_e4m3fn, got {codes.dtype}")
    if not codes.is_cuda or not scales.is_cuda or codes.device != scales.device:
        raise ValueError("fp8_block_dequant expects codes and scales on the same HIP device")
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
    with _on(codes.device):
        rc = _lib.lib().lrq_fp8_block_dequant(
            c.data_ptr(), s.data_ptr(), _IN_DTYPES[s.dtype], batch, rows, cols, br, bc,
            out.data_ptr(), _IN_DTYPES[out_dtype], _stream(codes.device))
    _lib.check(rc, "lrq_fp8_block_dequant")
    return out


def act_qdq(x: Tensor, block: int = 128, *, pow2: bool = False,
            out: Optional[Tensor] = None) -> Tensor:
    """Activation fake-quant of the FP8 W8A8 rollout linear (fp8_rollout.py:53-72).

    ``x`` [..., K] (bf16/fp16/fp32, K % block == 0) -> float32 [prod(...), K]
    with x_dq = float32(x / s) * s per 1 x block, s = clamp(amax/448, FLT_MIN).
    ``out``: optional contiguous float32 [prod(...), K] on x's device to write into.
    """
    _check_input(x, "act_qdq")
    last = x.shape[-1]
    rows = x.numel() // last if last else 0
    xm = x.reshape(rows, last)
    if xm.stride(-1) != 1:  # any row pitch and element alignment, but unit-stride rows
        xm = xm.contiguous()
    if out is None:
        out = torch.empty((rows, last), dtype=torch.float32, device=x.device)
    elif (out.dtype != torch.float32 or tuple(out.shape) != (rows, last) or not out.is_contiguous()
          or out.device != x.device):
        raise ValueError(f"act_qdq: out must be a contiguous float32 {(rows, last)} tensor on {x.device}")
    if out.numel() == 0:
        return out
    ld = xm.stride(0) if rows > 1 else last
    with _on(x.device):
        rc = _lib.lib().lrq_act_qdq(xm.data_ptr(), _IN_DTYPES[x.dtype], rows, last, ld, int(block),
                                    _lib.FLAG_POW2_SCALE if pow2 else 0, out.data_ptr(),
                                    _stream(x.device))
    _lib.check(rc, "lrq_act_qdq")
    return out


def cast_e4m3(x: Tensor) -> Tensor:
    """``x.to(torch.float8_e4m3fn)`` on the device, unscaled (weight_loader.py:19-43):
    round to nearest even; |x| rounding past 448, +-inf and NaN give NaN."""
    _check_input(x, "cast_e4m3")
    xc = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    if x.numel() == 0:
        return out
    with _on(x.device):
        rc = _lib.lib().lrq_cast_e4m3(xc.data_ptr(), _IN_DTYPES[x.dtype], xc.numel(),
                                      out.data_ptr(), _stream(x.device))
    _lib.check(rc, "lrq_cast_e4m3")
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
    with _on(x.device):
        rc = fn(xm.data_ptr(), _IN_DTYPES[x.dtype], rows_all, cols, ld, codes.data_ptr(),
                scales.data_ptr(), _stream(x.device))
    _lib.check(rc, "lrq_mxfp8_quant" if fmt == 8 else "lrq_mxfp4_quant")
    return codes, scales


def _mx_dequant(codes: Tensor, scales: Tensor, fmt: int, out_dtype: torch.dtype) -> Tensor:
    if codes.dtype not in (torch.float8_e4m3fn, torch.uint8) or scales.dtype not in (torch.uint8,
                                                                                     torch.float8_e8m0fnu):
        raise TypeError("MX dequant takes uint8/float8_e4m3fn codes and uint8/float8_e8m0fnu scales")
    if not codes.is_cuda or codes.device != scales.device:
        raise ValueError("MX dequant expects codes and scales on the same HIP device")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
    *lead, kc = codes.shape if codes.dim() else (1,)
    cols = kc if fmt == 8 else 2 * kc
    if cols % 32 or tuple(scales.shape) != (*lead, cols // 32):
        raise ValueError(f"codes {tuple(codes.shape)} and scales {tuple(scales.shape)} are not an "
                         f"MXFP{fmt} pair")
    c = codes.contiguous().view(torch.uint8)  # read at any byte alignment
    s = scales.contiguous().view(torch.uint8)
    out = torch.empty((*lead, cols), dtype=out_dtype, device=codes.device)
    if out.numel() == 0:
        return out
    with _on(codes.device):
        rc = _lib.lib().lrq_mx_dequant(_lib.FMT_MXFP8 if fmt == 8 else _lib.FMT_MXFP4, c.data_ptr(),
                                       s.data_ptr(), out.numel() // cols, cols, out.data_ptr(),
                                       _IN_DTYPES[out_dtype], _stream(codes.device))
    _lib.check(rc, "lrq_mx_dequant")
    return out


def dequantize_mxfp8(codes: Tensor, scales: Tensor, out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """Inverse of :func:`quantize_mxfp8`: code * 2^(E-127) per 1x32 group -> ``out_dtype``."""
    return _mx_dequant(codes, scales, 8, out_dtype)


def dequantize_mxfp4(codes: Tensor, scales: Tensor, out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """Inverse of :func:`quantize_mxfp4` (codes [..., K/2], low nibble first)."""
    return _mx_dequant(codes, scales, 4, out_dtype)


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
_FMTS = {"fp8_block": _lib.FMT_FP8_BLOCK, "mxfp8": _lib.FMT_MXFP8, "mxfp4": _lib.FMT_MXFP4,
         "fp8_dequant": _lib.FMT_FP8_DEQUANT, "tensor_scale": _lib.FMT_TENSOR_SCALE,
         "copy": _lib.FMT_COPY, "cast_e4m3": _lib.FMT_CAST_E4M3,
         "mxfp8_dequant": _lib.FMT_MXFP8_DEQUANT, "mxfp4_dequant": _lib.FMT_MXFP4_DEQUANT}


class _GroupLaunch:
    """A packed descriptor table (host + device copy) for one grouped launch."""

    def __init__(self, fmt: str, descs, n: int, in_dtype: int, block: tuple[int, int],
                 flags: int, device: torch.device) -> None:
        L = _lib.lib()
        with _on(device):
            if torch.cuda.is_current_stream_capturing():
                # a captured upload would re-read this plan's pinned table on every
                # replay, after the plan (and its table) may be gone
                raise RuntimeError("build lrq plans before HIP graph capture; capture only run()")
        br, bc = int(block[0]), int(block[1])
        need = L.lrq_group_table_bytes(_FMTS[fmt], descs, n, in_dtype, br, bc, flags)
        if need < 0:
            _lib.check(int(need), "lrq_group_table_bytes")
        self.host = torch.empty(int(need), dtype=torch.uint8, pin_memory=True)
        rc = L.lrq_group_pack(_FMTS[fmt], descs, n, in_dtype, br, bc, flags,
                              self.host.data_ptr(), int(need))
        _lib.check(rc, "lrq_group_pack")
        # The device table is allocated and written on the caller's current
        # stream: stream-ordered like any torch op, so a recycled allocation
        # is never overwritten while an earlier launch may still read it.  The
        # copy is from pinned memory and does not block the host (a pageable
        # copy would wait for the stream to drain, serializing plan building,
        # e.g. every quantize_state_dict call, with the device).  Only the
        # header and descriptors travel; the device writes the work-group map
        # behind them itself (4 bytes per work-group: 8 MB for a whole 8B state).
        dev_bytes = int(L.lrq_group_device_bytes(self.host.data_ptr()))
        if dev_bytes < 0:
            _lib.check(dev_bytes, "lrq_group_device_bytes")
        self.dev = torch.empty(dev_bytes, dtype=torch.uint8, device=device)
        with _on(device):
            self.home = torch.cuda.current_stream(device)
            self.dev[: int(need)].copy_(self.host, non_blocking=True)
            rc = L.lrq_group_build_map(self.host.data_ptr(), self.dev.data_ptr(), _stream(device))
            _lib.check(rc, "lrq_group_build_map")
            self.ready = torch.cuda.Event()
            self.ready.record(self.home)
        self.device = device
        self.units = int(L.lrq_group_units(self.host.data_ptr()))
        self.buffers: list[Tensor] = [self.dev]  # device memory the launches touch
        # Set once a run is recorded into a HIP graph: the graph holds this
        # table's device address, so the table must live and stay unchanged.
        self.captured = False

    def _enter(self) -> None:
        """Order a launch on another stream after the table upload, and tell the
        allocator that stream uses the plan's buffers (so freeing the plan
        cannot recycle them under a running launch).  Inside a graph capture
        this is skipped: the upload was ordered by the uncaptured warm-up run
        that capture requires anyway."""
        cur = torch.cuda.current_stream(self.device)
        if cur == self.home or torch.cuda.is_current_stream_capturing():
            return
        cur.wait_event(self.ready)
        for b in self.buffers:
            b.record_stream(cur)

    def run(self) -> None:
        with _on(self.device):
            self._enter()
            self.captured |= torch.cuda.is_current_stream_capturing()
            rc = _lib.lib().lrq_quant_grouped(self.host.data_ptr(), self.dev.data_ptr(),
                                              _stream(self.device))
        _lib.check(rc, "lrq_quant_grouped")

    def workspace_bytes(self) -> int:
        return int(_lib.lib().lrq_group_workspace_bytes(self.host.data_ptr()))

    def run_tensor_scale(self, workspace: Tensor) -> None:
        with _on(self.device):
            self._enter()
            self.captured |= torch.cuda.is_current_stream_capturing()
            rc = _lib.lib().lrq_tensor_scale_grouped(self.host.data_ptr(), self.dev.data_ptr(),
                                                     workspace.data_ptr(), _nbytes(workspace),
                                                     _stream(self.device))
        _lib.check(rc, "lrq_tensor_scale_grouped")

    def run_tensor_scale_static(self) -> None:
        with _on(self.device):
            self._enter()
            self.captured |= torch.cuda.is_current_stream_capturing()
            rc = _lib.lib().lrq_tensor_scale_grouped_static(self.host.data_ptr(), self.dev.data_ptr(),
                                                            _stream(self.device))
        _lib.check(rc, "lrq_tensor_scale_grouped_static")


# A grouped plan over many tensors runs as several launches of consecutive
# tensors, each about this many algorithmic bytes (2 GiB of bf16 input for a
# quantization).  On an MI355X the Qwen3-8B set (252 tensors, 20.8 GB) ran
# 1-2 points of the HBM peak faster in 5-7 such launches than in one: 128x128
# 81.5-81.8 % -> 82.5-82.7 %, 1x128 83.0 % -> 85.0 %, MXFP8 84.1 % -> 84.8 %
# (14 launches: 82.0 %, 36: 79.6 %).  Splitting one 4 GiB tensor into row bands
# gained nothing, so a tensor is never split.
GROUP_LAUNCH_BYTES = 3 << 30


def launch_ranges(sizes: Sequence[int], limit: Optional[int] = None) -> list[tuple[int, int]]:
    """Consecutive ``[i, j)`` ranges of ``sizes`` (algorithmic bytes per tensor)
    whose sums stay within ``limit`` (default ``GROUP_LAUNCH_BYTES``); a tensor
    larger than the limit is a range of its own.  Every index is covered once,
    in order."""
    limit = GROUP_LAUNCH_BYTES if limit is None else limit
    out, i, acc = [], 0, 0
    for j, n in enumerate(sizes):
        if j > i and acc + n > limit:
            out.append((i, j))
            i, acc = j, 0
        acc += n
    if i < len(sizes):
        out.append((i, len(sizes)))
    return out


class _GroupLaunches:
    """A plan's grouped launches: its tensors split by ``launch_ranges`` into
    consecutive runs, each with its own table, run in order on the caller's
    stream.  ``buffers[k]`` lists tensor k's plan-owned device buffers."""

    def __init__(self, fmt: str, descs, sizes: Sequence[int], in_dtype: int, block: tuple[int, int],
                 flags: int, device: torch.device, buffers: Optional[Sequence[Sequence[Tensor]]] = None) -> None:
        self.parts: list[_GroupLaunch] = []
        for i, j in launch_ranges(sizes):
            sub = (_lib.LrqTensor * (j - i))(*descs[i:j])
            part = _GroupLaunch(fmt, sub, j - i, in_dtype, block, flags, device)
            if buffers is not None:
                part.buffers += [b for k in range(i, j) for b in buffers[k]]
            self.parts.append(part)
        # One kernel for the whole list, as one table requires of its tensors,
        # wherever the launches split it: the first tensor of the first part
        # whose kernel differs is the first tensor that differs from tensor 0.
        kinds = [int(_lib.lib().lrq_group_kernel(p.host.data_ptr())) for p in self.parts]
        for k in kinds:
            if k < 0:
                _lib.check(k, "lrq_group_kernel")
        for (i, _), k in zip(launch_ranges(sizes), kinds):
            if k != kinds[0]:
                raise ValueError(f"tensor {i} needs a different kernel than tensor 0 "
                                 "(alignment/shape); group it separately")
        self.units = sum(p.units for p in self.parts)

    @property
    def captured(self) -> bool:
        return any(p.captured for p in self.parts)

    def run(self) -> None:
        for p in self.parts:
            p.run()


class ChunkedLaunches:
    """Grouped launches issued while the caller is still collecting tensors.

    ``add(group, name, item)`` files an item under a group key such as
    (dtype, device); a group calls ``run(items) -> outputs`` as soon as it holds
    the next chunk size (8, 16, 32, then 64), so the device starts on the first
    tensors of a state dict while the host still stages and plans the rest.
    ``flush()`` runs what is left and returns ``{name: output}``.  Host tensors
    are not staged here: ``run_host_windows`` moves them in bounded windows.
    """

    def __init__(self, run, *, first: int = 8, most: int = 64) -> None:
        self._run, self._first, self._most = run, first, most
        self._groups: dict = {}
        self.results: dict = {}

    def add(self, group, name, item) -> None:
        g = self._groups.get(group)
        if g is None:
            g = self._groups[group] = {"names": [], "items": [], "next": self._first}
        g["names"].append(name)
        g["items"].append(item)
        if len(g["names"]) == g["next"]:
            self._launch(g["names"], g["items"])
            g["names"], g["items"] = [], []
            g["next"] = min(2 * g["next"], self._most)

    def _launch(self, names, items) -> None:
        self.results.update(zip(names, self._run(items)))

    def flush(self) -> dict:
        for g in self._groups.values():
            names, items = g["names"], g["items"]
            i = 0
            for chunk in launch_chunks(names, g["next"], self._most):
                self._launch(chunk, items[i:i + len(chunk)])
                i += len(chunk)
            g["names"], g["items"] = [], []
        return self.results


HOST_WINDOW_BYTES = 512 << 20  # input bytes per staging window of run_host_windows
HOST_WINDOW_DEPTH = 2          # windows holding device memory at once


def run_host_windows(items: Sequence[tuple], launch, device: torch.device, *,
                     window_bytes: Optional[int] = None, depth: Optional[int] = None) -> dict:
    """Device launches over HOST-resident inputs, in bounded pipelined windows.

    ``items``: ``[(key, (host tensor, ...)), ...]`` in order; an item may carry a
    third element, a tuple of host tensors to receive its outputs (see
    ``host_items``).  ``launch(ins)`` takes ``[(device tensor, ...), ...]`` for
    one window, enqueues the work on the current stream and returns
    ``[(device output, ...), ...]`` in the same order.  Returns
    ``{key: (host output, ...)}``: pinned CPU tensors, complete when this returns.

    Per window (inputs up to ``window_bytes``, or one larger item): the host
    copies the inputs into pinned staging buffers (torch runs large copies on
    several threads), a copy stream sends them, ``launch`` runs on the current
    stream, and a second copy stream brings the outputs back into pinned host
    tensors.  The host stages window i+1 while the device still copies and
    computes window i; at most ``depth`` windows are in flight, so the device
    holds about ``depth`` windows of inputs and outputs however large the
    state.  Both copy streams keep the default priority.  The defaults are
    the module's ``HOST_WINDOW_BYTES`` and ``HOST_WINDOW_DEPTH``.
    """
    window_bytes = HOST_WINDOW_BYTES if window_bytes is None else window_bytes
    depth = HOST_WINDOW_DEPTH if depth is None else depth
    cur = torch.cuda.current_stream(device)
    s_in, s_out = torch.cuda.Stream(device), torch.cuda.Stream(device)
    inflight: list = []
    results: dict = {}
    for window in _windows(items, window_bytes):
        if len(inflight) >= depth:
            inflight.pop(0).synchronize()
        staged = [tuple(torch.empty(t.shape, dtype=t.dtype, pin_memory=True).copy_(t) for t in it[1])
                  for it in window]
        with torch.cuda.stream(s_in):
            dev_in = [tuple(p.to(device, non_blocking=True) for p in ps) for ps in staged]
        cur.wait_stream(s_in)
        for ts in dev_in:
            for d in ts:
                d.record_stream(cur)
        outs = launch(dev_in)
        s_out.wait_stream(cur)
        with torch.cuda.stream(s_out):
            for it, os_ in zip(window, outs):
                dests = it[2] if len(it) > 2 else [None] * len(os_)
                host = []
                for o, h in zip(os_, dests):
                    if h is None:
                        h = torch.empty(o.shape, dtype=o.dtype, pin_memory=True)
                    elif tuple(h.shape) != tuple(o.shape) or h.dtype != o.dtype:
                        raise ValueError(f"{it[0]}: output {tuple(o.shape)} {o.dtype} does not fit "
                                         f"its destination {tuple(h.shape)} {h.dtype}")
                    h.copy_(o, non_blocking=True)
                    o.record_stream(s_out)
                    host.append(h)
                results[it[0]] = tuple(host)
        inflight.append(s_out.record_event())
        del staged, dev_in, outs
    s_out.synchronize()
    return results


def host_items(key, ins: tuple, outs: tuple, *, window_bytes: Optional[int] = None,
               multiple: int = 1, out_div: Optional[tuple] = None) -> list[tuple]:
    """The run_host_windows items for one host work item whose results go to
    ``outs`` (pinned host tensors of the full results).

    Inputs that fit a window make one item.  Larger ones are split along dim 0
    into chunks of a multiple of ``multiple`` rows, each chunk an item that
    writes the matching rows of ``outs``, so the device never holds more than a
    window of any tensor.  Every input has the same dim-0 length R, rows are
    independent, and output j has ceil(R / out_div[j]) rows (default 1: the
    same R; 128 for the scales of 128-row tiles, with ``multiple`` 128)."""
    window_bytes = HOST_WINDOW_BYTES if window_bytes is None else window_bytes
    out_div = out_div or (1,) * len(outs)
    rows = ins[0].shape[0] if ins[0].dim() else 0
    nbytes = sum(_nbytes(t) for t in ins)
    if nbytes <= window_bytes or rows <= multiple:
        return [(key, ins, outs)]
    if any(multiple % d for d in out_div):
        raise ValueError("host_items: multiple must be a multiple of every out_div")
    per_row = max(1, nbytes // rows)
    step = max(multiple, (window_bytes // per_row) // multiple * multiple)
    return [((key, r0), tuple(t[r0:r0 + step] for t in ins),
             tuple(o[r0 // d:-(-(r0 + step) // d)] for o, d in zip(outs, out_div)))
            for r0 in range(0, rows, step)]


def _windows(items: Sequence[tuple], window_bytes: int):
    """Consecutive groups of items whose inputs total at most ``window_bytes``
    (an item larger than that is a window of its own)."""
    cur, size = [], 0
    for it in items:
        n = sum(_nbytes(t) for t in it[1])
        if cur and size + n > window_bytes:
            yield cur
            cur, size = [], 0
        cur.append(it)
        size += n
    if cur:
        yield cur


def launch_chunks(items: Sequence, first: int = 8, most: int = 64):
    """Consecutive slices of ``items`` for the per-call drop-ins (quantize_state_dict,
    dequantize_state_dict, load_weights): 8, 16, 32, then ``most`` tensors per grouped
    launch.  Each slice is launched as soon as its plan is built, so the device starts on
    the first tensors while the host still plans the rest (the planning costs a few
    microseconds per tensor, the launch tens of them)."""
    i, n = 0, first
    while i < len(items):
        yield items[i:i + n]
        i += n
        n = min(2 * n, most)


def _nbytes(t: Tensor) -> int:
    return t.numel() * t.element_size()


class QuantPlan:
    """Grouped kernel launches that quantize a whole list of weights: one launch
    per run of consecutive tensors of at most ``GROUP_LAUNCH_BYTES`` (a tensor is
    never split; a Qwen3-8B layer or a MoE layer's expert stacks is one launch).

    The plan allocates every output once (or takes caller-provided output
    views, e.g. slices of a transfer bucket) and uploads a small descriptor
    table (tensor pointers and shapes plus a work-group -> tensor map).
    ``run()`` re-quantizes whatever the inputs currently hold -- the RL
    weight-sync pattern, where the same parameters are refreshed every step.

    The table records each input's storage address, so ``run()`` checks them:
    if an input now points at other storage (``param.data = new``, an FSDP
    re-gather into a fresh buffer) the table is re-packed and uploaded before
    the launch.  Callers whose sync produces brand-new tensors every step (a
    ``DTensor.full_tensor()`` or a ``.to(dtype)``) pass them as
    ``run(inputs=...)``; they must have the planned shapes and dtype.  The
    outputs stay the same tensors across re-binds.

    Inputs are device tensors: any element-aligned view and any row pitch (the
    kernels' 16-byte loads take 2-byte-aligned addresses).  All tensors of a plan
    must take one kernel: 128x128 tiles with K % 8 == 0 and 1xB blocks (B from
    8 to 65536) take the vector kernels, other shapes the generic one, and a
    plan mixing the two raises ``ValueError`` (quantize those tensors with
    :func:`fp8_block_quant` one by one).  float64 weights take
    ``fmt="fp8_block"`` with ``native_arith=True`` (float64 arithmetic and
    scales, as ``quantize_tensor`` on a float64 tensor).
    """

    def __init__(self, tensors: Sequence[Tensor], fmt: str = "fp8_block",
                 block_size: tuple[int, int] = (128, 128), *, use_pow2_scale: bool = False,
                 native_arith: bool = False, scale_dtype: torch.dtype = torch.float32,
                 outputs: Optional[Sequence[tuple[Tensor, Tensor]]] = None) -> None:
        if fmt not in ("fp8_block", "mxfp8", "mxfp4"):
            raise ValueError(f"fmt must be fp8_block, mxfp8 or mxfp4, got {fmt!r}")
        if not tensors:
            raise ValueError("QuantPlan needs at least one tensor")
        dt = tensors[0].dtype
        dev = tensors[0].device
        for t in tensors:
            _check_input(t, "QuantPlan", allow_f64=True)
            if t.dtype != dt or t.device != dev:
                raise ValueError("all tensors of a QuantPlan must share dtype and device")
        if dt == torch.float64 and not (fmt == "fp8_block" and native_arith):
            raise ValueError("QuantPlan: float64 weights are quantized to fp8_block in float64 "
                             "arithmetic (native_arith=True); cast them to float32 otherwise")
        if outputs is not None and len(outputs) != len(tensors):
            raise ValueError("outputs must pair up with tensors")
        self.fmt = fmt
        self.device = dev
        self.dtype = dt
        self.outputs: list[tuple[Tensor, Tensor]] = []
        br, bc = (int(block_size[0]), int(block_size[1])) if fmt == "fp8_block" else (1, 32)
        self._block = (br, bc)
        flags = 0
        native = native_arith and dt != torch.float32
        if fmt == "fp8_block":
            if use_pow2_scale:
                flags |= _lib.FLAG_POW2_SCALE
            if native:
                flags |= _lib.FLAG_NATIVE_ARITH
            elif scale_dtype == torch.bfloat16:
                flags |= _lib.FLAG_SCALE_BF16
        self._flags = flags
        self._owned = outputs is None
        self._shapes = [tuple(t.shape) for t in tensors]
        nbytes = 0
        for i, t in enumerate(tensors):
            shape = tuple(t.shape) if t.dim() >= 2 else (1,) + tuple(t.shape)
            *_, rows, cols = shape
            if fmt == "fp8_block":
                cshape, cdt = shape, torch.float8_e4m3fn
                sdt = dt if native else (torch.bfloat16 if flags & _lib.FLAG_SCALE_BF16 else torch.float32)
                sshape = shape[:-2] + (-(-rows // br), -(-cols // bc))
            else:
                if cols % 32:
                    raise ValueError(f"tensor {i}: last dim {cols} is not a multiple of 32")
                lead = shape[:-1]
                cshape = shape if fmt == "mxfp8" else lead + (cols // 2,)
                cdt = torch.float8_e4m3fn if fmt == "mxfp8" else torch.uint8
                sshape, sdt = lead + (cols // 32,), torch.uint8
            if outputs is None:
                codes = torch.empty(cshape, dtype=cdt, device=dev)
                scales = torch.empty(sshape, dtype=sdt, device=dev)
            else:
                codes, scales = outputs[i]
                if (codes.numel() * codes.element_size() != _prod(cshape)
                        or scales.numel() * scales.element_size() != _prod(sshape) * _esize(sdt)
                        or not codes.is_contiguous() or not scales.is_contiguous()
                        or codes.device != dev or scales.device != dev):
                    raise ValueError(f"output {i} must be contiguous device views of "
                                     f"{cshape} codes and {sshape} {sdt} scales")
            self.outputs.append((codes, scales))
            nbytes += _nbytes(t) + _nbytes(codes) + _nbytes(scales)
        self.algorithmic_bytes = nbytes
        self._bind(list(tensors))

    def _bind(self, tensors: list[Tensor]) -> None:
        """Pack and upload the descriptor table for the tensors' current storage.

        Refused once a run of this plan was captured into a HIP graph: the graph
        keeps the current table's address and the old inputs' pointers, so
        replacing (and freeing) the table would leave it reading freed memory."""
        launch = getattr(self, "_launch", None)
        if launch is not None and launch.captured:
            raise RuntimeError("QuantPlan: a run of this plan was captured into a HIP graph, which "
                               "keeps its descriptor table; its inputs now live in other storage, so "
                               "build (and capture) a new plan instead of re-binding this one")
        descs = (_lib.LrqTensor * len(tensors))()
        views = []
        for i, (t, (codes, scales)) in enumerate(zip(tensors, self.outputs)):
            xm, batch, rows, cols, ld, bstride = matrix_view(t)
            if xm.data_ptr() != t.data_ptr():
                raise ValueError(f"tensor {i} is not a strided matrix view; pass .contiguous()")
            views.append(xm)
            descs[i].in_ = xm.data_ptr()
            descs[i].codes = codes.data_ptr()
            descs[i].scales = scales.data_ptr()
            descs[i].batch, descs[i].rows, descs[i].cols = batch, rows, cols
            descs[i].ld, descs[i].batch_stride = ld, bstride
        sizes = [_nbytes(t) + _nbytes(c) + _nbytes(sc) for t, (c, sc) in zip(tensors, self.outputs)]
        launch = _GroupLaunches(self.fmt, descs, sizes, _IN_DTYPES.get(self.dtype, _lib.DTYPE_F64),
                                self._block, self._flags, self.device,
                                buffers=[list(pair) for pair in self.outputs] if self._owned else None)
        self._launch = launch
        self._views = views
        self.inputs = tensors
        self._sig = [(t.data_ptr(), t.stride(), tuple(t.shape)) for t in tensors]
        self.units = launch.units

    def run(self, inputs: Optional[Sequence[Tensor]] = None) -> list[tuple[Tensor, Tensor]]:
        """Enqueue the launch on the current stream; returns the (codes, scales) list.

        ``inputs``: the current tensors, when the sync produced new ones (same
        count, shapes, dtype and device as planned).  Without it, the planned
        tensors are re-read, re-bound first if any now points at other storage.
        """
        if inputs is not None:
            inputs = list(inputs)
            if len(inputs) != len(self._shapes):
                raise ValueError(f"QuantPlan.run: {len(inputs)} inputs for a plan of {len(self._shapes)}")
            for i, t in enumerate(inputs):
                _check_input(t, "QuantPlan.run", allow_f64=self.dtype == torch.float64)
                if t.dtype != self.dtype or t.device != self.device or tuple(t.shape) != self._shapes[i]:
                    raise ValueError(f"QuantPlan.run: input {i} is {t.dtype} {tuple(t.shape)} on "
                                     f"{t.device}; the plan has {self.dtype} {self._shapes[i]} on "
                                     f"{self.device} (build a new plan)")
            if self._moved(inputs):
                self._bind(inputs)
            else:
                self.inputs = inputs  # same storage: keep the caller's current objects alive
        elif self._moved(self.inputs):
            for i, t in enumerate(self.inputs):
                if tuple(t.shape) != self._shapes[i] or t.dtype != self.dtype:
                    raise ValueError(f"QuantPlan.run: input {i} changed to {t.dtype} {tuple(t.shape)}"
                                     f" (planned {self.dtype} {self._shapes[i]}); build a new plan")
            self._bind(self.inputs)
        self._launch.run()
        return self.outputs

    def _moved(self, tensors: Sequence[Tensor]) -> bool:
        """True if any tensor's storage address, strides or shape differ from the
        table's (a shape change then raises in ``run``)."""
        return any(t.data_ptr() != p or t.stride() != st or tuple(t.shape) != sh
                   for t, (p, st, sh) in zip(tensors, self._sig))


class DequantPlan:
    """Grouped kernel launches that dequantize a list of (codes, scales) pairs
    (split between tensors as in ``QuantPlan``).

    fp32(code) * fp32(scale) per ``block_size`` block, written as ``out_dtype``
    (float32: dequantize_tensor; bfloat16: dequantize_state_dict's cast).
    ``fmt="mxfp8"`` / ``"mxfp4"`` takes MX pairs instead (E8M0 scales per 1x32
    group; ``block_size`` is then ignored).
    """

    def __init__(self, pairs: Sequence[tuple[Tensor, Tensor]], block_size: tuple[int, int],
                 out_dtype: torch.dtype = torch.float32, *, fmt: str = "fp8_block") -> None:
        if not pairs:
            raise ValueError("DequantPlan needs at least one (codes, scales) pair")
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
        if fmt in ("mxfp8", "mxfp4"):
            self._init_mx(pairs, fmt, out_dtype)
            return
        if fmt != "fp8_block":
            raise ValueError(f"fmt must be fp8_block, mxfp8 or mxfp4, got {fmt!r}")
        sdt = pairs[0][1].dtype
        dev = pairs[0][0].device
        if sdt not in _IN_DTYPES:
            raise TypeError(f"DequantPlan: scales must be float32, bfloat16 or float16, got {sdt} "
                            "(cast float64 scales to float32, as dequantize_tensor does)")
        br, bc = int(block_size[0]), int(block_size[1])
        descs = (_lib.LrqTensor * len(pairs))()
        self.inputs = []
        self.outputs: list[Tensor] = []
        nbytes = 0
        for i, (c, sc) in enumerate(pairs):
            if c.dtype not in (torch.float8_e4m3fn, torch.uint8) or not c.is_cuda or not c.is_contiguous():
                raise ValueError(f"pair {i}: codes must be contiguous float8_e4m3fn device tensors")
            if sc.dtype != sdt or sc.device != dev or not sc.is_contiguous():
                raise ValueError(f"pair {i}: scales must be contiguous {sdt} on {dev}")
            shape = tuple(c.shape) if c.dim() >= 2 else (1,) + tuple(c.shape)
            *lead, rows, cols = shape
            batch = _prod(lead)
            need = batch * (-(-rows // br)) * (-(-cols // bc))
            if sc.numel() != need:
                raise ValueError(f"pair {i}: scales have {sc.numel()} elements, blocks need {need}")
            out = torch.empty(c.shape, dtype=out_dtype, device=dev)
            self.inputs.append((c, sc))
            self.outputs.append(out)
            descs[i].in_ = c.data_ptr()
            descs[i].codes = out.data_ptr()
            descs[i].scales = sc.data_ptr()
            descs[i].batch, descs[i].rows, descs[i].cols = batch, rows, cols
            descs[i].ld, descs[i].batch_stride = cols, rows * cols
            nbytes += _nbytes(c) + _nbytes(sc) + _nbytes(out)
        self.algorithmic_bytes = nbytes
        flags = _lib.FLAG_OUT_BF16 if out_dtype == torch.bfloat16 else 0
        sizes = [_nbytes(c) + _nbytes(sc) + _nbytes(o) for (c, sc), o in zip(self.inputs, self.outputs)]
        self._launch = _GroupLaunches("fp8_dequant", descs, sizes, _IN_DTYPES[sdt], (br, bc), flags, dev,
                                      buffers=[[o] for o in self.outputs])
        self.units = self._launch.units

    def _init_mx(self, pairs, fmt: str, out_dtype: torch.dtype) -> None:
        """(codes, E8M0 scales) pairs of ``fmt``: contiguous, on one device."""
        dev = pairs[0][0].device
        descs = (_lib.LrqTensor * len(pairs))()
        self.inputs, self.outputs = [], []
        nbytes = 0
        for i, (c, sc) in enumerate(pairs):
            if (c.dtype not in (torch.float8_e4m3fn, torch.uint8) or sc.dtype not in (torch.uint8, torch.float8_e8m0fnu)
                    or not c.is_cuda or c.device != dev or sc.device != dev
                    or not c.is_contiguous() or not sc.is_contiguous()):
                raise ValueError(f"pair {i}: contiguous {fmt} codes and uint8 E8M0 scales on {dev} required")
            *lead, kc = c.shape
            cols = kc if fmt == "mxfp8" else 2 * kc
            if cols % 32 or tuple(sc.shape) != (*lead, cols // 32):
                raise ValueError(f"pair {i}: codes {tuple(c.shape)} and scales {tuple(sc.shape)} are not a pair")
            out = torch.empty((*lead, cols), dtype=out_dtype, device=dev)
            self.inputs.append((c, sc))
            self.outputs.append(out)
            descs[i].in_ = c.data_ptr()
            descs[i].codes = out.data_ptr()
            descs[i].scales = sc.data_ptr()
            descs[i].batch, descs[i].rows, descs[i].cols = 1, _prod(lead), cols
            descs[i].ld, descs[i].batch_stride = cols, _prod(lead) * cols
            nbytes += _nbytes(c) + _nbytes(sc) + _nbytes(out)
        self.algorithmic_bytes = nbytes
        flags = _lib.FLAG_OUT_BF16 if out_dtype == torch.bfloat16 else 0
        sizes = [_nbytes(c) + _nbytes(sc) + _nbytes(o) for (c, sc), o in zip(self.inputs, self.outputs)]
        self._launch = _GroupLaunches(fmt + "_dequant", descs, sizes, _lib.DTYPE_BF16, (1, 32), flags, dev,
                                      buffers=[[o] for o in self.outputs])
        self.units = self._launch.units

    def run(self) -> list[Tensor]:
        self._launch.run()
        return self.outputs


class TensorScalePlan:
    """Per-tensor FP8 scales of a list of weights in two launches.

    ``scales[i] = max(|w_i|.max(), FLT_MIN) / 448`` (float32), the clamp before
    the division as in FP8KVCacheQuantizer.recalibrate_scales
    (lumenrl/quantization/fp8_kv_cache.py:52-54).  The plan owns a float32 [n]
    device tensor ``scales`` (or writes into ``out``) and a partial-maximum
    workspace; ``run()`` recomputes the scales from the tensors' current values.
    """

    def __init__(self, tensors: Sequence[Tensor], out: Optional[Tensor] = None) -> None:
        if not tensors:
            raise ValueError("TensorScalePlan needs at least one tensor")
        dt, dev = tensors[0].dtype, tensors[0].device
        for t in tensors:
            _check_input(t, "TensorScalePlan")
            if t.dtype != dt or t.device != dev:
                raise ValueError("all tensors of a TensorScalePlan must share dtype and device")
            if t.numel() == 0:
                raise RuntimeError("max(): a per-tensor scale of an empty tensor is undefined")
        n = len(tensors)
        owned = out is None
        if owned:
            out = torch.empty(n, dtype=torch.float32, device=dev)
        elif out.dtype != torch.float32 or out.shape != (n,) or not out.is_contiguous() or out.device != dev:
            raise ValueError(f"out must be a contiguous float32 [{n}] tensor on {dev}")
        self.device = dev
        self.inputs = list(tensors)
        self.scales = out
        descs = (_lib.LrqTensor * n)()
        self._views = []
        nbytes = 0
        for i, t in enumerate(tensors):
            xm, batch, rows, cols, ld, bstride = matrix_view(t)
            if xm.data_ptr() != t.data_ptr():
                raise ValueError(f"tensor {i} is not a strided matrix view; pass .contiguous()")
            self._views.append(xm)
            descs[i].in_ = xm.data_ptr()
            descs[i].codes = None
            descs[i].scales = out.data_ptr() + 4 * i
            descs[i].batch, descs[i].rows, descs[i].cols = batch, rows, cols
            descs[i].ld, descs[i].batch_stride = ld, bstride
            nbytes += _nbytes(t)
        self.algorithmic_bytes = nbytes + 4 * n
        self._launch = _GroupLaunch("tensor_scale", descs, n, _IN_DTYPES[dt], (1, 1), 0, dev)
        self.units = self._launch.units
        self.workspace = torch.empty(self._launch.workspace_bytes(), dtype=torch.uint8, device=dev)
        self._launch.buffers.append(self.workspace)
        if owned:
            self._launch.buffers.append(out)

    def run(self) -> Tensor:
        """Enqueue both launches on the current stream; returns ``scales``."""
        self._launch.run_tensor_scale(self.workspace)
        return self.scales

    def run_static(self) -> Tensor:
        """``run()`` through lrq_tensor_scale_grouped_static: the partial maxima
        go to the library's per-device static workspace, so the launch itself
        allocates nothing.  Calls that overlap on one device race on that
        workspace; calls ordered on one stream do not.  Tables needing more than
        ``_lib.STATIC_WORKSPACE_BYTES`` of workspace raise ValueError."""
        self._launch.run_tensor_scale_static()
        return self.scales


class CopyPlan:
    """One launch that copies many (dst, src) byte ranges on one device.

    ``pairs`` are contiguous tensors of equal byte size, 16-byte aligned (any
    dtype: the copy is bytewise).  Used for the pass-through tensors of a
    transfer bucket, which would otherwise take one copy launch each.
    """

    def __init__(self, pairs: Sequence[tuple[Tensor, Tensor]]) -> None:
        if not pairs:
            raise ValueError("CopyPlan needs at least one (dst, src) pair")
        dev = pairs[0][0].device
        descs = (_lib.LrqTensor * len(pairs))()
        self.pairs = list(pairs)
        nbytes = 0
        for i, (dst, src) in enumerate(pairs):
            n = _nbytes(src)
            if (not dst.is_cuda or not src.is_cuda or dst.device != dev or src.device != dev
                    or not dst.is_contiguous() or not src.is_contiguous() or _nbytes(dst) != n):
                raise ValueError(f"pair {i}: contiguous device tensors of equal size on {dev} required")
            descs[i].in_ = src.data_ptr()
            descs[i].codes = dst.data_ptr()
            descs[i].scales = None
            descs[i].batch, descs[i].rows, descs[i].cols = 1, 1, n
            descs[i].ld, descs[i].batch_stride = n, n
            nbytes += 2 * n
        self.algorithmic_bytes = nbytes
        self._launch = _GroupLaunch("copy", descs, len(pairs), _lib.DTYPE_BF16, (1, 1), 0, dev)
        self.units = self._launch.units

    def run(self) -> None:
        self._launch.run()


class CastPlan:
    """One launch that casts many tensors to float8_e4m3fn, unscaled.

    ``tensors`` are contiguous device tensors of one dtype (bf16, fp16 or
    float32); ``outputs`` are float8_e4m3fn tensors of the same shapes, made
    by the plan.  ``run()`` recasts whatever the inputs currently hold.
    """

    def __init__(self, tensors: Sequence[Tensor]) -> None:
        if not tensors:
            raise ValueError("CastPlan needs at least one tensor")
        dt, dev = tensors[0].dtype, tensors[0].device
        descs = (_lib.LrqTensor * len(tensors))()
        self.inputs = list(tensors)
        self.outputs: list[Tensor] = []
        nbytes = 0
        for i, t in enumerate(tensors):
            _check_input(t, "CastPlan")
            if t.dtype != dt or t.device != dev or not t.is_contiguous():
                raise ValueError(f"tensor {i}: CastPlan needs contiguous {dt} tensors on {dev}")
            out = torch.empty(t.shape, dtype=torch.float8_e4m3fn, device=dev)
            self.outputs.append(out)
            descs[i].in_ = t.data_ptr()
            descs[i].codes = out.data_ptr()
            descs[i].scales = None
            descs[i].batch, descs[i].rows, descs[i].cols = 1, 1, t.numel()
            descs[i].ld, descs[i].batch_stride = t.numel(), t.numel()
            nbytes += _nbytes(t) + _nbytes(out)
        self.algorithmic_bytes = nbytes
        self._launch = _GroupLaunch("cast_e4m3", descs, len(tensors), _IN_DTYPES[dt], (1, 1), 0, dev)
        self._launch.buffers += self.outputs
        self.units = self._launch.units

    def run(self) -> list[Tensor]:
        self._launch.run()
        return self.outputs


def _prod(shape) -> int:
    p = 1
    for d in shape:
        p *= int(d)
    return p


def _esize(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()
