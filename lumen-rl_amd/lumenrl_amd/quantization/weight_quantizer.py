"""Drop-in ``WeightQuantizer`` running on MI355X HIP kernels.

Mirrors lumenrl/quantization/weight_quantizer.py (same class, method names,
arguments, return layouts and ValueError texts); the arithmetic runs in
liblrq's kernels and is bit-identical to the reference evaluated by torch on an
x86 CPU:

* ``quantize_tensor`` on a float32 tensor computes in float32; on a bf16 or
  fp16 tensor it computes in that dtype, as the reference's torch ops do
  (:59-71).  NaN blocks in bf16 arithmetic give scale 0xFFFF and codes 0xFF
  (torch's vectorized x86 kernels; its scalar tail loop writes 0x7FC0/0x7F).
* ``quantize_state_dict`` upcasts to float32 (:109); for bf16/fp16 weights the
  upcast is exact, so the kernel reads them directly in float32 arithmetic and
  writes the bf16 ``_fp8_scales`` sidecar itself (:111).  The eligible weights
  go through a few grouped kernel launches (8, 16, 32, then 64 tensors each),
  each issued as soon as it is planned, so the device works while the host
  plans the rest.
* ``quantize_tensor`` on a float64 tensor computes in float64 (float64 scales)
  and rounds each quotient to float32 before the e4m3 cast, as :59-71 do.

Tensors on the CPU are staged through the current HIP device and the results
copied back, so the reference's CPU-tensor call sites keep working; there is no
CPU compute path.  The state-dict calls move host tensors in bounded,
pipelined windows (``ops.run_host_windows``), so device memory stays at a few
hundred MB whatever the size of the state.
"""

from __future__ import annotations

import logging
from typing import Any

import torch
from torch import Tensor

from lumenrl_amd.quantization import ops
from lumenrl_amd.quantization.fp8_config import FP8Config

logger = logging.getLogger(__name__)

_FP8_DTYPE = getattr(torch, "float8_e4m3fn", None)


def fp8_e4m3_max() -> float:
    """weight_quantizer.py:18-21."""
    if _FP8_DTYPE is not None:
        return float(torch.finfo(_FP8_DTYPE).max)
    return 448.0


def _check_unfold(last: int, block_size: int) -> None:
    """The errors ``flat.unfold(-1, block_size, block_size)`` raises on the
    reference's 2-D ``[leading, last]`` view (:58-59, :85-86): a negative block,
    a zero step, or a block wider than the row -- which includes every
    zero-width row (``[N, 0]``, ``(0,)``) that passes the divisibility check.
    Checked before any staging or device call."""
    if block_size < 0:
        raise RuntimeError(f"size is {block_size} but must be >= 0")
    if block_size == 0:
        raise RuntimeError("step is 0 but must be > 0")
    if block_size > last:
        raise RuntimeError(f"maximum size for tensor at dimension 1 is {last} but size is {block_size}")


def _stage(t: Tensor) -> tuple[Tensor, torch.device | None]:
    """Device copy of a CPU tensor (and the device to return results to)."""
    if t.is_cuda:
        return t, None
    dev = ops.require_device()
    return t.to(dev, non_blocking=False), t.device


class WeightQuantizer:
    """BF16 <-> FP8 (E4M3) blockwise transforms for ``state_dict`` tensors (:30-134)."""

    def __init__(self, config: FP8Config) -> None:
        self._config = config
        if _FP8_DTYPE is None:  # pragma: no cover - torch 2.10 has it
            raise RuntimeError("torch.float8_e4m3fn is required by lumenrl_amd")

    # -- single tensors ------------------------------------------------------
    def quantize_tensor(self, tensor: Tensor, block_size: int = 128) -> tuple[Tensor, Tensor]:
        """Blockwise FP8 quantization along the last dimension (:40-77).

        Returns ``(quantized, scales)``: ``quantized`` is float8_e4m3fn with the
        input shape, ``scales`` has shape ``tensor.shape[:-1] + (last // block_size,)``
        and the compute dtype, which is the input dtype (bf16, fp16, fp32 or fp64).
        """
        if tensor.dim() < 1:
            raise ValueError("quantize_tensor expects tensor.dim() >= 1")
        last = tensor.shape[-1]
        if last % block_size != 0:
            raise ValueError(f"Last dim {last} must be divisible by block_size={block_size}")
        _check_unfold(last, block_size)
        x, home = _stage(tensor)
        pow2 = self._config.use_weight_pow2_scale
        if x.dim() == 2:  # codes [N, K] and scales [N, K/B] as the kernel writes them
            q, s = ops.fp8_block_quant(x, (1, block_size), native_arith=True, pow2=pow2)
        else:
            leading = 1
            for d in tensor.shape[:-1]:
                leading *= int(d)
            q, s = ops.fp8_block_quant(x.reshape(leading, last), (1, block_size), native_arith=True,
                                       pow2=pow2)
            q = q.reshape(tensor.shape)
            s = s.reshape(tuple(tensor.shape[:-1]) + (last // block_size,))
        if home is not None:
            q, s = q.to(home), s.to(home)
        return q, s

    def dequantize_tensor(self, quantized: Tensor, scales: Tensor, block_size: int = 128) -> Tensor:
        """Inverse of :meth:`quantize_tensor` for a single tensor (:79-89): float32 out."""
        return self._dequant(quantized, scales, block_size, torch.float32)

    def _dequant(self, quantized: Tensor, scales: Tensor, block_size: int,
                 out_dtype: torch.dtype) -> Tensor:
        last = quantized.shape[-1]
        _check_unfold(last, block_size)
        q, home = _stage(quantized)
        s = scales.to(q.device)
        if s.dtype == torch.float64:
            s = s.to(torch.float32)
        leading = 1
        for d in quantized.shape[:-1]:
            leading *= int(d)
        qm = q.reshape(leading, last)
        sm = s.reshape(leading, last // block_size)
        out = ops.fp8_block_dequant(qm, sm, (1, block_size), out_dtype).reshape(quantized.shape)
        return out.to(home) if home is not None else out

    # -- state dicts ---------------------------------------------------------
    @staticmethod
    def _eligible(value: Any) -> bool:
        """Pass-through rules of quantize_state_dict (:95-108)."""
        if not isinstance(value, Tensor):
            return False
        if value.dtype not in (torch.bfloat16, torch.float16, torch.float32, torch.float64):
            return False
        if value.ndim != 2:
            return False
        if value.shape[1] % 128 != 0:
            logger.debug("Skipping tensor: in_features=%s not aligned to 128", value.shape[1])
            return False
        return True

    def quantize_state_dict(self, state_dict: dict[str, Tensor]) -> dict[str, Tensor | Any]:
        """Return a new dict with 2-D float weights converted to FP8 + sidecar scales (:91-115).

        Device weights go through chunked grouped launches; host weights go
        through bounded pipelined windows (``ops.run_host_windows``) and come
        back as (pinned) CPU tensors, as the reference returns them.
        """
        pow2 = self._config.use_weight_pow2_scale

        def quantize(xs: list[Tensor]) -> list[tuple[Tensor, Tensor]]:
            launches = ops.ChunkedLaunches(
                lambda ys: ops.QuantPlan(ys, "fp8_block", (1, 128), use_pow2_scale=pow2,
                                         scale_dtype=torch.bfloat16).run())
            done: dict[int, tuple[Tensor, Tensor]] = {}
            for i, x in enumerate(xs):
                if x.dtype == torch.float64:
                    x = x.to(torch.float32)  # the reference's own upcast (:109)
                x = x if x.is_contiguous() else x.contiguous()
                if x.numel() > 0:
                    launches.add((x.dtype, x.device), i, x)
                else:  # empty: no launch, codes and scales of the right shapes
                    done[i] = ops.fp8_block_quant(x, (1, 128), pow2=pow2, scale_dtype=torch.bfloat16)
            done.update(launches.flush())
            return [done[i] for i in range(len(xs))]

        keys = [k for k, v in state_dict.items() if self._eligible(v)]
        for k in keys:  # a [N, 0] weight reaches quantize_tensor's unfold (:105-109)
            _check_unfold(state_dict[k].shape[1], 128)
        on_dev = [k for k in keys if state_dict[k].is_cuda]
        on_host = [k for k in keys if not state_dict[k].is_cuda]
        results = dict(zip(on_dev, quantize([state_dict[k] for k in on_dev])))
        if on_host:
            dev = ops.require_device()
            items = []
            for k in on_host:
                v = state_dict[k]
                outs = (torch.empty(v.shape, dtype=torch.float8_e4m3fn, pin_memory=True),
                        torch.empty((v.shape[0], v.shape[1] // 128), dtype=torch.bfloat16,
                                    pin_memory=True))
                results[k] = outs
                items += ops.host_items(k, (v,), outs)
            ops.run_host_windows(items, lambda ins: quantize([x for (x,) in ins]), dev)

        out: dict[str, Tensor | Any] = {}
        for key, value in state_dict.items():
            if key not in results:
                out[key] = value
                continue
            q, s = results[key]
            out_features, in_features = value.shape
            out[key] = q
            out[f"{key}_fp8_scales"] = s.reshape(out_features, in_features // 128)
            out[f"{key}_fp8_meta"] = torch.tensor(
                [out_features, in_features], dtype=torch.int64, device="cpu"
            )
        return out

    def dequantize_state_dict(self, state_dict: dict[str, Tensor]) -> dict[str, Tensor | Any]:
        """Strip FP8 tensors back to BF16 weights using stored scales (:117-134).

        The (codes, scales) pairs go through grouped kernel launches (chunked as in
        quantize_state_dict) that write bf16 directly (fp32 product, then the bf16
        cast of :133); host pairs go through bounded pipelined windows.
        """
        consumed_suffixes = {"_fp8_scales", "_fp8_meta"}
        pairs: dict[str, tuple[Tensor, Tensor]] = {}
        for key, value in state_dict.items():
            if any(key.endswith(sfx) for sfx in consumed_suffixes) or not isinstance(value, Tensor):
                continue
            scale_key = f"{key}_fp8_scales"
            if scale_key in state_dict:
                if value.dim() > 0:  # dequantize_tensor's unfold (:132, :86)
                    _check_unfold(value.shape[-1], 128)
                pairs[key] = (value, state_dict[scale_key])

        def dequant(items: list[tuple[Tensor, Tensor]]) -> list[Tensor]:
            launches = ops.ChunkedLaunches(
                lambda ps: ops.DequantPlan(ps, (1, 128), torch.bfloat16).run())
            done: dict[int, Tensor] = {}
            for i, (q, s) in enumerate(items):
                s = s.to(q.device)
                if s.dtype == torch.float64:
                    s = s.to(torch.float32)
                last = q.shape[-1]
                leading = 1
                for d in q.shape[:-1]:
                    leading *= int(d)
                qm = q.contiguous().reshape(leading, last)
                sm = s.contiguous().reshape(leading, last // 128)
                if qm.numel() > 0:
                    launches.add((sm.dtype, qm.device), i, (qm, sm))
                else:
                    done[i] = ops.fp8_block_dequant(qm, sm, (1, 128), torch.bfloat16)
            done.update(launches.flush())
            return [done[i].reshape(q.shape) for i, (q, _) in enumerate(items)]

        on_dev = [k for k, (q, _) in pairs.items() if q.is_cuda]
        on_host = [k for k, (q, _) in pairs.items() if not q.is_cuda]
        results = dict(zip(on_dev, dequant([pairs[k] for k in on_dev])))
        if on_host:
            dev = ops.require_device()
            items = []
            for k in on_host:
                q, s = pairs[k]
                last = q.shape[-1]
                qm = q.reshape(-1, last)
                sm = s.cpu().reshape(qm.shape[0], last // 128)
                out = torch.empty(qm.shape, dtype=torch.bfloat16, pin_memory=True)
                results[k] = out.view(q.shape)
                items += ops.host_items(k, (qm, sm), (out,))
            ops.run_host_windows(items, lambda ins: [(d,) for d in dequant(ins)], dev)

        out: dict[str, Tensor | Any] = {}
        for key, value in state_dict.items():
            if any(key.endswith(sfx) for sfx in consumed_suffixes):
                continue
            out[key] = results.get(key, value)
        return out
