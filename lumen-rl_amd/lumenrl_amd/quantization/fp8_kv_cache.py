"""Per-step FP8 KV-cache scale recalibration on MI355X kernels.

Behaviour of ``FP8KVCacheQuantizer`` (lumenrl/quantization/fp8_kv_cache.py:26-80):
each RL step, every ``nn.Linear`` whose last name component is ``q_proj``,
``k_proj`` or ``v_proj`` gets a float32 0-dim buffer
``_lumenrl_fp8_kv_scale_<q_proj|k_proj|v_proj>`` equal to
``max(|W|.max(), FLT_MIN) / 448``.  A buffer that exists is updated in place,
and a missing one is registered on the weight's device.

The reference runs one torch reduction per projection.  Here all projections
of a model share one ``TensorScalePlan``: two kernel launches for the whole
model, bit-identical to the torch ops on x86.  The plan is kept while the
weights' storage stays put (the optimizer updates parameters in place).
Buffers this class registers are views of the plan's scale vector, so a later
recalibration writes them with no per-module copy.
"""

from __future__ import annotations

import logging
from typing import Any, Optional

import torch
import torch.nn as nn
from torch import Tensor

from lumenrl_amd.quantization import ops
from lumenrl_amd.quantization.fp8_config import FP8Config

logger = logging.getLogger(__name__)

_KV_PROJECTIONS = frozenset({"q_proj", "k_proj", "v_proj"})
_BUFFER_PREFIX = "_lumenrl_fp8_kv_scale_"


def _atom_quant_spec() -> Any:
    """ATOM's quant_spec module if that engine is installed (it reads the buffers)."""
    try:
        from atom import quant_spec  # type: ignore[attr-defined]
    except ImportError:
        return None
    return quant_spec


class _ScaleGroup:
    """A TensorScalePlan over one dtype's projections, with staging for
    weights the kernels cannot read in place (host memory, float64)."""

    def __init__(self, sources: list[Tensor], device: torch.device) -> None:
        self.sources = sources
        self.staged: list[Optional[Tensor]] = []
        inputs = []
        for w in sources:
            if w.device == device and w.dtype != torch.float64:
                view, *_ = ops.matrix_view(w)
                if view.data_ptr() == w.data_ptr():
                    self.staged.append(None)
                    inputs.append(w)
                    continue
            buf = torch.empty(w.shape, dtype=_kernel_dtype(w), device=device)
            self.staged.append(buf)
            inputs.append(buf)
        self.plan = ops.TensorScalePlan(inputs)

    def run(self) -> Tensor:
        for src, buf in zip(self.sources, self.staged):
            if buf is not None:
                buf.copy_(src, non_blocking=True)  # float64 -> float32 rounds like w.to(float32)
        return self.plan.run()


def _kernel_dtype(w: Tensor) -> torch.dtype:
    return torch.float32 if w.dtype == torch.float64 else w.dtype


def _signature(ws: list[Tensor]) -> tuple:
    return tuple((w.device, w.dtype, tuple(w.shape), tuple(w.stride()), w.data_ptr()) for w in ws)


class FP8KVCacheQuantizer:
    """Maintains the per-step q/k/v projection FP8 scales the inference KV caches use."""

    def __init__(self, config: FP8Config) -> None:
        self._config = config
        self._enabled = False
        self._atom_spec = _atom_quant_spec()
        if self._atom_spec is None:
            logger.debug("atom.quant_spec not available; KV cache path uses torch heuristics only.")
        self._groups: dict[torch.dtype, _ScaleGroup] = {}
        self._signature: tuple = ()

    def _scales(self, weights: list[Tensor]) -> list[Tensor]:
        """0-dim float32 device scales, one per weight, in order."""
        sig = _signature(weights)
        if sig != self._signature:
            dev = next((w.device for w in weights if w.is_cuda), None) or ops.require_device()
            by_dtype: dict[torch.dtype, list[Tensor]] = {}
            for w in weights:
                by_dtype.setdefault(_kernel_dtype(w), []).append(w)
            self._groups = {dt: _ScaleGroup(ws, dev) for dt, ws in by_dtype.items()}
            self._signature = sig
        vecs = {dt: g.run() for dt, g in self._groups.items()}
        taken = {dt: 0 for dt in vecs}
        out = []
        for w in weights:
            dt = _kernel_dtype(w)
            out.append(vecs[dt][taken[dt]])
            taken[dt] += 1
        return out

    def recalibrate_scales(self, model: nn.Module) -> None:
        """Recompute every q/k/v projection's scale from its current weight."""
        if not self._config.is_fp8_enabled():
            logger.debug("FP8 disabled; skipping KV scale recalibration.")
            return
        targets = []
        for name, module in model.named_modules():
            short = name.rpartition(".")[2]
            if isinstance(module, nn.Linear) and short in _KV_PROJECTIONS:
                targets.append((short, module))
        if not targets:
            logger.warning("recalibrate_scales: no q_proj/k_proj/v_proj Linear layers found on model.")
            return
        scales = self._scales([m.weight.detach() for _, m in targets])
        for (short, module), s in zip(targets, scales):
            name = _BUFFER_PREFIX + short
            if hasattr(module, name):
                buf = getattr(module, name)
                if not (isinstance(buf, Tensor) and buf.device == s.device and buf.data_ptr() == s.data_ptr()):
                    buf.copy_(s.to(buf.device))
            else:
                home = module.weight.device
                module.register_buffer(name, s if home == s.device else s.to(home))
        logger.debug("recalibrate_scales: updated %d projection layers.", len(targets))

    def enable(self, model: nn.Module) -> None:
        """Flag the model for FP8 KV caches and create/refresh the scale buffers."""
        if not self._config.is_fp8_enabled():
            logger.info("FP8 disabled; FP8KVCacheQuantizer.enable is a no-op.")
            return
        setattr(model, "_lumenrl_fp8_kv_cache_enabled", True)
        self._enabled = True
        self.recalibrate_scales(model)
        if self._atom_spec is not None:
            logger.debug("atom.quant_spec present; ATOM engine may consume _lumenrl_fp8_kv_scale_* buffers.")

    @property
    def enabled(self) -> bool:
        return self._enabled
