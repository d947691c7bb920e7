"""Drop-in ``DynamicWeightLoader`` (lumenrl/engine/inference/weight_loader.py:13-78).

Same class, method, arguments, config keys and log texts.  With FP8 enabled the
reference casts every floating tensor of the state dict with
``tensor.to(torch.float8_e4m3fn)`` (unscaled, :19-43) one tensor at a time;
here the tensors of one dtype go through a few grouped liblrq launches (8, 16,
32, then 64 tensors each, issued as each is planned) whose bytes equal torch's
cast (round to nearest even; |x| rounding past 448, +-inf and NaN -> NaN
0x7F|sign).  CPU tensors go through the current HIP device in bounded
pipelined windows and come back on the CPU (pinned), as the reference returns
them; a process with no HIP device raises rather than casting on the CPU.

Opt-in extension (no reference counterpart): ``fp8_config["scaled"] = True``
replaces the unscaled cast by blockwise FP8 with float32 ``<name>_scale_inv``
scales -- the layout vLLM/ATOM FP8 loaders take -- for the tensors
``quantize_if`` accepts (default: 2-D/3-D linear weights with a 128-aligned
input dim, embeddings and lm_head excluded); every other tensor keeps its dtype.
``fp8_config["block_size"]`` sets the block (default [128, 128]).
"""

from __future__ import annotations

import logging
from typing import Any, Callable, Optional, Protocol

import torch

from lumenrl_amd.quantization import ops
from lumenrl_amd.quantization.bucket import default_quantize_if

logger = logging.getLogger(__name__)

_FP8_NAMES = ("float8_e4m3fn", "fp8", "fp8_e4m3")
_KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


class _SupportsWeightUpdate(Protocol):
    """Minimal protocol for engines that accept a PyTorch ``state_dict`` (:13-16)."""

    def update_weights(self, state_dict: dict[str, torch.Tensor]) -> None: ...


def _fp8_target(fp8_config: dict[str, Any] | None) -> Optional[bool]:
    """None: FP8 off; True: cast to e4m3fn; False: unsupported dtype name (:25-41)."""
    if fp8_config is None or not fp8_config.get("enabled", False):
        return None
    name = str(fp8_config.get("dtype", "float8_e4m3fn")).lower()
    return hasattr(torch, "float8_e4m3fn") and name in _FP8_NAMES


def _warn_kept(fp8_config: dict[str, Any]) -> None:
    """The reference's warning for a dtype name it does not cast to (:36-40)."""
    logger.warning(
        "FP8 dtype %s requested but this PyTorch build has no float8_e4m3fn; "
        "keeping original dtype.",
        str(fp8_config.get("dtype", "float8_e4m3fn")).lower(),
    )


def _kernel_input(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Contiguous device copy the cast kernel reads: other float dtypes are
    widened (float8 variants exactly) or narrowed (float64) to float32 first,
    which is the path torch's own cast takes through float."""
    x = t.to(device, non_blocking=False) if not t.is_cuda else t
    if x.dtype not in _KERNEL_DTYPES:
        x = x.to(torch.float32)
    return x.contiguous()


def _cast_all(tensors: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """e4m3fn casts of ``tensors``: device tensors in chunked grouped launches
    per (device, dtype); host tensors through bounded pipelined windows
    (``ops.run_host_windows``), returned as (pinned) CPU tensors."""

    def cast(xs: list[torch.Tensor]) -> list[torch.Tensor]:
        launches = ops.ChunkedLaunches(lambda ys: ops.CastPlan(ys).run())
        done: dict[int, torch.Tensor] = {}
        for i, t in enumerate(xs):
            x = _kernel_input(t, t.device)
            if x.numel():
                launches.add((x.device, x.dtype), i, x)
            else:
                done[i] = torch.empty(t.shape, dtype=torch.float8_e4m3fn, device=t.device)
        done.update(launches.flush())
        return [done[i] for i in range(len(xs))]

    out = dict(tensors)
    # tensor.to(its own dtype) is the tensor itself
    todo = {n: t for n, t in tensors.items() if t.dtype != torch.float8_e4m3fn}
    on_dev = [n for n, t in todo.items() if t.is_cuda]
    on_host = [n for n, t in todo.items() if not t.is_cuda]
    out.update(zip(on_dev, cast([todo[n] for n in on_dev])))
    if on_host:
        dev = ops.require_device()
        items = []
        for n in on_host:
            t = todo[n]
            q = torch.empty(t.shape, dtype=torch.float8_e4m3fn, pin_memory=True)
            out[n] = q
            items += ops.host_items(n, (t.reshape(-1),), (q.view(-1),))  # elementwise: any split
        ops.run_host_windows(items, lambda ins: [(q,) for q in cast([x for (x,) in ins])], dev)
    return out


def _scaled(tensors: dict[str, torch.Tensor], block: tuple[int, int],
            quantize_if: Callable[[str, torch.Tensor], bool]) -> dict[str, torch.Tensor]:
    """Blockwise FP8 + ``<name>_scale_inv`` for accepted tensors, the rest kept."""

    def quantize(xs: list[torch.Tensor]) -> list[tuple[torch.Tensor, torch.Tensor]]:
        launches = ops.ChunkedLaunches(lambda ys: ops.QuantPlan(ys, "fp8_block", block).run())
        done: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        for i, t in enumerate(xs):
            x = _kernel_input(t, t.device)
            if x.numel() and x.shape[-1] % 8 == 0:
                launches.add((x.device, x.dtype), i, x)
            elif x.numel():  # a width the grouped kernels do not take: a launch of its own
                done[i] = ops.fp8_block_quant(x, block)
            else:  # nothing to launch: empty codes and scales of the right shapes
                *lead, r, c = x.shape
                done[i] = (torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device),
                           torch.empty((*lead, -(-r // block[0]), -(-c // block[1])),
                                       dtype=torch.float32, device=x.device))
        done.update(launches.flush())
        return [done[i] for i in range(len(xs))]

    todo = [n for n, t in tensors.items() if quantize_if(n, t)]
    on_dev = [n for n in todo if tensors[n].is_cuda]
    on_host = [n for n in todo if not tensors[n].is_cuda]
    results = dict(zip(on_dev, quantize([tensors[n] for n in on_dev])))
    if on_host:
        dev = ops.require_device()
        items = []
        for n in on_host:
            t = tensors[n]
            *lead, r, c = t.shape
            outs = (torch.empty(t.shape, dtype=torch.float8_e4m3fn, pin_memory=True),
                    torch.empty((*lead, -(-r // block[0]), -(-c // block[1])), dtype=torch.float32,
                                pin_memory=True))
            results[n] = outs
            # 2-D: whole tile rows per chunk; 3-D: whole matrices (experts) per chunk
            tiles = t.dim() == 2
            items += ops.host_items(n, (t,), outs, multiple=block[0] if tiles else 1,
                                    out_div=(1, block[0]) if tiles else (1, 1))
        ops.run_host_windows(items, lambda ins: quantize([x for (x,) in ins]), dev)
    out: dict[str, torch.Tensor] = {}
    for name, t in tensors.items():
        if name not in results:
            out[name] = t
            continue
        codes, scales = results[name]
        out[name] = codes
        out[f"{name}_scale_inv"] = scales
    return out


def _maybe_fp8_quantize_tensor(tensor: torch.Tensor,
                               fp8_config: dict[str, Any] | None) -> torch.Tensor:
    """One tensor through the loader's FP8 rule (:19-43)."""
    target = _fp8_target(fp8_config)
    if target is None:
        return tensor
    if not target:
        _warn_kept(fp8_config)
        return tensor
    return _cast_all({"": tensor})[""]


class DynamicWeightLoader:
    """Loads PyTorch checkpoints into inference engines with optional FP8 paths (:46-78).

    Called by WeightSyncManager.transfer (lumenrl/engine/training/weight_sync.py:85-93,
    107-116) on the gathered state dict before it fans out.
    """

    @staticmethod
    def load_weights(
        engine: _SupportsWeightUpdate,
        state_dict: dict[str, torch.Tensor],
        fp8_config: dict[str, Any] | None = None,
        quantize_if: Callable[[str, torch.Tensor], bool] = default_quantize_if,
    ) -> None:
        """Load ``state_dict`` into ``engine`` with optional FP8 on-the-fly conversion.

        ``fp8_config``: ``enabled`` (bool) and ``dtype`` (str) as in the
        reference; ``scaled`` / ``block_size`` select the blockwise extension.
        """
        if fp8_config and fp8_config.get("enabled"):
            target = _fp8_target(fp8_config)
            floats = {n: t for n, t in state_dict.items() if t.dtype.is_floating_point}
            if target and fp8_config.get("scaled", False):
                block = tuple(int(b) for b in fp8_config.get("block_size", (128, 128)))
                state_dict = _scaled(state_dict, block, quantize_if)
            elif target:
                cast = _cast_all(floats)
                state_dict = {n: cast.get(n, t) for n, t in state_dict.items()}
            else:
                for _ in floats:  # once per floating tensor, as the reference warns
                    _warn_kept(fp8_config)
                state_dict = dict(state_dict)
            logger.info(
                "DynamicWeightLoader: applied FP8 conversion for %d tensors.", len(state_dict)
            )
        engine.update_weights(state_dict)
