"""Quantize weights straight into a weight-transfer bucket.

Lumen-RL's sync copies bf16 weights into a flat uint8 device bucket, one tensor
after another, and ships the bucket with per-tensor metadata.  Two transports
carry it:
- `BucketedWeightSender` (ZMQ + IPC) uses `{name, shape, dtype, offset, handle}`
  (lumenrl/engine/inference/bucketed_weight_transfer.py:129-171);
- the RCCL bucket broadcast uses `{name, shape, dtype, offset, nbytes}` JSON
  entries (lumenrl/engine/inference/rdma_weight_transfer.py:22-57).

The rollout engine then re-quantizes the bf16 weights to FP8 itself
(vllm_fp8_utils.py:111-118).

`QuantizedBucketWriter` moves that quantization to the sender.  Each planned bucket is ONE
kernel launch per input dtype that reads the weights and writes e4m3 codes and
`<name>_scale_inv` scales directly at their offsets in the bucket (no
intermediate tensors, no copy).  Tensors that are not quantized (norms,
embeddings, lm_head, anything the predicate rejects) are copied in as-is, as
the reference sender does.  The bucket then carries about half (FP8) or a
quarter (MXFP4) of the bf16 bytes, and the receiver gets exactly what a
vLLM/ATOM FP8 loader takes.
"""

from __future__ import annotations

import json
from typing import Callable, Iterator, Optional, Sequence

import torch
from torch import Tensor

from lumenrl_amd.quantization import ops

_ALIGN = 256


def default_quantize_if(name: str, t: Tensor) -> bool:
    """2-D linear weights with a 128-aligned input dim; embeddings and lm_head stay bf16."""
    lname = name.lower()
    if "embed" in lname or "lm_head" in lname:
        return False
    return t.dim() in (2, 3) and t.shape[-1] % 128 == 0 and t.dtype in (
        torch.bfloat16, torch.float16, torch.float32)


class _Entry:
    __slots__ = ("name", "shape", "dtype", "offset", "nbytes", "src")

    def __init__(self, name, shape, dtype, offset, nbytes, src=None):
        self.name, self.shape, self.dtype = name, tuple(shape), dtype
        self.offset, self.nbytes, self.src = offset, nbytes, src


class Bucket:
    """One planned bucket: grouped quantize launches (one per input dtype: a
    bucket may hold bf16 weights next to an fp32 router gate; weights whose
    width 8 does not divide, which a custom ``quantize_if`` may admit, get a
    launch of their own kind) plus the
    pass-through copies, which (16-byte-aligned sources, the torch norm) go in
    one grouped copy launch.

    Sources are looked up in the writer's name -> tensor map at every
    ``fill()``: a weight re-bound by ``QuantizedBucketWriter.rebind`` or moved to
    other storage (``param.data = new``) is re-planned before its launch."""

    def __init__(self, buffer: Tensor, entries: list[_Entry],
                 quant: list[tuple[str, Tensor, Tensor]], copies: list[_Entry], src: dict,
                 fmt: str, block_size: tuple[int, int]) -> None:
        self.buffer = buffer
        self.entries = entries
        self.copies = copies
        self._src = src
        self.nbytes = max((e.offset + e.nbytes for e in entries), default=0)
        by_dtype: dict[tuple, list[tuple[str, Tensor, Tensor]]] = {}
        for name, codes, scales in quant:
            key = (src[name].dtype, src[name].shape[-1] % 8 == 0)  # one kernel per plan
            by_dtype.setdefault(key, []).append((name, codes, scales))
        self.plans: list[tuple[list[str], ops.QuantPlan]] = [
            ([n for n, _, _ in items],
             ops.QuantPlan([src[n] for n, _, _ in items], fmt, block_size,
                           outputs=[(c, sc) for _, c, sc in items]))
            for items in by_dtype.values()]
        self._plan_copies()

    def _plan_copies(self) -> None:
        old = getattr(self, "copy_plan", None)
        if old is not None and old._launch.captured:
            # a captured fill() keeps the copy table's address: it must not be freed
            raise RuntimeError("Bucket: a fill() of this bucket was captured into a HIP graph, which "
                               "keeps its copy table; a pass-through tensor now lives in other "
                               "storage, so build (and capture) a new writer instead")
        pairs, self._loose = [], []
        for e in self.copies:
            dst = self.buffer[e.offset:e.offset + e.nbytes]
            src = self._src[e.name].reshape(-1).view(torch.uint8)
            if e.nbytes and src.data_ptr() % 16 == 0 and dst.data_ptr() % 16 == 0:
                pairs.append((dst, src))
            elif e.nbytes:
                self._loose.append((dst, src))
        self._copy_ptrs = [self._src[e.name].data_ptr() for e in self.copies]
        self.copy_plan = ops.CopyPlan(pairs) if pairs else None

    @property
    def algorithmic_bytes(self) -> int:
        """Bytes one fill() reads and writes: quantized inputs, codes and scales,
        and twice each pass-through tensor."""
        q = sum(plan.algorithmic_bytes for _, plan in self.plans)
        return q + 2 * sum(e.nbytes for e in self.copies)

    def fill(self) -> "Bucket":
        """Enqueue the quantize launches and the pass-through copies (current stream)."""
        for names, plan in self.plans:
            plan.run([self._src[n] for n in names])
        if [self._src[e.name].data_ptr() for e in self.copies] != self._copy_ptrs:
            self._plan_copies()
        if self.copy_plan is not None:
            self.copy_plan.run()
        for dst, src in self._loose:
            dst.copy_(src, non_blocking=True)
        return self

    def bucket_meta(self) -> dict:
        """BucketedWeightSender metadata (bucketed_weight_transfer.py:155-161)."""
        return {e.name: {"name": e.name, "shape": torch.Size(e.shape), "dtype": e.dtype,
                         "offset": e.offset, "handle": None} for e in self.entries}

    def rdma_entries(self) -> list[dict]:
        """RCCL bucket entries (rdma_weight_transfer.py:36-44)."""
        return [{"name": e.name, "shape": list(e.shape), "dtype": str(e.dtype).removeprefix("torch."),
                 "offset": e.offset, "nbytes": e.nbytes} for e in self.entries]

    def views(self) -> list[tuple[str, Tensor]]:
        """What a receiver rebuilds from the metadata: (name, tensor) views of the buffer."""
        out = []
        for e in self.entries:
            n = 1
            for d in e.shape:
                n *= int(d)
            t = self.buffer[e.offset:e.offset + e.nbytes].view(e.dtype)[:n].view(e.shape)
            out.append((e.name, t))
        return out


class BucketLayout:
    """Where every entry of one bucket goes: (name, shape, dtype, offset, nbytes)
    per entry, codes and ``<name><scale_suffix>`` scales for quantized weights."""

    def __init__(self) -> None:
        self.items: list[tuple[str, bool]] = []       # (weight name, quantized)
        self.entries: list[_Entry] = []
        self.nbytes = 0


def entry_sizes(shape: tuple, dtype: torch.dtype, quantized: bool, fmt: str,
                block_size: tuple[int, int]) -> list[tuple[tuple, torch.dtype, int]]:
    """(shape, dtype, bytes) of the entries one weight occupies in a bucket."""
    if not quantized:
        return [(tuple(shape), dtype, _prod(shape) * torch.empty((), dtype=dtype).element_size())]
    shape = tuple(shape)
    *lead, rows, cols = shape if len(shape) >= 2 else (1,) + shape
    lead = tuple(lead)
    if fmt == "fp8_block":
        br, bc = block_size
        sshape = lead + (-(-rows // br), -(-cols // bc))
        return [(shape, torch.float8_e4m3fn, _prod(shape)), (sshape, torch.float32, 4 * _prod(sshape))]
    cshape = shape if fmt == "mxfp8" else lead + (rows, cols // 2)
    ctype = torch.float8_e4m3fn if fmt == "mxfp8" else torch.uint8
    sshape = lead + (rows, cols // 32)
    return [(cshape, ctype, _prod(cshape)), (sshape, torch.uint8, _prod(sshape))]


def plan_layout(weights: Sequence[tuple[str, tuple, torch.dtype, bool]], bucket_bytes: int,
                fmt: str = "fp8_block", block_size: tuple[int, int] = (128, 128),
                scale_suffix: str = "_scale_inv") -> list[BucketLayout]:
    """Split (name, shape, dtype, quantized) weights, in order, into buckets of at
    most ``bucket_bytes``; every entry starts on a 256-byte boundary.  Pure host
    arithmetic (no device), shared by :class:`QuantizedBucketWriter`."""
    layouts: list[BucketLayout] = []
    cur = BucketLayout()
    for name, shape, dtype, q in weights:
        sizes = entry_sizes(shape, dtype, q, fmt, block_size)
        need = sum(_align(n) for _, _, n in sizes)
        if need > bucket_bytes:
            raise ValueError(f"{name} needs {need} bytes, more than the bucket ({bucket_bytes})")
        if cur.items and cur.nbytes + need > bucket_bytes:
            layouts.append(cur)
            cur = BucketLayout()
        names = [name] if not q else [name, name + scale_suffix]
        for nm, (eshape, edt, n) in zip(names, sizes):
            cur.entries.append(_Entry(nm, eshape, edt, cur.nbytes, n))
            cur.nbytes += _align(n)
        cur.items.append((name, q))
    if cur.items:
        layouts.append(cur)
    return layouts


class QuantizedBucketWriter:
    """Plans buckets over a fixed list of named weights and fills them on demand.

    Plan once, then per sync:
    ``for bucket in writer: bucket.fill(); send(bucket.buffer, bucket.bucket_meta())``.
    A sync whose weights are new tensors (a ``DTensor.full_tensor()`` or a
    dtype cast every step) first calls ``writer.rebind(named_weights)`` with
    them; weights whose storage merely moved are picked up by ``fill()``.
    All buckets share one device buffer of ``bucket_bytes``; the caller must not
    refill it before the receiver has consumed the previous bucket (the
    reference's REQ/REP handshake guarantees that).
    """

    def __init__(self, named_weights: Sequence[tuple[str, Tensor]], bucket_bytes: int,
                 fmt: str = "fp8_block", block_size: tuple[int, int] = (128, 128),
                 quantize_if: Callable[[str, Tensor], bool] = default_quantize_if,
                 scale_suffix: str = "_scale_inv", buffer: Optional[Tensor] = None) -> None:
        if fmt not in ("fp8_block", "mxfp8", "mxfp4"):
            raise ValueError(f"fmt must be fp8_block, mxfp8 or mxfp4, got {fmt!r}")
        if not named_weights:
            raise ValueError("no weights to plan")
        dev = named_weights[0][1].device
        if buffer is None:
            buffer = torch.empty(int(bucket_bytes), dtype=torch.uint8, device=dev)
        if buffer.dtype != torch.uint8 or buffer.dim() != 1 or buffer.numel() < bucket_bytes:
            raise ValueError("buffer must be a flat uint8 tensor of at least bucket_bytes")
        self.buffer = buffer
        self.bucket_bytes = int(bucket_bytes)
        self.scale_suffix = scale_suffix
        self.fmt = fmt
        self.block_size = block_size
        for name, w in named_weights:
            if not w.is_contiguous():
                raise ValueError(f"{name}: bucket planning needs contiguous weights "
                                 "(the plan keeps pointers to their storage)")
        self._src = dict(named_weights)   # name -> current tensor, shared with the buckets
        self._planned = {n: (tuple(w.shape), w.dtype, w.device) for n, w in named_weights}
        layouts = plan_layout([(n, tuple(w.shape), w.dtype, bool(quantize_if(n, w)))
                               for n, w in named_weights],
                              self.bucket_bytes, fmt, block_size, scale_suffix)
        self.buckets = [self._bucket(lay) for lay in layouts]

    def _bucket(self, lay: BucketLayout) -> Bucket:
        by_name = {e.name: e for e in lay.entries}
        copies, quant = [], []
        for name, q in lay.items:
            if not q:
                e = by_name[name]
                e.src = self._src[name]
                copies.append(e)
                continue
            ce, se = by_name[name], by_name[name + self.scale_suffix]
            codes = self.buffer[ce.offset:ce.offset + ce.nbytes].view(ce.dtype).view(ce.shape)
            scales = self.buffer[se.offset:se.offset + se.nbytes].view(se.dtype).view(se.shape)
            quant.append((name, codes, scales))
        return Bucket(self.buffer, lay.entries, quant, copies, self._src, self.fmt, self.block_size)

    def rebind(self, named_weights: Sequence[tuple[str, Tensor]]) -> None:
        """Point the planned weights at this sync's tensors (same names, shapes,
        dtypes, device; contiguous).  Weights left out keep their tensors."""
        new = {}
        for name, w in named_weights:
            if name not in self._planned:
                raise KeyError(f"{name} was not planned")
            shape, dtype, dev = self._planned[name]
            if tuple(w.shape) != shape or w.dtype != dtype or w.device != dev or not w.is_contiguous():
                raise ValueError(f"{name}: got {w.dtype} {tuple(w.shape)} on {w.device}, planned "
                                 f"contiguous {dtype} {shape} on {dev}")
            new[name] = w
        self._src.update(new)
        for b in self.buckets:
            for e in b.copies:
                e.src = self._src[e.name]

    def __iter__(self) -> Iterator[Bucket]:
        return iter(self.buckets)

    def __len__(self) -> int:
        return len(self.buckets)


def encode_bucket(weights: Sequence[tuple[str, Tensor]], *, fmt: str = "fp8_block",
                  block_size: tuple[int, int] = (128, 128),
                  quantize_if: Callable[[str, Tensor], bool] = default_quantize_if,
                  scale_suffix: str = "_scale_inv") -> tuple[Tensor, Tensor]:
    """The RCCL sender's ``_encode_bucket`` (rdma_weight_transfer.py:22-57) with the
    quantization fused into the payload fill.

    Returns ``(metadata, payload)`` as the reference does: ``metadata`` is the
    compact JSON of the entries ``{name, shape, dtype, offset, nbytes}`` as a
    uint8 device tensor, ``payload`` the uint8 device bytes the entries point
    into.  Weights ``quantize_if`` accepts arrive as codes plus
    ``<name><scale_suffix>`` scales, written by one grouped launch per dtype;
    the rest are copied unchanged.  Entries start on 256-byte boundaries (the
    receiver reads offsets from the metadata, rdma_weight_transfer.py:176-180).
    CPU tensors are moved to the current HIP device first, as the reference
    does.  For a sync that repeats over the same weights, plan once with
    ``QuantizedBucketWriter`` instead (this builds the plan on every call).
    """
    if not weights:
        raise ValueError("cannot encode an empty weight bucket")
    prepared = []
    for name, tensor in weights:
        value = tensor.detach()
        if not value.is_cuda:
            value = value.to(ops.require_device(), non_blocking=True)
        prepared.append((name, value.contiguous()))
    layouts = plan_layout([(n, tuple(v.shape), v.dtype, bool(quantize_if(n, v))) for n, v in prepared],
                          1 << 62, fmt, block_size, scale_suffix)
    writer = QuantizedBucketWriter(prepared, bucket_bytes=max(layouts[0].nbytes, 1), fmt=fmt,
                                   block_size=block_size, quantize_if=quantize_if,
                                   scale_suffix=scale_suffix)
    bucket = writer.buckets[0].fill()
    raw = json.dumps(bucket.rdma_entries(), separators=(",", ":")).encode("utf-8")
    device = bucket.buffer.device
    metadata = torch.tensor(list(raw), dtype=torch.uint8, device=device)
    return metadata, bucket.buffer[:bucket.nbytes]


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def _prod(shape) -> int:
    p = 1
    for d in shape:
        p *= int(d)
    return p
