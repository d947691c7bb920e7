#!/usr/bin/env python3
"""Quantize-kernel benchmark on one MI355X (BASELINE.json metric).

A step is one weight-sync quantization pass over one synthetic weight set
already resident in HBM:

  c2 (default, the metric's config): the full Qwen3-8B linear set, 36 layers x
     {q,k,v,o,gate,up,down}, bf16 N(0, 0.02^2) with 0.1% +-U(0.5, 4) outliers,
     -> FP8 E4M3 with one fp32 scale per 128x128 tile: one grouped plan, run as
     7 launches of consecutive tensors (~3 GiB of bytes each).
  c1: one [4096, 4096] weight, 128x128 (L2/MALL flushed between launches).
  c3: Qwen3-30B-A3B experts, 48 layers x 128 experts (gate_up [E,1536,2048],
      down [E,2048,768]) with one zero and one inf tile per layer; one launch
      per layer (48 per step).
  c4: c2 shapes, Student-t(4) x 0.02/sqrt(2), MXFP8.
  c5: c2 shapes, N(0, 0.02^2) x per-row log-uniform[0.25, 4], MXFP4.
  c2r: c2 weights with the reference's own 1x128 blocks (scales [N, K/128]).
  c2pc: c2 weights with per-channel scales (1xK blocks: quantize_tensor with
       block_size = in_features), one grouped launch per row width.
  c2d: dequantize_state_dict of the c2r result: e4m3 codes + bf16 1x128 scales ->
       bf16 weights, one grouped plan.
  c2sd: the drop-in WeightQuantizer.quantize_state_dict on the c2 weights held
       in a device state dict (1x128 blocks, bf16 `_fp8_scales` sidecar, new
       outputs every call): the API path end to end, host work included.
  bucket: one trainer-side weight sync of the whole Qwen3-8B state into 2 GiB
       transfer buckets (QuantizedBucketWriter): the c2 linears quantized to
       128x128 FP8 straight into the buckets, and embed_tokens, lm_head and
       every norm (input/post-attention, q_norm/k_norm, final) copied through.
  kv:  FP8KVCacheQuantizer scale recalibration: max(|W|.max(), FLT_MIN)/448 over
       the 108 q/k/v_proj weights of Qwen3-8B (c2's values), one grouped
       amax launch + one per-tensor finishing launch.
  c2host / casthost: quantize_state_dict on the c2 weights / DynamicWeightLoader
       on the whole Qwen3-8B state, both held in HOST memory: PCIe-inclusive
       rates (the inputs are not resident in HBM), reported apart from the metric.
  rollout: FP8RolloutQuantizer.quantize_model on a 36-layer Qwen3-8B-shaped
       module of nn.Linear layers on the device (quantize, swap, restore).
  act: the W8A8 rollout linear's activation fake-quant (fp8_rollout.py:53-72)
       on the seven linear inputs of one Qwen3-8B layer for an 8192-token
       prefill chunk (bf16 in, float32 out), one launch per linear, every input
       its own buffer.

Prints ONE JSON line on stdout.  value = algorithmic bytes (bf16 in + codes +
scales) per step / step time, in GB/s (1e9 B/s).  With --config c2 (the
default) the line also carries `also`: c3, c4 and c5 timed on the device the
same way after c2's set is freed (ms_per_step, step GB/s, kernel GB/s and its
fraction of 8 TB/s; no CPU leg; --no-also skips them).  The roofline object uses the
same bytes over the step's kernel time (HIP events on the launch stream around
each span of back-to-back launches: a plan run, or a whole step of several plan
runs): `launch_ms` is the mean launch (a span's event time over its launches),
as rocprofv3 averages a kernel; `span_ms` the span itself; `traffic` the
profiled HBM bytes per launch beside `algorithmic_bytes_per_launch`.  cpu_baseline times the reference's op sequence in torch on the host
CPU (oracle/torch_ref.py) over a bounded sample of the same weights.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "lumen-rl_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
QWEN3_8B = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096),
            ("o_proj", 4096, 4096), ("gate_proj", 12288, 4096), ("up_proj", 12288, 4096),
            ("down_proj", 4096, 12288)]


PROFILE_FOR = {"c1": "k_tile128_single_4096x4096_c1", "c2": "k_tile128_qwen3_8b_fp8_128x128", "c2r": "k_row_qwen3_8b_fp8_1x128",
               "c3": "k_tile128_qwen3_30b_a3b_experts", "c4": "k_mx_qwen3_8b_mxfp8",
               "c5": "k_mx_qwen3_8b_mxfp4", "c2d": "k_dequant_qwen3_8b_fp8_1x128_to_bf16",
               "act": "k_act_qdq_qwen3_8b_prefill_8192", "kv": "k_amax_qwen3_8b_qkv_scales",
               "cast": "k_cast_e4m3_qwen3_8b_state_dynamic_weight_loader",
               "c4d": "k_mx_dequant_qwen3_8b_mxfp8_to_bf16", "c2sd": "k_row_qwen3_8b_state_dict_dropin",
               "rollout": "k_row_qwen3_8b_rollout_quantize_model", "c2pc": "k_row_wide_qwen3_8b_per_channel",
               "f64": "k_row_f64_qwen3_8b_4_layers_quantize_tensor",
               "bucket": "k_tile128_k_copy_qwen3_8b_state_bucket_sync"}
KERNEL_FOR = {"c1": "k_tile128", "c2": "k_tile128", "c3": "k_tile128", "c4": "k_mx", "c5": "k_mx",
              "c2r": "k_row", "c2d": "k_dequant", "act": "k_act_qdq8", "kv": "k_amax", "c2sd": "k_row", "bucket": "k_tile128",
              "cast": "k_cast_e4m3", "c4d": "k_mx_dequant", "rollout": "k_row", "f64": "k_row_f64",
              "c2pc": "k_row_wide"}
PREFILL_TOKENS = 8192


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def metric_name() -> str:
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


# ---------------------------------------------------------------------------
# synthetic weights (generated on the device from a seed; per-layer seed = base + layer)
# ---------------------------------------------------------------------------
def gen_weight(torch, rows, cols, gen, dev, kind="normal"):
    w = torch.empty(rows, cols, dtype=torch.float32, device=dev)
    if kind == "student_t":
        # t(4) = N / sqrt(chi2_4 / 4); std of t(4) is sqrt(2)
        n = torch.randn(rows, cols, generator=gen, device=dev)
        chi = torch.randn(4, rows, cols, generator=gen, device=dev).square_().sum(0).div_(4.0)
        w = n.div_(chi.sqrt_()).mul_(0.02 / math.sqrt(2.0))
        del chi
    else:
        w.normal_(0.0, 0.02, generator=gen)
        if kind == "rowscale":
            u = torch.rand(rows, 1, generator=gen, device=dev)
            w.mul_(torch.exp(math.log(0.25) + u * (math.log(4.0) - math.log(0.25))))
        else:
            k = max(1, w.numel() // 1000)
            idx = torch.randint(0, w.numel(), (k,), generator=gen, device=dev)
            sign = torch.randint(0, 2, (k,), generator=gen, device=dev).float().mul_(2).sub_(1)
            mag = torch.rand(k, generator=gen, device=dev).mul_(3.5).add_(0.5)
            w.view(-1)[idx] = sign * mag
    return w.to(torch.bfloat16)


def qwen3_8b_set(torch, dev, seed, kind="normal", layers=36):
    ws, names = [], []
    for layer in range(layers):
        gen = torch.Generator(device=dev).manual_seed(seed + layer)
        for name, r, c in QWEN3_8B:
            ws.append(gen_weight(torch, r, c, gen, dev, kind))
            names.append(f"layers.{layer}.{name}")
    return ws, names


def qwen3_8b_state(torch, dev, seed):
    """The whole Qwen3-8B state in HF key order: embed_tokens, per layer the two
    RMSNorms, q_norm/k_norm and the seven linears (c2's values), final norm, lm_head."""
    ws, names = qwen3_8b_set(torch, dev, seed, "normal")
    g = torch.Generator(device=dev).manual_seed(seed - 1)

    def emb():
        return (torch.randn(151936, 4096, generator=g, device=dev) * 0.02).to(torch.bfloat16)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=dev)).to(torch.bfloat16)

    named = [("model.embed_tokens.weight", emb())]
    lin = iter(zip(names, ws))
    for layer in range(36):
        pre = f"model.layers.{layer}"
        named += [(f"{pre}.input_layernorm.weight", norm(4096)),
                  (f"{pre}.post_attention_layernorm.weight", norm(4096)),
                  (f"{pre}.self_attn.q_norm.weight", norm(128)),
                  (f"{pre}.self_attn.k_norm.weight", norm(128))]
        for _ in range(7):
            n, w = next(lin)
            kind = "self_attn" if n.split(".")[-1] in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
            named.append((f"{pre}.{kind}.{n.split('.')[-1]}.weight", w))
    named += [("model.norm.weight", norm(4096)), ("lm_head.weight", emb())]
    return named


def moe_layer(torch, dev, seed, layer, experts=128):
    gen = torch.Generator(device=dev).manual_seed(seed + layer)
    gu = torch.empty(experts, 1536, 2048, dtype=torch.float32, device=dev).normal_(0.0, 0.02, generator=gen)
    dn = torch.empty(experts, 2048, 768, dtype=torch.float32, device=dev).normal_(0.0, 0.02, generator=gen)
    e = int(torch.randint(0, experts, (1,), generator=gen, device=dev))
    gu[e, 128:256, 256:384] = 0.0                      # one all-zero tile
    e2 = int(torch.randint(0, experts, (1,), generator=gen, device=dev))
    dn[e2, 512 + 3, 128 + 5] = float("inf")            # one tile holding an inf
    return gu.to(torch.bfloat16), dn.to(torch.bfloat16)


# ---------------------------------------------------------------------------
# CPU baseline: the reference's op sequence in torch on the host (bounded sample)
# ---------------------------------------------------------------------------
def cpu_baseline(torch, ws, fmt, fmt_block, seconds, full_bytes=None):
    """The CPU path on the host: one warm-up pass, then the median of 3 passes
    over the same bounded sample.

    The sample is the first tensors of the workload, as many as fit in about
    ``seconds / 4`` of 16-thread work (so the four passes take about ``seconds``);
    the 1-thread leg does the same on a sample sized for 1 thread.  GB/s counts
    algorithmic bytes, so a rate extrapolates linearly to the whole workload;
    the extrapolated whole-set time is reported with it.

    FP8 blockwise: the reference's torch op sequence (oracle/torch_ref.py).
    MX formats have no reference CPU path: the C oracle's MX restatement.
    """
    import numpy as np

    from oracle import oracle as O
    from oracle import torch_ref

    threads = max(1, min(os.cpu_count() or 1, 16))
    prev = torch.get_num_threads()
    legs = {}
    try:
        for nt, budget in ((threads, seconds / 4), (1, seconds / 8)):
            torch.set_num_threads(nt)
            sample = _cpu_sample(torch, O, torch_ref, np, ws, fmt, fmt_block, budget, nt)
            _cpu_pass(torch, O, torch_ref, np, sample, fmt, fmt_block, nt)  # warm-up
            times, nbytes = [], 0
            for _ in range(3):
                nbytes, t = _cpu_pass(torch, O, torch_ref, np, sample, fmt, fmt_block, nt)
                times.append(t)
            legs[nt] = (len(sample), nbytes, sorted(times)[1])
    finally:
        torch.set_num_threads(prev)
    f64 = not isinstance(ws[0], (tuple, list)) and ws[0].dtype == torch.float64
    what = {
        "fp8_block": (f"oracle/torch_ref.py (weight_quantizer.py op order on "
                      + (f"{fmt_block[0]}x{fmt_block[1]} blocks, " if fmt_block[1] else "1xK (whole-row) blocks, ")
                      + ("float64 arithmetic, no upcast)" if f64 else "fp32 upcast first)")),
        "fp8_dequant": "oracle/torch_ref.py (weight_quantizer.py:79-89 then the bf16 cast of :133)",
        "act": "oracle/torch_ref.py (fp8_rollout.py:53-72 op order)",
        "kv": "oracle/torch_ref.py (fp8_kv_cache.py:52-54 op order, one tensor at a time)",
        "cast": "torch's own tensor.to(float8_e4m3fn) per tensor, as weight_loader.py:19-43 runs it",
        "mx_dequant": "oracle/torch_ref.py mx_dequant (torch decode, E8M0 widen, product, bf16 cast)",
    }.get(fmt, f"the C oracle's {fmt} restatement (the reference has no MX CPU path)")
    n, nb, t = legs[threads]
    n1, nb1, t1 = legs[1]
    rate, rate1 = nb / t / 1e9, nb1 / t1 / 1e9
    whole = "" if not full_bytes else (
        f"; extrapolated to the whole workload ({full_bytes / 1e9:.2f} GB): "
        f"{full_bytes / 1e9 / rate:.1f} s at {threads} threads, {full_bytes / 1e9 / rate1:.1f} s at 1 thread")
    return {
        "value": round(rate, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {n} tensors of the same weight set ({nb / 1e9:.2f} GB algorithmic) through "
                   f"{what}; {threads} threads on {os.cpu_count()} visible cores; 1 warm-up pass, then the "
                   f"median of 3 passes ({t:.2f} s){whole}"),
        "value_1thread": round(rate1, 3),
        "sample_1thread": (f"first {n1} tensors ({nb1 / 1e9:.2f} GB), 1 thread, 1 warm-up + median of 3 "
                           f"({t1:.2f} s); GB/s extrapolates linearly to the whole set"),
        "cpu_model": _cpu_model(),
    }


def _cpu_sample(torch, O, torch_ref, np, ws, fmt, fmt_block, budget, threads):
    """The first tensors of ``ws`` whose CPU pass takes about ``budget`` seconds,
    judged from a pass over the first tensor (at least one tensor)."""
    _, t0 = _cpu_pass(torch, O, torch_ref, np, ws[:1], fmt, fmt_block, threads)
    b0 = _item_bytes(ws[0])
    total, out = 0, []
    for w in ws:
        if out and total * t0 / b0 >= budget:
            break
        out.append(w)
        total += _item_bytes(w)
    return out


def _item_bytes(w) -> int:
    if isinstance(w, (tuple, list)):
        return sum(t.numel() * t.element_size() for t in w)
    return w.numel() * w.element_size()


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_pass(torch, O, torch_ref, np, ws, fmt, fmt_block, threads):
    """One pass over whole tensors through the CPU path: (algorithmic bytes, seconds)."""
    done_bytes = 0
    t_total = 0.0
    for w in ws:
        if fmt == "mx_dequant":
            c, sc = w[0].cpu(), w[1].cpu()
            t0 = time.perf_counter()
            out = torch_ref.mx_dequant(c, sc, 8, torch.bfloat16)
            t_total += time.perf_counter() - t0
            done_bytes += c.numel() + sc.numel() + out.numel() * 2
            continue
        if fmt == "fp8_dequant":
            c, sc = w[0].cpu(), w[1].cpu()
            t0 = time.perf_counter()
            out = torch_ref.dequantize_tensor(c, sc, fmt_block[1]).to(torch.bfloat16)
            t_total += time.perf_counter() - t0
            done_bytes += c.numel() + sc.numel() * 2 + out.numel() * 2
            continue
        x = w.cpu()
        if fmt == "kv":
            t0 = time.perf_counter()
            torch_ref.kv_scale(x)
            t_total += time.perf_counter() - t0
            done_bytes += x.numel() * 2 + 4
        elif fmt == "cast":
            t0 = time.perf_counter()
            q = x.to(torch.float8_e4m3fn)  # weight_loader.py:33, the reference's own op
            t_total += time.perf_counter() - t0
            done_bytes += x.numel() * x.element_size() + q.numel()
        elif fmt == "act":
            t0 = time.perf_counter()
            out = torch_ref.act_qdq(x, fmt_block[1])
            t_total += time.perf_counter() - t0
            done_bytes += x.numel() * 2 + out.numel() * 4
        elif fmt == "fp8_block":
            t0 = time.perf_counter()
            if fmt_block == (128, 128):
                q, s = torch_ref.quantize_tensor_tiles(x.float(), (128, 128))
            else:  # float64 weights keep float64 arithmetic (weight_quantizer.py:40-77)
                q, s = torch_ref.quantize_tensor(x if x.dtype == torch.float64 else x.float(),
                                                 fmt_block[1] or x.shape[-1])
            t_total += time.perf_counter() - t0
            done_bytes += x.numel() * x.element_size() + q.numel() + s.numel() * s.element_size()
        else:
            xb = x.view(torch.int16).numpy().view(np.uint16)
            t0 = time.perf_counter()
            q, s = O.mx_quant(xb, "bf16", 8 if fmt == "mxfp8" else 4, nthreads=threads)
            t_total += time.perf_counter() - t0
            done_bytes += x.numel() * 2 + q.size + s.size
    return done_bytes, t_total


class _BucketFill:
    """One bucket of a weight sync: the grouped quantize launch plus the copies."""

    def __init__(self, bucket):
        self.bucket = bucket
        self.algorithmic_bytes = bucket.algorithmic_bytes

    def run(self):
        self.bucket.fill()


class _StateDictCall:
    """One drop-in quantize_state_dict call (plan, allocations and launch)."""

    launch_timed_inside = True  # events bracket the grouped launch, not the host work

    def __init__(self, wq, sd):
        self.wq, self.sd = wq, sd
        n = sum(w.numel() for w in sd.values())
        self.algorithmic_bytes = n * 2 + n + (n // 128) * 2

    def run(self):
        self.out = self.wq.quantize_state_dict(self.sd)


class _LoaderCall:
    """One drop-in DynamicWeightLoader.load_weights call with FP8 on: the whole
    state's unscaled e4m3 cast (plan, allocations and one grouped launch)."""

    launch_timed_inside = True

    def __init__(self, sd):
        from lumenrl_amd.engine.inference import DynamicWeightLoader

        self.loader, self.sd = DynamicWeightLoader, sd
        self.algorithmic_bytes = sum(w.numel() * (w.element_size() + 1) for w in sd.values())

    def update_weights(self, sd):
        self.out = sd

    def run(self):
        self.loader.load_weights(self, self.sd, fp8_config={"enabled": True})


class _RolloutCall:
    """FP8RolloutQuantizer.quantize_model on a Qwen3-8B-shaped module (36 layers x
    q,k,v,o,gate,up,down nn.Linear on the device), then restore_model: the
    weight quantization of every linear plus the module swaps, host work
    included."""

    launch_timed_inside = True

    def __init__(self, torch, ws, names):
        import torch.nn as nn

        from lumenrl_amd.quantization import FP8Config, FP8RolloutQuantizer

        layers = nn.ModuleList()
        it = iter(zip(names, ws))
        for _ in range(36):
            blk = nn.Module()
            for _ in range(7):
                name, w = next(it)
                lin = nn.Linear(w.shape[1], w.shape[0], bias=False, device="meta")
                lin.weight = nn.Parameter(w, requires_grad=False)
                setattr(blk, name.split(".")[-1], lin)
            layers.append(blk)
        self.model = layers
        self.rq = FP8RolloutQuantizer(FP8Config(precision="fp8"))
        n = sum(w.numel() for w in ws)
        self.algorithmic_bytes = n * 2 + n + (n // 128) * 2

    def run(self):
        self.rq.quantize_model(self.model)
        self.rq.restore_model(self.model)


class _F64Calls:
    """WeightQuantizer.quantize_tensor on each float64 weight, one call per
    tensor as the reference's callers make them: float64 arithmetic, float64
    scales, new outputs per call.  One event pair brackets all the calls of a
    step (the host enqueues them ahead of the device)."""

    def __init__(self, torch, ws):
        from lumenrl_amd.quantization import FP8Config, WeightQuantizer

        self.wq, self.ws = WeightQuantizer(FP8Config()), ws
        n = sum(w.numel() for w in ws)
        self.algorithmic_bytes = n * 8 + n + (n // 128) * 8

    def run(self):
        self.out = [self.wq.quantize_tensor(w) for w in self.ws]


class _ActLayer:
    """The activation fake-quant of one layer's linear inputs: one launch per
    input, back to back, each into a preallocated float32 output.  Timed as one
    span per step: an event pair around each 30-100 us launch would add its own
    ~3 us to every launch."""

    def __init__(self, torch, ops, xs):
        self.ops, self.xs = ops, xs
        self.outs = [torch.empty(x.shape, dtype=torch.float32, device=x.device) for x in xs]
        self.algorithmic_bytes = sum(x.numel() * (x.element_size() + 4) for x in xs)

    def run(self):
        for x, out in zip(self.xs, self.outs):
            self.ops.act_qdq(x, 128, out=out)


def _launches(plans) -> int:
    """Kernel launches one step of these grouped plans makes (a plan over many
    tensors runs as several launches of consecutive tensors)."""
    return sum(len(p._launch.parts) for p in plans)


def _bucket_launches(writer) -> int:
    """lrq launches of one sync through these buckets: each bucket's grouped
    quantize launches and its one grouped copy of the pass-through tensors."""
    return sum(_launches([plan for _, plan in b.plans]) + (b.copy_plan is not None) for b in writer)


def setup(torch, ops, cfg, args, dev):
    """The workload of one config, resident on the device: plans (each with
    run() and algorithmic_bytes), the input tensors, and what the JSON line and
    the CPU leg need."""
    flush = None
    if cfg == "c2d":
        ws, _ = qwen3_8b_set(torch, dev, args.seed, "normal")
        qp = ops.QuantPlan(ws, "fp8_block", (1, 128), scale_dtype=torch.bfloat16)
        pairs = qp.run()
        torch.cuda.synchronize()
        plans = [ops.DequantPlan(pairs, (1, 128), torch.bfloat16)]
        workload = "qwen3-8b-linears-fp8-1x128-dequant-to-bf16"
        cpu_ws, cpu_blk, cpu_fmt = pairs, (1, 128), "fp8_dequant"
        extra = {"tensors": len(pairs), "layers": 36, "elements": sum(c.numel() for c, _ in pairs),
                 "format": "fp8_dequant", "launches_per_step": _launches(plans)}
    elif cfg == "c4d":
        ws, _ = qwen3_8b_set(torch, dev, args.seed, "student_t")
        qp = ops.QuantPlan(ws, "mxfp8", (1, 32))
        pairs = qp.run()
        torch.cuda.synchronize()
        del ws
        plans = [ops.DequantPlan(pairs, (1, 32), torch.bfloat16, fmt="mxfp8")]
        ws = [c for c, _ in pairs]
        workload = "qwen3-8b-linears-mxfp8-dequant-to-bf16"
        cpu_ws, cpu_blk, cpu_fmt = pairs, (1, 32), "mx_dequant"
        extra = {"tensors": len(pairs), "layers": 36, "elements": sum(c.numel() for c, _ in pairs),
                 "format": "mxfp8_dequant", "launches_per_step": _launches(plans)}
    elif cfg in ("c2", "c4", "c5", "c2r"):
        kind = {"c2": "normal", "c4": "student_t", "c5": "rowscale", "c2r": "normal"}[cfg]
        fmt = {"c2": "fp8_block", "c4": "mxfp8", "c5": "mxfp4", "c2r": "fp8_block"}[cfg]
        blk = (1, 128) if cfg == "c2r" else (128, 128)
        ws, _ = qwen3_8b_set(torch, dev, args.seed, kind)
        plans = [ops.QuantPlan(ws, fmt, blk)]
        workload = {"c2": "qwen3-8b-linears-fp8-e4m3-128x128", "c4": "qwen3-8b-linears-mxfp8",
                    "c5": "qwen3-8b-linears-mxfp4", "c2r": "qwen3-8b-linears-fp8-e4m3-1x128"}[cfg]
        cpu_ws, cpu_blk, cpu_fmt = ws, blk, fmt
        extra = {"tensors": len(ws), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": fmt, "launches_per_step": _launches(plans)}
    elif cfg == "c2pc":
        # per-channel scales, quantize_tensor(w, block_size=in_features): one
        # grouped launch per row width (1x4096 for six projections, 1x12288
        # for down_proj), since a plan holds one block shape
        ws, _ = qwen3_8b_set(torch, dev, args.seed, "normal")
        by_k: dict = {}
        for w in ws:
            by_k.setdefault(w.shape[1], []).append(w)
        plans = [ops.QuantPlan(g, "fp8_block", (1, k)) for k, g in sorted(by_k.items())]
        workload = "qwen3-8b-linears-fp8-e4m3-per-channel"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 0), "fp8_block"
        extra = {"tensors": len(ws), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": "fp8_block_1xK_per_channel", "launches_per_step": _launches(plans)}
    elif cfg == "f64":
        ws, _ = qwen3_8b_set(torch, dev, args.seed, "normal", layers=4)
        ws = [w.double() for w in ws]  # bf16 values widened exactly
        torch.cuda.synchronize()
        plans = [_F64Calls(torch, ws)]
        workload = "qwen3-8b-4-layers-float64-quantize-tensor-1x128"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 128), "fp8_block"
        extra = {"tensors": len(ws), "layers": 4, "elements": sum(w.numel() for w in ws),
                 "format": "fp8_block_1x128_float64_arithmetic", "launches_per_step": len(ws)}
    elif cfg == "c2sd":
        from lumenrl_amd.quantization import FP8Config, WeightQuantizer

        ws, names = qwen3_8b_set(torch, dev, args.seed, "normal")
        plans = [_StateDictCall(WeightQuantizer(FP8Config()), dict(zip(names, ws)))]
        workload = "qwen3-8b-state-dict-quantize-fp8-1x128-dropin"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 128), "fp8_block"
        extra = {"tensors": len(ws), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": "fp8_block_1x128_bf16_scales",
                 "launches_per_step": len(list(ops.launch_chunks(ws))),
                 "host_work_timed": True}
    elif cfg == "rollout":
        ws, names = qwen3_8b_set(torch, dev, args.seed, "normal")
        plans = [_RolloutCall(torch, ws, names)]
        workload = "qwen3-8b-module-fp8-rollout-quantize-model-1x128"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 128), "fp8_block"
        extra = {"tensors": len(ws), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": "fp8_block_1x128_bf16_scales + module swap and restore",
                 "launches_per_step": len(list(ops.launch_chunks(ws))), "host_work_timed": True}
    elif cfg == "bucket":
        from lumenrl_amd.quantization import QuantizedBucketWriter

        named = qwen3_8b_state(torch, dev, args.seed)
        writer = QuantizedBucketWriter(named, bucket_bytes=2 << 30, fmt="fp8_block")
        plans = [_BucketFill(b) for b in writer]
        ws = [w for _, w in named]
        workload = "qwen3-8b-state-sync-into-fp8-buckets"
        cpu_ws, cpu_blk, cpu_fmt = [], (128, 128), "fp8_block"
        extra = {"tensors": len(named), "buckets": len(writer), "layers": 36,
                 "elements": sum(w.numel() for w in ws),
                 "passthrough_tensors": sum(len(b.copies) for b in writer),
                 "format": "fp8_block_128x128 + passthrough copies",
                 "launches_per_step": _bucket_launches(writer)}
    elif cfg == "cast":
        named = qwen3_8b_state(torch, dev, args.seed)
        plans = [_LoaderCall(dict(named))]
        ws = [w for _, w in named]
        workload = "qwen3-8b-state-unscaled-e4m3-cast-dynamic-weight-loader"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 1), "cast"
        extra = {"tensors": len(named), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": "float8_e4m3fn_unscaled_cast",
                 "launches_per_step": len(list(ops.launch_chunks(ws))),
                 "host_work_timed": True}
    elif cfg == "kv":
        ws, names = qwen3_8b_set(torch, dev, args.seed, "normal")
        ws = [w for w, nm in zip(ws, names) if nm.split(".")[-1] in ("q_proj", "k_proj", "v_proj")]
        plans = [ops.TensorScalePlan(ws)]
        workload = "qwen3-8b-qkv-proj-fp8-kv-scales"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 1), "kv"
        extra = {"tensors": len(ws), "layers": 36, "elements": sum(w.numel() for w in ws),
                 "format": "per_tensor_e4m3_scale", "launches_per_step": 2}
    elif cfg == "act":
        g = torch.Generator(device=dev).manual_seed(args.seed)
        ins = [("q_proj", 4096), ("k_proj", 4096), ("v_proj", 4096), ("o_proj", 4096),
               ("gate_proj", 4096), ("up_proj", 4096), ("down_proj", 12288)]
        ws = []
        for _, k in ins:
            x = torch.empty(PREFILL_TOKENS, k, device=dev, dtype=torch.float32)
            x.normal_(0.0, 1.0, generator=g)
            x[:, :: 97] *= 30.0  # outlier channels
            ws.append(x.to(torch.bfloat16))
            del x
        plans = [_ActLayer(torch, ops, ws)]
        workload = f"qwen3-8b-layer-act-fake-quant-1x128-prefill-{PREFILL_TOKENS}"
        cpu_ws, cpu_blk, cpu_fmt = ws, (1, 128), "act"
        extra = {"tensors": len(ws), "tokens": PREFILL_TOKENS, "elements": sum(x.numel() for x in ws),
                 "format": "act_qdq_1x128_bf16_to_f32", "launches_per_step": len(ws)}
    elif cfg == "c1":
        g = torch.Generator(device=dev).manual_seed(args.seed)
        ws = [gen_weight(torch, 4096, 4096, g, dev)]
        plans = [ops.QuantPlan(ws, "fp8_block", (128, 128))]
        flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        workload = "single-4096x4096-fp8-e4m3-128x128"
        cpu_ws, cpu_blk, cpu_fmt = ws, (128, 128), "fp8_block"
        extra = {"tensors": 1, "elements": ws[0].numel(), "format": "fp8_block",
                 "launches_per_step": 1, "l2_mall_flushed": True}
    elif cfg == "c3":
        plans, ws = [], []
        for layer in range(48):
            gu, dn = moe_layer(torch, dev, args.seed, layer)
            ws += [gu, dn]
            plans.append(ops.QuantPlan([gu, dn], "fp8_block", (128, 128)))
        workload = "qwen3-30b-a3b-experts-fp8-e4m3-128x128"
        cpu_ws, cpu_blk, cpu_fmt = ws[:2], (128, 128), "fp8_block"
        extra = {"tensors": len(ws), "layers": 48, "experts": 128,
                 "elements": sum(w.numel() for w in ws), "format": "fp8_block",
                 "launches_per_step": 48}
    else:
        raise SystemExit(f"unknown config {cfg}")
    return {"plans": plans, "ws": ws, "workload": workload, "extra": extra, "flush": flush,
            "cpu": (cpu_ws, cpu_blk, cpu_fmt)}


def measure(torch, ops, plans, flush, args, stream):
    """Time exactly args.steps steps (after args.warmup untimed ones) of the
    plans, bracketed by synchronizations, with HIP events on the launch stream
    around each event span: a plan run (its grouped launches back to back), or
    the whole step when a step is several plan runs back to back.  ms_per_step
    is the wall time per step (the spans' summed event time when an L2 flush
    separates them); kern_ms is the mean event time of one span,
    spans_per_step how many a step has, and `achieved` the algorithmic GB/s."""
    # A drop-in call (quantize_state_dict, load_weights) plans on the host
    # before and between its grouped launches.  Its kernel time spans its first
    # launch to the end of its last (the small table uploads between launches
    # included), bracketed on the launch stream by one event pair per call: an
    # event per launch would itself stall the stream.  ms_per_step keeps the
    # whole call, host planning included.
    inner = []
    base_run = ops._GroupLaunch.run

    def timed_run(self):
        if inner and not inner[0]:
            a = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            inner[0].append(a)
        return base_run(self)

    ops._GroupLaunch.run = timed_run
    try:
        return _timed_steps(torch, plans, flush, args, stream, inner)
    finally:
        ops._GroupLaunch.run = base_run


def _timed_steps(torch, plans, flush, args, stream, inner):
    # A step of several back-to-back plan runs (C3's 48 per-layer launches) is
    # one event span: an event pair around every 0.28 ms run read C3 0.7 points
    # of HBM peak lower (timed in turns on an MI355X).  A single plan run, the
    # drop-in calls and the L2-flushed C1 keep one span per plan run.
    step_span = (flush is None and len(plans) > 1
                 and not any(getattr(p, "launch_timed_inside", False) for p in plans))
    step_bytes = sum(p.algorithmic_bytes for p in plans)

    def step(ev_pairs=None):
        if step_span and ev_pairs is not None:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for p in plans:
                p.run()
            b.record(stream)
            ev_pairs.append(([(a, b)], step_bytes))
            return
        for p in plans:
            if flush is not None:
                flush.zero_()
            if ev_pairs is not None and getattr(p, "launch_timed_inside", False):
                inner[:] = [[]]
                p.run()
                b = torch.cuda.Event(enable_timing=True)
                b.record(stream)
                ev_pairs.append(([(inner[0][0], b)] if inner[0] else [], p.algorithmic_bytes))
                inner.clear()
            elif ev_pairs is not None:
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                p.run()
                b.record(stream)
                ev_pairs.append(([(a, b)], p.algorithmic_bytes))
            else:
                p.run()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: exactly K steps, synchronized on both sides
    evs = []
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for _ in range(args.steps):
        step(evs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    per = 1 if step_span else len(plans)  # event spans per step
    if len(evs) != per * args.steps or not all(pairs for pairs, _ in evs):
        raise SystemExit("expected timed launches for every plan and step")
    launch_ms = [sum(a.elapsed_time(b) for a, b in pairs) for pairs, _ in evs]
    launch_bytes = [nb for _, nb in evs]
    step_ev_ms = sorted(sum(launch_ms[i * per:(i + 1) * per]) for i in range(args.steps))
    median_step_ms = step_ev_ms[len(step_ev_ms) // 2] if len(step_ev_ms) % 2 else \
        0.5 * (step_ev_ms[len(step_ev_ms) // 2 - 1] + step_ev_ms[len(step_ev_ms) // 2])
    kern_ms = sum(launch_ms) / len(launch_ms)
    achieved = sum(launch_bytes) / len(launch_bytes) / (kern_ms * 1e-3) / 1e9
    if flush is None:
        ms_per_step = wall * 1e3 / args.steps
    else:  # the L2 flush between launches is not part of the step
        ms_per_step = sum(launch_ms) / args.steps
    return {"ms_per_step": ms_per_step, "median_step_ms": median_step_ms, "kern_ms": kern_ms,
            "achieved": achieved, "spans_per_step": per}



# ---------------------------------------------------------------------------
def run(args):
    import torch

    from lumenrl_amd.quantization import ops

    if not torch.cuda.is_available():
        log("bench.py needs a HIP device")
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    cfg = args.config
    t0 = time.time()

    w = setup(torch, ops, cfg, args, dev)
    plans, ws, workload, extra, flush = w["plans"], w["ws"], w["workload"], w["extra"], w["flush"]
    cpu_ws, cpu_blk, cpu_fmt = w["cpu"]
    torch.cuda.synchronize()
    step_bytes = sum(p.algorithmic_bytes for p in plans)
    log(f"[bench] {workload}: {len(ws)} tensors, {step_bytes / 1e9:.3f} GB per step, "
        f"setup {time.time() - t0:.1f}s")

    r = measure(torch, ops, plans, flush, args, stream)
    ms_per_step, median_step_ms, kern_ms, achieved = (r["ms_per_step"], r["median_step_ms"], r["kern_ms"],
                                                      r["achieved"])
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] {ms_per_step:.4f} ms/step, {value:.1f} GB/s; kernel avg {kern_ms:.4f} ms "
        f"({achieved:.1f} GB/s = {achieved / HBM_PEAK_GBS:.1%} of 8 TB/s)")

    # Per launch, as rocprofv3 reports a kernel: a step makes `launches` launches
    # in r["spans_per_step"] event spans, each span's launches back to back, so
    # the mean launch is a span's event time over its launches (the few us
    # between back-to-back launches included).  HBM bytes per launch: the
    # committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of this workload
    # (copy-calibrated), per step, over the step's launches.
    launches = extra["launches_per_step"]
    per_run = launches / r["spans_per_step"]
    traffic = None
    pfile = os.path.join(ROOT, "profiles", PROFILE_FOR.get(cfg, "") + ".md")
    if os.path.exists(pfile):
        with open(pfile) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_step:"):
                    traffic = round(int(line.split(":", 1)[1]) / launches)

    result = {
        "metric": metric_name(),
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "median_ms_per_step_events": round(median_step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if cfg == "f64" else "f32",
        "data": "synthetic (seeded on-device bf16 weights, BASELINE.json distribution"
                + ("; widened to float64)" if cfg == "f64" else ")"),
        "config": {"workload": workload, **extra, "algorithmic_bytes_per_step": step_bytes},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": round(step_bytes / launches),
            "kernel": KERNEL_FOR[cfg],
            "launch_ms": round(kern_ms / per_run, 5),
            "launches_per_span": round(per_run, 3),
            "span_ms": round(kern_ms, 5),
        },
    }
    if not args.no_cpu and cpu_ws:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(torch, cpu_ws, cpu_fmt, cpu_blk, args.cpu_seconds,
                                              full_bytes=step_bytes)
    if cfg == "c2" and not args.no_also:
        del w, plans, ws, cpu_ws
        result["also"] = also_configs(torch, ops, args, dev, stream)
    print(json.dumps(result), flush=True)


ALSO = ("c3", "c4", "c5")


def also_configs(torch, ops, args, dev, stream):
    """The other BASELINE.json quantization configs timed on the device the
    same way (HIP events around every launch, args.steps steps after
    args.warmup), each set freed before the next is built: C3's 48 per-layer
    expert launches, C4 (MXFP8) and C5 (MXFP4) on the whole Qwen3-8B set.
    No CPU leg."""
    out = {}
    for c in ALSO:
        torch.cuda.empty_cache()
        t0 = time.time()
        w = setup(torch, ops, c, args, dev)
        torch.cuda.synchronize()
        nb = sum(p.algorithmic_bytes for p in w["plans"])
        r = measure(torch, ops, w["plans"], w["flush"], args, stream)
        out[c] = {"workload": w["workload"], "kernel": KERNEL_FOR[c],
                  "launches_per_step": w["extra"]["launches_per_step"],
                  "algorithmic_bytes_per_step": nb, "ms_per_step": round(r["ms_per_step"], 5),
                  "value": round(nb / (r["ms_per_step"] * 1e-3) / 1e9, 2),
                  "achieved": round(r["achieved"], 2), "frac": round(r["achieved"] / HBM_PEAK_GBS, 4),
                  "launch_ms": round(r["kern_ms"] * r["spans_per_step"] / w["extra"]["launches_per_step"], 5),
                  "span_ms": round(r["kern_ms"], 5)}
        log(f"[bench] also {c} ({w['workload']}): {r['ms_per_step']:.4f} ms/step, kernel "
            f"{r['achieved']:.1f} GB/s = {r['achieved'] / HBM_PEAK_GBS:.1%}, setup {time.time() - t0:.1f}s")
        del w
    torch.cuda.empty_cache()
    return out


def run_host(args):
    """Host-resident workloads: the drop-in calls on state dicts held in host
    memory, PCIe transfers included.  A step is one whole call; ``value`` is the
    call's algorithmic bytes over its wall time.  These rates are bound by the
    PCIe link, not by HBM, so they carry a ``pcie`` object instead of a kernel
    roofline; the reference's CPU path is timed beside them."""
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = args.config
    t0 = time.time()
    if cfg == "c2host":
        from lumenrl_amd.quantization import FP8Config, WeightQuantizer

        ws, names = qwen3_8b_set(torch, dev, args.seed, "normal")
        sd = {n: w.cpu() for n, w in zip(names, ws)}
        del ws
        wq = WeightQuantizer(FP8Config())
        call = lambda: wq.quantize_state_dict(sd)  # noqa: E731
        n = sum(w.numel() for w in sd.values())
        h2d, d2h = 2 * n, n + (n // 128) * 2
        workload = "qwen3-8b-linears-host-resident-quantize-state-dict-fp8-1x128"
        cpu_ws, cpu_fmt, cpu_blk = list(sd.values()), "fp8_block", (1, 128)
    else:  # casthost
        from lumenrl_amd.engine.inference import DynamicWeightLoader

        named = qwen3_8b_state(torch, dev, args.seed)
        sd = {k: w.cpu() for k, w in named}
        del named

        class _Eng:
            def update_weights(self, s):
                self.sd = s

        eng = _Eng()
        call = lambda: DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True})  # noqa: E731
        n = sum(w.numel() for w in sd.values())
        h2d, d2h = 2 * n, n
        workload = "qwen3-8b-state-host-resident-dynamic-weight-loader-e4m3-cast"
        cpu_ws, cpu_fmt, cpu_blk = list(sd.values()), "cast", (1, 1)
    torch.cuda.synchronize()
    alg = h2d + d2h
    log(f"[bench] {workload}: {len(sd)} host tensors, {alg / 1e9:.3f} GB per call, "
        f"setup {time.time() - t0:.1f}s")
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    times = []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        a = time.perf_counter()
        call()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - a)
    peak = torch.cuda.max_memory_allocated() - base
    ms = sum(times) / len(times) * 1e3
    med = sorted(times)[len(times) // 2] * 1e3
    value = alg / (ms * 1e-3) / 1e9
    log(f"[bench] {ms:.1f} ms/call ({value:.1f} GB/s algorithmic, H2D {h2d / ms / 1e6:.1f} GB/s), "
        f"device peak {peak / 2**20:.0f} MiB")
    result = {
        "metric": metric_name() + " [host-resident variant: PCIe-inclusive, not the HBM metric]",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "median_ms_per_step": round(med, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded on-device bf16 weights copied to host memory)",
        "config": {"workload": workload, "tensors": len(sd), "elements": n, "host_resident": True,
                   "algorithmic_bytes_per_step": alg,
                   "window_bytes": _ops().HOST_WINDOW_BYTES, "window_depth": _ops().HOST_WINDOW_DEPTH},
        "roofline": None,
        "pcie": {"h2d_bytes": h2d, "d2h_bytes": d2h, "h2d_GBps": round(h2d / ms / 1e6, 2),
                 "d2h_GBps": round(d2h / ms / 1e6, 2), "link_peak_GBps_per_direction": 64.0,
                 "device_peak_bytes": int(peak)},
    }
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(torch, cpu_ws, cpu_fmt, cpu_blk, args.cpu_seconds,
                                              full_bytes=alg)
    print(json.dumps(result), flush=True)


def _ops():
    from lumenrl_amd.quantization import ops

    return ops


def run_copy(args):
    """Plain device copy of a known size, for scaling rocprof FETCH/WRITE counters."""
    import torch

    dev = torch.device("cuda", 0)
    n = args.copy_bytes
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    print(json.dumps({"mode": "copy", "bytes_read": n, "bytes_written": n, "ms": ms,
                      "GBps": 2 * n / (ms * 1e-3) / 1e9}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "c2r", "c2pc", "c2d", "c2sd", "bucket",
                                                      "act", "kv", "cast", "c4d", "c2host", "casthost",
                                                      "rollout", "f64"])
    ap.add_argument("--seed", type=int, default=1000)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-also", action="store_true",
                    help="with --config c2: skip the C3/C4/C5 device timings of the `also` object")
    ap.add_argument("--mode", default="quant", choices=["quant", "copy"])
    ap.add_argument("--copy-bytes", type=int, default=1 << 30)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the quantize path is per-device with no "
              "collectives (each rank would quantize its own shard); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if args.mode == "copy":
        run_copy(args)
    elif args.config in ("c2host", "casthost"):
        run_host(args)
    else:
        run(args)


if __name__ == "__main__":
    main()
