"""BASELINE configs 2-5 at their full sizes on an MI355X.

The inputs are the ones bench.py times, from its generators and seed.
- C2 (the whole Qwen3-8B linear set, 128x128 FP8), C4 (MXFP8) and C5 (MXFP4)
  are compared with the CPU oracle bit for bit, tensor by tensor.
- C3 (Qwen3-30B-A3B experts, 48 layers x 128 experts, one launch per layer)
  is too large for the oracle in a test's time.  Every layer is checked
  through exact size-independent properties:
  - each tile's scale equals max(RN(amax/448), FLT_MIN) computed by numpy
    from the device's exact tile amax;
  - each tile's largest |code| is 448 (0x7E) unless the tile is zero or
    non-finite.
  Three whole layers, and every layer's planted zero-tile and inf-tile
  experts, are also compared with the oracle bit for bit.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import bench as B
from oracle import oracle as O
from lumenrl_amd.quantization import QuantPlan

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
SEED = 1000  # bench.py's default --seed
THREADS = max(1, min(os.cpu_count() or 1, 16))


def say(*a):
    print(*a, flush=True)


def host16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def host8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _compare_set(kind: str, fmt: str) -> None:
    ws, names = B.qwen3_8b_set(torch, DEV, SEED, kind)
    blk = (128, 128) if fmt == "fp8_block" else (1, 32)
    plan = QuantPlan(ws, fmt, blk)
    outs = plan.run()
    torch.cuda.synchronize()
    say(fmt, kind, len(ws), "tensors quantized; comparing with the oracle")
    for name, w, (codes, scales) in zip(names, ws, outs):
        xb = host16(w)
        if fmt == "fp8_block":
            oc, osc = O.fp8_block_quant(xb, "bf16", "f32", blk, False, nthreads=THREADS)
            assert np.array_equal(host8(codes), oc[0]), name
            sc = scales.detach().cpu().numpy()
            assert np.array_equal(sc.view(np.uint32), osc[0].view(np.uint32)), name
        else:
            oc, osc = O.mx_quant(xb, "bf16", 8 if fmt == "mxfp8" else 4, nthreads=THREADS)
            assert np.array_equal(host8(codes).reshape(oc.shape), oc), name
            assert np.array_equal(host8(scales).reshape(osc.shape), osc), name


def test_c2_full_qwen3_8b_set_fp8_128x128_bit_exact():
    _compare_set("normal", "fp8_block")


def test_c4_full_qwen3_8b_set_mxfp8_bit_exact():
    _compare_set("student_t", "mxfp8")


def test_c5_full_qwen3_8b_set_mxfp4_bit_exact():
    _compare_set("rowscale", "mxfp4")


def _tile_amax(w: torch.Tensor) -> np.ndarray:
    """Exact per-128x128-tile max |x| of an [E, R, C] bf16 stack, as float32."""
    e, r, c = w.shape
    a = w.view(e, r // 128, 128, c // 128, 128).abs().amax(dim=(2, 4))
    return a.float().cpu().numpy()


def test_c3_all_48_layers_experts():
    tiny = np.float32(np.finfo(np.float32).tiny)
    oracle_layers = {0, 23, 47}
    for layer in range(48):
        gu, dn = B.moe_layer(torch, DEV, SEED, layer)
        plan = QuantPlan([gu, dn], "fp8_block", (128, 128))
        outs = plan.run()
        torch.cuda.synchronize()
        for w, (codes, scales) in zip((gu, dn), outs):
            amax = _tile_amax(w)
            with np.errstate(over="ignore"):
                want = np.maximum(amax / np.float32(448.0), tiny).astype(np.float32)
            got = scales.detach().cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), layer
            e, r, c = w.shape
            cm = codes.view(torch.uint8).view(e, r // 128, 128, c // 128, 128)
            top = (cm & 0x7F).amax(dim=(2, 4)).cpu().numpy()
            finite = np.isfinite(amax) & (amax > 0)
            assert np.all(top[finite] == 0x7E), layer
            assert np.all(top[amax == 0] == 0), layer
            # the planted zero and inf tiles: their experts bit-exact with the oracle
            special = sorted(set(np.nonzero(~finite)[0].tolist()))
            for ex in special:
                oc, osc = O.fp8_block_quant(host16(w[ex]), "bf16", "f32", (128, 128), False,
                                            nthreads=THREADS)
                assert np.array_equal(host8(codes[ex]), oc[0]), (layer, ex)
                assert np.array_equal(got[ex].view(np.uint32), osc[0].view(np.uint32)), (layer, ex)
            if layer in oracle_layers:
                say("C3 layer", layer, "whole layer against the oracle")
                oc, osc = O.fp8_block_quant(host16(w), "bf16", "f32", (128, 128), False,
                                            nthreads=THREADS)
                assert np.array_equal(host8(codes), oc), layer
                assert np.array_equal(got.view(np.uint32), osc.view(np.uint32)), layer
        del gu, dn, plan, outs


def test_cast_full_qwen3_8b_state_through_the_loader():
    """bench.py's cast workload at full size: the whole Qwen3-8B state (399 tensors,
    8.19 G elements, embeddings and lm_head included) through DynamicWeightLoader's
    chunked grouped launches (2 M work-groups in all), each tensor bit-equal to
    torch's own cast of it.  The state is finite, where torch's device cast and
    its x86 cast agree (every bf16 pattern is checked against the x86 cast in
    test_gpu_cast.py)."""
    from lumenrl_amd.engine.inference import DynamicWeightLoader

    class Sink:
        def update_weights(self, sd):
            self.sd = sd

    named = B.qwen3_8b_state(torch, DEV, SEED)
    sd = dict(named)
    sink = Sink()
    DynamicWeightLoader.load_weights(sink, sd, fp8_config={"enabled": True})
    torch.cuda.synchronize()
    say("cast of the whole state done; comparing", len(sd), "tensors")
    assert list(sink.sd) == list(sd)
    for name, w in sd.items():
        assert torch.isfinite(w).all(), name
        want = w.to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(sink.sd[name].view(torch.uint8), want), name


@pytest.mark.parametrize("kind,fmt", [("student_t", "mxfp8"), ("rowscale", "mxfp4")])
def test_mx_full_set_dequantize_then_requantize_is_identity(kind, fmt):
    """C4 / C5 at full size, size-independent property: MX dequantization is exact
    (element * 2^(E-127)), and re-quantizing those float32 values gives back the same
    E8M0 exponents and codes (the group maximum keeps its binade), so
    quantize -> dequantize -> quantize is the identity on every one of the 252 tensors."""
    from lumenrl_amd.quantization.ops import DequantPlan

    ws, names = B.qwen3_8b_set(torch, DEV, SEED, kind)
    q1 = QuantPlan(ws, fmt, (1, 32)).run()
    torch.cuda.synchronize()
    del ws
    back = DequantPlan(q1, (1, 32), torch.float32, fmt=fmt).run()
    q2 = QuantPlan(back, fmt, (1, 32)).run()
    torch.cuda.synchronize()
    say(fmt, "round trip of", len(names), "tensors done; comparing")
    for name, (c1, s1), (c2, s2) in zip(names, q1, q2):
        assert torch.equal(c1.view(torch.uint8), c2.view(torch.uint8)), name
        assert torch.equal(s1, s2), name


def test_c2d_full_dequantize_state_dict_layout_matches_torch_ops():
    """bench.py's c2d workload at full size: the C2 weights quantized to 1x128 blocks
    with bf16 scales (quantize_state_dict's layout), then dequantized to bf16 in one
    grouped launch, equal on every tensor to the reference's op sequence
    (weight_quantizer.py:79-89, :133: fp32(code) * fp32(scale), then bf16) run by
    torch on the same device (finite data: no NaN payloads involved)."""
    from lumenrl_amd.quantization.ops import DequantPlan

    ws, names = B.qwen3_8b_set(torch, DEV, SEED, "normal")
    pairs = QuantPlan(ws, "fp8_block", (1, 128), scale_dtype=torch.bfloat16).run()
    torch.cuda.synchronize()
    del ws
    outs = DequantPlan(pairs, (1, 128), torch.bfloat16).run()
    torch.cuda.synchronize()
    say("c2d", len(names), "tensors dequantized; comparing with torch's ops")
    for name, (c, s), out in zip(names, pairs, outs):
        want = (c.float() * s.float().repeat_interleave(128, dim=1)).to(torch.bfloat16)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), name


def test_act_and_kv_full_size_match_torch_ops_on_device():
    """bench.py's act and kv workloads at full size against the reference's op
    sequences (fp8_rollout.py:53-72; fp8_kv_cache.py:52-54) run by torch on the same
    device: the 7 linear inputs of a Qwen3-8B layer for an 8192-token prefill chunk,
    and the 108 q/k/v_proj weights of the C2 set (finite data)."""
    from oracle import torch_ref as T
    from lumenrl_amd.quantization import TensorScalePlan, act_qdq

    g = torch.Generator(device=DEV).manual_seed(SEED)
    for k in (4096,) * 6 + (12288,):
        x = torch.empty(B.PREFILL_TOKENS, k, device=DEV, dtype=torch.float32).normal_(0.0, 1.0, generator=g)
        x[:, ::97] *= 30.0
        xb = x.to(torch.bfloat16)
        got = act_qdq(xb, 128)
        want = T.act_qdq(xb, 128)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), k
    ws, names = B.qwen3_8b_set(torch, DEV, SEED, "normal")
    qkv = [w for w, n in zip(ws, names) if n.split(".")[-1] in ("q_proj", "k_proj", "v_proj")]
    assert len(qkv) == 108
    scales = TensorScalePlan(qkv).run()
    want = torch.stack([T.kv_scale(w) for w in qkv])
    torch.cuda.synchronize()
    assert torch.equal(scales.view(torch.int32), want.view(torch.int32))


def test_bucket_full_qwen3_8b_state_sync():
    """bench.py's bucket workload at full size: the whole Qwen3-8B state synced into
    2 GiB transfer buckets.  Every quantized entry (codes and `_scale_inv`) read back
    through the receiver's views equals a separate grouped launch on the same weight,
    whose bytes test_c2 pins to the oracle; every pass-through tensor arrives intact."""
    from lumenrl_amd.quantization import QuantizedBucketWriter

    named = B.qwen3_8b_state(torch, DEV, SEED)
    src = dict(named)
    writer = QuantizedBucketWriter(named, bucket_bytes=2 << 30, fmt="fp8_block")
    quantized = [n for n, _ in named if n.endswith("proj.weight")]
    ref = dict(zip(quantized, QuantPlan([src[n] for n in quantized], "fp8_block", (128, 128)).run()))
    seen = set()
    for bucket in writer:
        bucket.fill()
        torch.cuda.synchronize()
        for name, t in bucket.views():
            seen.add(name)
            if name.endswith("_scale_inv"):
                assert torch.equal(t, ref[name[: -len("_scale_inv")]][1]), name
            elif name in ref:
                assert torch.equal(t.view(torch.uint8), ref[name][0].view(torch.uint8)), name
            else:
                assert torch.equal(t, src[name]), name
    assert seen == set(src) | {n + "_scale_inv" for n in quantized}
    say("bucket sync of", len(src), "tensors in", len(writer), "buckets checked")
