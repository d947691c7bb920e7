"""Weight-sync plans across steps, on an MI355X.

A plan is built once and run every sync.  These tests change what the caller
hands over between runs -- parameters moved to other storage (``p.data = new``),
brand-new tensors each sync (as ``DTensor.full_tensor()`` produces,
actor_worker.py:1208-1216) -- and check every run's output bit for bit against
the CPU oracle.  The transfer buckets are decoded exactly as the reference's
two receivers decode them (bucketed_weight_transfer.py:262-270,
rdma_weight_transfer.py:176-180), including a bucket that mixes bf16 weights
with an fp32 one.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import oracle as O
from lumenrl_amd.quantization import QuantizedBucketWriter, encode_bucket, ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
RNG = np.random.default_rng(90210)


def say(*a):
    print(*a, flush=True)


def weight(shape, dtype=torch.bfloat16):
    x = RNG.normal(0.0, 0.02, shape).astype(np.float32)
    x.flat[RNG.integers(0, x.size)] = RNG.uniform(0.5, 4.0)
    return torch.from_numpy(x).to(dtype).to(DEV)


def host(t: torch.Tensor) -> tuple[np.ndarray, str]:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy(), "f32"
    return t.view(torch.int16).numpy().view(np.uint16), "bf16"


def oracle_tiles(t: torch.Tensor):
    x, dt = host(t)
    c, s = O.fp8_block_quant(x.reshape((-1,) + x.shape[-2:]), dt, "f32", (128, 128))
    return c.reshape(-1), s.view(np.uint32).reshape(-1)


def assert_plan_matches(plan: ops.QuantPlan, tensors):
    torch.cuda.synchronize()
    for (codes, scales), t in zip(plan.outputs, tensors):
        oc, osc = oracle_tiles(t)
        assert np.array_equal(codes.view(torch.uint8).cpu().numpy().reshape(-1), oc)
        assert np.array_equal(scales.cpu().numpy().view(np.uint32).reshape(-1), osc)


def test_plan_follows_moved_storage_and_new_inputs():
    params = [torch.nn.Parameter(weight(s), requires_grad=False)
              for s in [(256, 384), (128, 512), (3, 128, 256)]]
    plan = ops.QuantPlan(params, "fp8_block", (128, 128))
    plan.run()
    assert_plan_matches(plan, params)
    outputs = [pair for pair in plan.outputs]
    # an FSDP-style re-gather: the parameter now lives in a fresh allocation
    params[1].data = weight((128, 512))
    plan.run()
    assert_plan_matches(plan, params)
    # a sync that produces brand-new tensors every step (full_tensor() / .to())
    fresh = [weight(tuple(p.shape)) for p in params]
    plan.run(inputs=fresh)
    assert_plan_matches(plan, fresh)
    # same storage handed over again: no re-pack, same outputs
    table = plan._launch
    plan.run(inputs=fresh)
    assert plan._launch is table
    assert all(a[0] is b[0] and a[1] is b[1] for a, b in zip(plan.outputs, outputs))
    # a changed shape or dtype needs a new plan
    with pytest.raises(ValueError, match="build a new plan"):
        plan.run(inputs=[fresh[0], weight((128, 640)), fresh[2]])
    with pytest.raises(ValueError, match="build a new plan"):
        plan.run(inputs=[fresh[0], fresh[1].float(), fresh[2]])
    # the plan now reads `fresh`: changing the old parameters leaves it alone ...
    params[2].data = weight((3, 128, 256))
    plan.run()
    assert_plan_matches(plan, fresh)
    # ... and a bound input that changes shape is refused
    fresh[0].data = weight((128, 384))
    with pytest.raises(ValueError, match="build a new plan"):
        plan.run()


def test_plan_refuses_an_input_resized_in_place():
    """A shrink by ``resize_`` keeps the storage address and strides; the plan
    must still notice that the planned shape is gone."""
    w = weight((3, 128, 256))
    plan = ops.QuantPlan([w], "fp8_block", (128, 128))
    plan.run()
    assert_plan_matches(plan, [w])
    ptr = w.data_ptr()
    w.resize_(2, 128, 256)
    assert w.data_ptr() == ptr
    with pytest.raises(ValueError, match="build a new plan"):
        plan.run()


def decode_zmq(bucket):
    """BucketedWeightReceiver's decode of one bucket (bucketed_weight_transfer.py:262-270)."""
    weights = []
    for name, meta in bucket.bucket_meta().items():
        shape, dtype, offset, handle = meta["shape"], meta["dtype"], meta["offset"], meta["handle"]
        assert handle is None
        size = dtype.itemsize * shape.numel()
        tensor = bucket.buffer[offset: offset + size].view(dtype=dtype).view(shape)
        weights.append((name, tensor))
    return weights


def decode_rdma(bucket):
    """The RCCL receiver's decode (rdma_weight_transfer.py:176-180), metadata via JSON."""
    metadata = json.loads(json.dumps(bucket.rdma_entries()).encode("utf-8").decode("utf-8"))
    payload = bucket.buffer
    weights = []
    for entry in metadata:
        dtype = getattr(torch, entry["dtype"])
        start = int(entry["offset"])
        end = start + int(entry["nbytes"])
        value = payload[start:end].view(dtype).view(entry["shape"])
        weights.append((entry["name"], value))
    return weights


def check_received(writer, named_src):
    seen = set()
    for bucket in writer:
        bucket.fill()
        torch.cuda.synchronize()
        a, b = decode_zmq(bucket), decode_rdma(bucket)
        assert [n for n, _ in a] == [n for n, _ in b]
        for (name, t), (_, t2) in zip(a, b):
            assert t.dtype == t2.dtype and t.shape == t2.shape
            assert torch.equal(t.view(torch.uint8), t2.view(torch.uint8))
            seen.add(name)
            base = name[: -len("_scale_inv")] if name.endswith("_scale_inv") else name
            w = named_src[base]
            if name == base and t.dtype == w.dtype:  # pass-through
                assert torch.equal(t, w), name
                continue
            oc, osc = oracle_tiles(w)
            if name == base:
                assert t.dtype == torch.float8_e4m3fn and tuple(t.shape) == tuple(w.shape)
                assert np.array_equal(t.view(torch.uint8).cpu().numpy().reshape(-1), oc), name
            else:
                assert t.dtype == torch.float32
                assert np.array_equal(t.cpu().numpy().view(np.uint32).reshape(-1), osc), name
    return seen


def test_mixed_dtype_bucket_decoded_like_the_reference_receivers():
    named = [("model.embed_tokens.weight", weight((512, 256))),
             ("model.layers.0.self_attn.q_proj.weight", weight((512, 512))),
             ("model.layers.0.mlp.gate.weight", weight((128, 512), torch.float32)),  # fp32 router
             ("model.layers.0.input_layernorm.weight", torch.ones(512, dtype=torch.bfloat16, device=DEV)),
             ("model.layers.0.mlp.experts.w13", weight((4, 256, 384))),
             ("model.layers.0.mlp.down_proj.weight", weight((256, 1024), torch.float32)),
             ("lm_head.weight", weight((512, 256)))]
    writer = QuantizedBucketWriter(named, bucket_bytes=8 << 20, fmt="fp8_block")
    assert len(writer) == 1
    assert sorted(str(p.dtype) for _, p in writer.buckets[0].plans) == ["torch.bfloat16", "torch.float32"]
    src = dict(named)
    seen = check_received(writer, src)
    quantized = {n for n, _ in named if "proj" in n or "gate" in n or "experts" in n}
    assert seen == set(src) | {n + "_scale_inv" for n in quantized}

    # next sync: new tensors for some weights (rebind), a moved norm (p.data swap)
    fresh = {n: weight(tuple(w.shape), w.dtype) for n, w in named if n in quantized}
    fresh["lm_head.weight"] = weight((512, 256))
    writer.rebind(list(fresh.items()))
    src.update(fresh)
    norm = src["model.layers.0.input_layernorm.weight"]
    norm.data = torch.full((512,), 0.5, dtype=torch.bfloat16, device=DEV)
    check_received(writer, src)
    with pytest.raises(ValueError):
        writer.rebind([("lm_head.weight", weight((512, 128)))])
    with pytest.raises(KeyError):
        writer.rebind([("nope", weight((512, 128)))])


def test_bucket_with_a_width_8_does_not_divide():
    """A custom quantize_if may admit a [130, 100] weight: its 128x128 tiles need
    the generic kernel, so it gets a launch of its own next to the vector one."""
    named = [("a.q_proj.weight", weight((256, 512))), ("a.odd_proj.weight", weight((130, 100))),
             ("a.k_proj.weight", weight((128, 256)))]
    writer = QuantizedBucketWriter(named, bucket_bytes=4 << 20, fmt="fp8_block",
                                   quantize_if=lambda n, t: t.dim() == 2)
    assert len(writer) == 1 and len(writer.buckets[0].plans) == 2
    seen = check_received(writer, dict(named))
    assert seen == {n for n, _ in named} | {n + "_scale_inv" for n, _ in named}


def test_encode_bucket_like_the_rccl_sender():
    """encode_bucket mirrors _encode_bucket (rdma_weight_transfer.py:22-57): compact
    JSON metadata as a uint8 device tensor, and a payload the receiver decodes with
    its own expressions (rdma_weight_transfer.py:170-180) -- here with FP8 codes and
    scales for the linear weights and the rest unchanged, CPU inputs included."""
    named = [("model.embed_tokens.weight", weight((256, 256))),
             ("model.layers.0.self_attn.o_proj.weight", weight((384, 512))),
             ("model.layers.0.post_attention_layernorm.weight", torch.ones(512, dtype=torch.bfloat16)),
             ("model.layers.0.mlp.experts.w2", weight((2, 256, 128)).cpu()),
             ("model.layers.0.mlp.gate.weight", weight((64, 256), torch.float32))]
    metadata, payload = encode_bucket(named)
    torch.cuda.synchronize()
    assert metadata.dtype == torch.uint8 and metadata.is_cuda and payload.dtype == torch.uint8
    entries = json.loads(bytes(metadata.cpu().tolist()).decode("utf-8"))
    raw = json.dumps(entries, separators=(",", ":")).encode("utf-8")
    assert bytes(metadata.cpu().tolist()) == raw
    src = {n: w.to(DEV) for n, w in named}
    seen = set()
    for entry in entries:
        dtype = getattr(torch, entry["dtype"])
        start = int(entry["offset"])
        end = start + int(entry["nbytes"])
        value = payload[start:end].view(dtype).view(entry["shape"])
        name = entry["name"]
        seen.add(name)
        base = name[: -len("_scale_inv")] if name.endswith("_scale_inv") else name
        w = src[base]
        if name == base and value.dtype == w.dtype:
            assert torch.equal(value, w), name
            continue
        oc, osc = oracle_tiles(w)
        got = value.view(torch.uint8) if name == base else value
        want = oc if name == base else osc
        assert np.array_equal(got.cpu().numpy().reshape(-1).view(np.uint8 if name == base else np.uint32), want), name
    assert seen == set(src) | {n + "_scale_inv" for n in src if "proj" in n or "experts" in n or "gate" in n}
    with pytest.raises(ValueError, match="empty weight bucket"):
        encode_bucket([])
