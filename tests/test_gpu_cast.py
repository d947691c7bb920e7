"""Unscaled e4m3fn cast and the DynamicWeightLoader drop-in on an MI355X.

The oracle is torch's own CPU cast, ``tensor.to(torch.float8_e4m3fn)`` -- the
reference's op (lumenrl/engine/inference/weight_loader.py:33) -- and
oracle.cast_e4m3, which test_oracle.py pins to it on every 16-bit pattern.
Bit-exact throughout, NaN signs included.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from lumenrl_amd import _lib
from lumenrl_amd.engine.inference import DynamicWeightLoader
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
RNG = np.random.default_rng(99)


def say(*a):
    print(*a, flush=True)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def torch_cast(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float8_e4m3fn).view(torch.uint8).numpy()


@pytest.mark.parametrize("tdt", [torch.bfloat16, torch.float16])
def test_every_16bit_pattern(tdt):
    """All 65536 bit patterns, repeated to 1 MiB so the vector path, the
    misaligned walk (offset views) and ragged tails all see them."""
    say("cast every pattern", tdt)
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(np.tile(b, 16).view(np.int16)).view(tdt).to(DEV)
    want = torch_cast(x)
    assert np.array_equal(u8(ops.cast_e4m3(x)), want)
    for off, n in ((1, 65535), (3, 40001), (8, 4097), (5, 7)):
        v = x[off:off + n]
        assert np.array_equal(u8(ops.cast_e4m3(v)), want[off:off + n]), (off, n)


def test_float32_patterns_and_specials():
    say("cast float32")
    f = RNG.integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    f[:10] = [464.0, 464.00003, -464.0, 448.0, 1e-9, -0.0, np.inf, -np.inf, np.nan, -np.nan]
    x = torch.from_numpy(f).to(DEV)
    assert np.array_equal(u8(ops.cast_e4m3(x)), O.cast_e4m3(f, "f32"))
    assert np.array_equal(u8(ops.cast_e4m3(x[1:100003])), torch_cast(x[1:100003]))


def test_grouped_cast_of_ragged_tensors():
    say("grouped cast")
    shapes = [(4096, 1000), (3,), (0,), (1, 8), (129, 7), (8191,), (2, 3, 4097)]
    ws = [(torch.randn(s, device=DEV) * 40).to(torch.bfloat16) for s in shapes]
    ws[1][1] = float("nan")
    ws[4][5, 6] = -float("inf")
    plan = ops.CastPlan(ws)
    outs = plan.run()
    torch.cuda.synchronize()
    for w, q in zip(ws, outs):
        assert q.dtype == torch.float8_e4m3fn and q.shape == w.shape
        assert np.array_equal(u8(q), torch_cast(w))
    for w in ws:  # re-run on new values
        w.mul_(-3)
    plan.run()
    torch.cuda.synchronize()
    for w, q in zip(ws, outs):
        assert np.array_equal(u8(q), torch_cast(w))


class _Engine:
    def update_weights(self, sd):
        self.sd = sd


def _mixed_state():
    g = torch.Generator(device=DEV).manual_seed(5)
    sd = {
        "model.embed_tokens.weight": (torch.randn(1000, 256, generator=g, device=DEV) * 0.02).to(torch.bfloat16),
        "model.layers.0.mlp.down_proj.weight": (torch.randn(256, 384, generator=g, device=DEV) * 300).to(torch.bfloat16),
        "model.layers.0.input_layernorm.weight": torch.randn(256, generator=g, device=DEV).to(torch.float16),
        "model.layers.0.self_attn.q_proj.weight": torch.randn(384, 256, generator=g, device=DEV) * 0.5,
        "model.layers.0.self_attn.rotary.inv_freq": torch.rand(64, dtype=torch.float64) * 1e3,
        "model.layers.0.mlp.gate.e_score_bias": (torch.randn(32) * 100).to(torch.float8_e5m2),
        "cpu.bf16.weight": (torch.randn(130, 256) * 10).to(torch.bfloat16),
        "already.e4m3": torch.randn(16, device=DEV).to(torch.float8_e4m3fn),
        "empty.weight": torch.empty(0, 128, dtype=torch.bfloat16, device=DEV),
        "step": torch.tensor([7], device=DEV),
        "mask": torch.tensor([True, False]),
    }
    sd["model.layers.0.mlp.down_proj.weight"][3, 5] = float("nan")
    return sd


def test_dynamic_weight_loader_matches_the_reference_cast():
    """Every floating tensor becomes torch's .to(float8_e4m3fn) of it, on its
    own device; the rest pass through untouched, in the same key order."""
    say("DynamicWeightLoader unscaled")
    sd, eng = _mixed_state(), _Engine()
    DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True, "dtype": "FP8"})
    out = eng.sd
    assert list(out) == list(sd)
    for k, t in sd.items():
        if not t.dtype.is_floating_point or t.dtype == torch.float8_e4m3fn:
            assert out[k] is t, k
            continue
        q = out[k]
        assert q.dtype == torch.float8_e4m3fn and q.shape == t.shape and q.device == t.device, k
        assert np.array_equal(u8(q), torch_cast(t)), k


def test_dynamic_weight_loader_scaled_extension():
    """fp8_config["scaled"]: linear weights become 128x128 blockwise codes plus
    float32 <name>_scale_inv (the oracle's fp8_block_quant); embeddings, norms
    and everything else keep their dtype and identity."""
    say("DynamicWeightLoader scaled")
    sd, eng = _mixed_state(), _Engine()
    # a contiguous weight view 2 bytes into its buffer: not 16-byte aligned, so it
    # cannot share the grouped launch (its own launch instead)
    base = (torch.randn(64 * 256 + 1, device=DEV) * 0.02).to(torch.bfloat16)
    sd["model.layers.1.self_attn.o_proj.weight"] = base[1:].view(64, 256)
    DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True, "scaled": True})
    out = eng.sd
    quantized = {"model.layers.0.mlp.down_proj.weight", "model.layers.0.self_attn.q_proj.weight",
                 "cpu.bf16.weight", "model.layers.1.self_attn.o_proj.weight"}
    empty = out["empty.weight"], out["empty.weight_scale_inv"]
    assert empty[0].shape == (0, 128) and empty[1].shape == (0, 1)
    for k, t in sd.items():
        if k == "empty.weight":
            continue
        if k not in quantized:
            assert out[k] is t, k
            continue
        codes, scales = out[k], out[f"{k}_scale_inv"]
        assert codes.device == t.device and scales.dtype == torch.float32
        dt = "f32" if t.dtype == torch.float32 else "bf16"
        xh = t.detach().cpu().contiguous()
        xh = xh.numpy() if dt == "f32" else xh.view(torch.int16).numpy().view(np.uint16)
        oc, osc = O.fp8_block_quant(xh[None], dt, "f32", (128, 128))
        assert np.array_equal(u8(codes).reshape(oc.shape), oc), k
        assert np.array_equal(scales.cpu().numpy().view(np.uint32).reshape(-1),
                              osc.view(np.uint32).reshape(-1)), k
    keys = list(out)
    for k in quantized:
        assert keys.index(f"{k}_scale_inv") == keys.index(k) + 1


def test_single_call_entry_point_through_the_c_abi():
    x = (torch.randn(10007, device=DEV) * 100).to(torch.bfloat16)
    out = torch.empty(10007, dtype=torch.uint8, device=DEV)
    rc = _lib.lib().lrq_cast_e4m3(x.data_ptr(), _lib.DTYPE_BF16, x.numel(), out.data_ptr(), None)
    _lib.check(rc, "lrq_cast_e4m3")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), torch_cast(x))


def test_dynamic_weight_loader_over_several_launches():
    """A 45-tensor state of two dtypes: each dtype's group launches in chunks
    (8, 16, then the rest); every tensor equals torch's own cast, in key order."""
    g = torch.Generator(device=DEV).manual_seed(8)
    sd = {}
    for i in range(45):
        n = 1000 + 37 * i
        t = torch.randn(n, generator=g, device=DEV) * (0.01 * (1 + i % 5))
        if i % 11 == 4:
            t[7] = float("inf")
        sd[f"t{i}"] = t.to(torch.float16 if i % 3 == 0 else torch.bfloat16)
    say("DynamicWeightLoader over several launches")
    eng = _Engine()
    DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True})
    assert list(eng.sd) == list(sd)
    for k, t in sd.items():
        q = eng.sd[k]
        assert q.dtype == torch.float8_e4m3fn and q.shape == t.shape, k
        assert np.array_equal(u8(q), torch_cast(t)), k
