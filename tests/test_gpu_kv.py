"""Per-tensor FP8 scales (KV-cache recalibration) on an MI355X: the grouped
amax + scale kernels against the CPU oracle and the reference's torch ops
(bit-exact), and the ``FP8KVCacheQuantizer`` mirror
(lumenrl/quantization/fp8_kv_cache.py:26-80)."""

from __future__ import annotations

import logging

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import oracle as O
from oracle import torch_ref as T
from lumenrl_amd.quantization import FP8Config, FP8KVCacheQuantizer, TensorScalePlan

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
RNG = np.random.default_rng(4242)


def say(*a):
    print(*a, flush=True)


def oracle_scale(t: torch.Tensor, dt: str) -> int:
    t = t.detach().cpu().contiguous()
    x = t.numpy() if dt == "f32" else t.view(torch.int16).numpy().view(np.uint16)
    return int(O.tensor_scale(x, dt))


def bits(s: torch.Tensor) -> int:
    return s.detach().cpu().reshape(1).view(torch.int32).item() & 0xFFFFFFFF


def weight(shape, dt, case="weights"):
    x = (RNG.standard_normal(shape) * 0.02).astype(np.float32)
    x.flat[RNG.integers(0, x.size)] = RNG.choice([-1.0, 1.0]) * RNG.uniform(0.5, 4.0)
    if case == "zero":
        x[:] = 0.0
    elif case == "subnormal":
        x[:] = 1e-40 if dt != "f16" else 3e-8
    elif case == "inf":
        x.flat[x.size // 3] = -np.inf
    elif case == "nan":
        x.flat[x.size - 5] = np.nan
    elif case == "huge":
        x.flat[7] = 3.0e38 if dt != "f16" else -65504.0
    return torch.from_numpy(x).to(DT[dt]).to(DEV)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_tensor_scales_qwen3_layers_vs_oracle(dt):
    """Two Qwen3-8B layers' q/k/v plus ragged and special-value tensors in one table."""
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096)] * 2 + [(1000, 4100), (3, 8), (1, 1), (77, 129)]
    cases = ["weights"] * 6 + ["weights", "weights", "weights", "weights"]
    ws = [weight(s, dt, c) for s, c in zip(shapes, cases)]
    for c in ("zero", "subnormal", "inf", "nan", "huge"):
        ws.append(weight((512, 256), dt, c))
    say("tensor scales", dt, len(ws))
    plan = TensorScalePlan(ws)
    got = plan.run().cpu()
    for i, w in enumerate(ws):
        assert (got[i:i + 1].view(torch.int32).item() & 0xFFFFFFFF) == oracle_scale(w, dt), i
    # re-run after an in-place update: the plan reads current values
    ws[0].mul_(2.0)
    ws[7].zero_()
    got2 = plan.run().cpu()
    assert bits(got2[0]) == oracle_scale(ws[0], dt)
    assert bits(got2[7]) == oracle_scale(ws[7], dt)


def test_tensor_scales_strided_and_batched_vs_reference():
    big = weight((600, 4160), "bf16")
    views = [big[:, 64:4160], big[100:300, :4096], big[:, 3:131]]  # aligned, row slice, misaligned
    stack = weight((8, 256, 512), "bf16")
    ws = views + [stack, stack[2]]
    plan = TensorScalePlan(ws)
    got = plan.run()
    for i, w in enumerate(ws):
        assert bits(got[i]) == bits(T.kv_scale(w.cpu())), i


@pytest.mark.parametrize("lead", [1, 2, 3, 4])
def test_tensor_scale_many_partials_any_slice_offset(lead):
    """A [70001, 4096] bf16 weight (one 8 KiB amax unit per row, so 70001
    partials: several rounds of the finishing kernel's 16-byte loads) after
    `lead` one-unit tensors, so its partials start at every 4-byte offset of a
    16-byte line.  The maximum sits in the first unit (read singly before the
    first boundary), a middle one, and the last (read singly after the last),
    then a NaN in the last unit."""
    say("tensor scale many partials", lead)
    rows = 70001
    big = torch.full((rows, 4096), 0.01, dtype=torch.bfloat16, device=DEV)
    ws = [weight((1, 64), "bf16") for _ in range(lead)] + [big]
    plan = TensorScalePlan(ws)
    for row, v in ((0, 3.5), (rows // 2, -2.25), (rows - 1, 1.75), (rows - 1, float("nan"))):
        big.fill_(0.01)
        big[row, 4095] = v
        want = oracle_scale(torch.tensor([[v, 0.01]], dtype=torch.bfloat16), "bf16")  # the same max |x|
        assert bits(plan.run()[lead]) == want, (lead, row, v)
        for i in range(lead):
            assert bits(plan.run()[i]) == oracle_scale(ws[i], "bf16"), (lead, i)


def test_tensor_scale_errors():
    with pytest.raises(RuntimeError):
        TensorScalePlan([torch.empty(0, 128, device=DEV, dtype=torch.bfloat16)])
    with pytest.raises(ValueError):
        TensorScalePlan([torch.ones(4, 8, device=DEV, dtype=torch.bfloat16),
                         torch.ones(4, 8, device=DEV, dtype=torch.float32)])


class _Attn(nn.Module):
    def __init__(self, hidden, kv):
        super().__init__()
        self.q_proj = nn.Linear(hidden, hidden, bias=False)
        self.k_proj = nn.Linear(hidden, kv, bias=False)
        self.v_proj = nn.Linear(hidden, kv, bias=False)
        self.o_proj = nn.Linear(hidden, hidden, bias=False)


class _Model(nn.Module):
    def __init__(self, layers=3, hidden=512, kv=128):
        super().__init__()
        self.layers = nn.ModuleList([nn.Module() for _ in range(layers)])
        for layer in self.layers:
            layer.self_attn = _Attn(hidden, kv)
        self.lm_head = nn.Linear(hidden, 1000, bias=False)


def _check_buffers(model, buf_dtype=torch.float32):
    n = 0
    for name, m in model.named_modules():
        short = name.rpartition(".")[2]
        buf = getattr(m, f"_lumenrl_fp8_kv_scale_{short}", None)
        if short in ("q_proj", "k_proj", "v_proj"):
            assert buf is not None and buf.dtype == buf_dtype and buf.dim() == 0, name
            assert buf.device == m.weight.device
            assert bits(buf.float()) == bits(T.kv_scale(m.weight.detach().cpu())), name
            n += 1
        elif isinstance(m, nn.Linear):
            assert not any(k.startswith("_lumenrl_fp8_kv_scale_") for k, _ in m.named_buffers()), name
    return n


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kv_quantizer_matches_reference(dtype):
    torch.manual_seed(1)
    model = _Model().to(DEV, dtype)
    kv = FP8KVCacheQuantizer(FP8Config(precision="fp8"))
    assert not kv.enabled
    kv.enable(model)
    assert kv.enabled and getattr(model, "_lumenrl_fp8_kv_cache_enabled") is True
    assert _check_buffers(model) == 9
    # an RL step updates the weights in place; recalibration follows them
    plan_before = dict(kv._groups)
    with torch.no_grad():
        for layer in model.layers:
            layer.self_attn.k_proj.weight.mul_(3.0)
        model.layers[1].self_attn.v_proj.weight[5, 7] = float("nan")
        model.layers[2].self_attn.q_proj.weight.zero_()
    kv.recalibrate_scales(model)
    assert {k: id(v) for k, v in kv._groups.items()} == {k: id(v) for k, v in plan_before.items()}
    assert _check_buffers(model) == 9
    assert np.isnan(model.layers[1].self_attn.v_proj._lumenrl_fp8_kv_scale_v_proj.item())


def test_kv_quantizer_existing_buffers_cpu_model_and_disabled(caplog):
    torch.manual_seed(2)
    model = _Model(layers=2, hidden=256, kv=64)  # CPU module: staged to the device
    for layer in model.layers:  # buffers that already exist are updated in place
        layer.self_attn.q_proj.register_buffer("_lumenrl_fp8_kv_scale_q_proj", torch.zeros(()))
    kept = model.layers[0].self_attn.q_proj._lumenrl_fp8_kv_scale_q_proj
    kv = FP8KVCacheQuantizer(FP8Config(precision="fp8"))
    kv.recalibrate_scales(model)
    assert model.layers[0].self_attn.q_proj._lumenrl_fp8_kv_scale_q_proj is kept
    assert _check_buffers(model) == 6
    model.double()  # float64 weights (and buffers): the reference's .to(float32) first
    kv.recalibrate_scales(model)
    assert _check_buffers(model, torch.float64) == 6
    off = FP8KVCacheQuantizer(FP8Config(precision="bf16"))
    fresh = _Model(layers=1, hidden=128, kv=128)
    off.enable(fresh)
    assert not off.enabled and not hasattr(fresh, "_lumenrl_fp8_kv_cache_enabled")
    assert not hasattr(fresh.layers[0].self_attn.q_proj, "_lumenrl_fp8_kv_scale_q_proj")
    with caplog.at_level(logging.WARNING):
        FP8KVCacheQuantizer(FP8Config(precision="fp8")).recalibrate_scales(nn.Sequential(nn.Linear(8, 8)))
    assert "no q_proj/k_proj/v_proj" in caplog.text
