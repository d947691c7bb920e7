"""W8A8 rollout path on an MI355X: the activation fake-quant kernel against the
CPU oracle and torch fixtures (bit-exact), and the ``_FP8W8A8Linear`` /
``FP8RolloutQuantizer`` mirror against the reference's op sequence
(lumenrl/quantization/fp8_rollout.py:25-149)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from conftest import load_golden
from oracle import oracle as O
from oracle import torch_ref as T
from lumenrl_amd.quantization import FP8Config, FP8RolloutQuantizer, act_qdq
from lumenrl_amd.quantization.fp8_rollout import _FP8W8A8Linear
from lumenrl_amd.quantization.weight_quantizer import WeightQuantizer

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
RNG = np.random.default_rng(77)


def say(*a):
    print(*a, flush=True)


def to_dev(x: np.ndarray, dt: str) -> torch.Tensor:
    """Device tensor of dtype ``dt`` from float32 values (bf16/f16 round to nearest)."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DT[dt]).to(DEV)


def oracle_in(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def f32bits(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu().contiguous().numpy()
    return np.ascontiguousarray(t, np.float32).view(np.uint32)


def acts(shape, scale=0.7) -> np.ndarray:
    """Heavy-tailed activations with a few outlier channels (LLM hidden states)."""
    x = (RNG.standard_t(3, shape) * scale).astype(np.float32)
    cols = RNG.choice(shape[-1], max(1, shape[-1] // 256), replace=False)
    x[..., cols] *= 40.0
    return x


def plant_edges(x: np.ndarray, blk: int) -> np.ndarray:
    x = x.copy()
    x[0, :blk] = 0.0
    x[0, 1] = -0.0
    x[1, 3], x[1, 4] = np.inf, -np.inf
    x[2, blk + 2] = np.nan
    x[3, :blk] = np.float32(1e-40)
    x[4, :blk] = RNG.normal(0, 1e-30, blk)
    x[5, 9], x[5, 10] = 3.3e38, -3.3e38
    x[6, blk - 1] = -np.nan
    return x


@pytest.mark.parametrize("name", ["act_bf16.npz", "act_bf16_b32_pow2.npz", "act_f32_pow2.npz"])
def test_act_golden(name):
    g = load_golden(name)
    x = g["x"]
    if x.dtype == np.float32:
        t = torch.from_numpy(x).to(DEV)
    else:
        t = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    say("act golden", name)
    out = act_qdq(t, int(g["block"][0]), pow2=bool(g["pow2"][0]))
    assert np.array_equal(f32bits(out), g["out"].view(np.uint32))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("blk", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("pow2", [False, True])
def test_act_vs_oracle(dt, blk, pow2):
    x = plant_edges(acts((300, 1024)), blk)
    t = to_dev(x, dt)
    say("act", dt, blk, pow2, tuple(t.shape))
    out = act_qdq(t, blk, pow2=pow2)
    want = O.act_qdq(oracle_in(t), dt, blk, pow2)
    assert out.dtype == torch.float32 and tuple(out.shape) == (300, 1024)
    assert np.array_equal(f32bits(out), want.view(np.uint32))


@pytest.mark.parametrize("blk", [1, 16, 40, 96, 100, 200, 512, 1024, 3000, 4096])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_act_other_widths_vs_oracle(dt, blk):
    """Block widths the vector kernels do not take: whole 16-byte chunks on
    padded lane groups (up to 32 chunks) or one wave per block (up to 512),
    other widths walked twice by one wave per block; dense, as a strided view
    and as a view one element off its 16-byte alignment, with
    NaN/inf/zero/subnormal blocks."""
    cols = blk * max(1, 3000 // blk) if blk < 3000 else 2 * blk
    x = plant_edges(acts((40, cols + 8)), min(blk, 64))
    t = to_dev(x, dt)
    for pow2 in (False, True):
        for v in (t[:, :cols].contiguous(), t[:, 8:], t[:, 1:cols + 1]):
            say("act other widths", dt, blk, pow2, tuple(v.shape), v.stride())
            out = act_qdq(v, blk, pow2=pow2)
            want = O.act_qdq(oracle_in(v), dt, blk, pow2)
            assert np.array_equal(f32bits(out), want.view(np.uint32)), (dt, blk, pow2, v.stride())


def test_act_vs_torch_reference_bf16():
    x = acts((64, 2048))
    t = to_dev(x, "bf16")
    want = T.act_qdq(t.cpu(), 128, False)
    assert np.array_equal(f32bits(act_qdq(t, 128)), f32bits(want))


def test_act_3d_and_strided():
    x = acts((4, 33, 512))
    t = to_dev(x, "bf16")
    out = act_qdq(t, 128)
    want = O.act_qdq(oracle_in(t).reshape(-1, 512), "bf16", 128, False)
    assert tuple(out.shape) == (132, 512)
    assert np.array_equal(f32bits(out), want.view(np.uint32))
    big = to_dev(acts((96, 1536)), "f32")
    view = big[:, 256:1280]  # row stride 1536, no copy
    out = act_qdq(view, 64, pow2=True)
    want = O.act_qdq(oracle_in(view), "f32", 64, True)
    assert np.array_equal(f32bits(out), want.view(np.uint32))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("ld,c0", [(1544, 8), (1028, 4), (1032, 0)])
def test_act_strided_16bit(dt, ld, c0):
    """Row strides with and without 16-byte row alignment (the 8-per-lane and
    4-per-lane kernels), and an unaligned start."""
    big = to_dev(plant_edges(acts((97, ld)), 128), dt)
    view = big[:, c0:c0 + 1024]
    say("act strided", dt, ld, c0)
    for blk in (32, 256):
        out = act_qdq(view, blk)
        want = O.act_qdq(oracle_in(view), dt, blk, False)
        assert np.array_equal(f32bits(out), want.view(np.uint32))


def test_act_prefill_size():
    """A Qwen3-8B prefill chunk: 8192 tokens x 4096 hidden."""
    t = to_dev(acts((8192, 4096)), "bf16")
    say("act prefill", tuple(t.shape))
    out = act_qdq(t, 128)
    want = O.act_qdq(oracle_in(t), "bf16", 128, False)
    assert np.array_equal(f32bits(out), want.view(np.uint32))


def test_act_empty_and_errors():
    assert act_qdq(torch.empty(0, 256, device=DEV, dtype=torch.bfloat16)).shape == (0, 256)
    with pytest.raises(ValueError, match="multiple of the block"):
        act_qdq(torch.ones(4, 200, device=DEV, dtype=torch.bfloat16), 128)
    with pytest.raises(ValueError, match="activation block must be"):
        act_qdq(torch.ones(4, 256, device=DEV, dtype=torch.bfloat16), 0)
    with pytest.raises(ValueError):
        act_qdq(torch.ones(4, 256, dtype=torch.bfloat16))


# ---------------------------------------------------------------- module
def reference_forward(lin: nn.Linear, x: torch.Tensor, cfg: FP8Config) -> tuple:
    """fp8_rollout.py:45-78 with the CPU torch restatement; GEMM on the device."""
    q, s = T.quantize_tensor(lin.weight.data.cpu().float(), 128, cfg.use_weight_pow2_scale)
    s16 = s.to(torch.bfloat16)
    x_dq = T.act_qdq(x.cpu(), 128, cfg.use_activation_pow2_scale)
    w_dq = T.dequantize_tensor(q, s16, 128).float()
    b = lin.bias.data.float().to(DEV) if lin.bias is not None else None
    y = F.linear(x_dq.to(DEV), w_dq.to(DEV), b)
    return q, s16, y.to(x.dtype)  # [prod(leading), out_features] (fp8_rollout.py:56-78)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("pow2", [False, True])
@pytest.mark.parametrize("bias", [True, False])
def test_fp8_linear_matches_reference(dtype, pow2, bias):
    torch.manual_seed(3)
    lin = nn.Linear(512, 384, bias=bias).to(DEV, dtype)
    cfg = FP8Config(precision="fp8", use_weight_pow2_scale=pow2, use_activation_pow2_scale=pow2)
    mod = _FP8W8A8Linear(lin, WeightQuantizer(cfg), cfg, 128)
    x = torch.from_numpy(acts((3, 17, 512))).to(DEV, dtype)
    q, s16, y_ref = reference_forward(lin, x, cfg)
    assert mod.weight_fp8.dtype == torch.float8_e4m3fn and mod.weight_scale.dtype == torch.bfloat16
    assert np.array_equal(mod.weight_fp8.cpu().view(torch.uint8).numpy(), q.view(torch.uint8).numpy())
    assert torch.equal(mod.weight_scale.cpu().view(torch.int16), s16.view(torch.int16))
    with torch.no_grad():
        y = mod(x)
    assert y.dtype == dtype and y.shape == (51, 384)  # the reference's flattened shape
    assert torch.equal(y, y_ref)
    keep = _FP8W8A8Linear(lin, WeightQuantizer(cfg), cfg, 128, keep_leading_dims=True)
    with torch.no_grad():
        yk = keep(x)
    assert yk.shape == (3, 17, 384) and torch.equal(yk.reshape(51, 384), y_ref)


def test_fp8_linear_any_activation_block():
    """activation_block_size = 96 (any divisor of in_features, fp8_rollout.py:36-44)
    against the reference's op sequence."""
    torch.manual_seed(4)
    lin = nn.Linear(384, 200).to(DEV, torch.bfloat16)
    cfg = FP8Config(precision="fp8")
    mod = _FP8W8A8Linear(lin, WeightQuantizer(cfg), cfg, 96)
    x = torch.from_numpy(acts((2, 9, 384))).to(DEV, torch.bfloat16)
    q, s = T.quantize_tensor(lin.weight.data.cpu().float(), 96, False)
    s16 = s.to(torch.bfloat16)
    x_dq = T.act_qdq(x.cpu(), 96, False)
    w_dq = T.dequantize_tensor(q, s16, 96).float()
    y_ref = F.linear(x_dq.to(DEV), w_dq.to(DEV), lin.bias.data.float()).to(torch.bfloat16)
    with torch.no_grad():
        y = mod(x)
    assert np.array_equal(mod.weight_fp8.cpu().view(torch.uint8).numpy(), q.view(torch.uint8).numpy())
    assert torch.equal(y, y_ref)


def test_fp8_linear_float64_activations():
    """x.to(float32) first, everything in float32, then y.to(float64) (fp8_rollout.py:53-78)."""
    torch.manual_seed(5)
    lin = nn.Linear(256, 128).to(DEV)
    cfg = FP8Config(precision="fp8")
    mod = _FP8W8A8Linear(lin, WeightQuantizer(cfg), cfg, 128)
    x = torch.from_numpy(acts((2, 7, 256)).astype(np.float64) * (1 + 1e-9)).to(DEV)
    with torch.no_grad():
        y = mod(x)
    _, _, y_ref = reference_forward(lin, x.float(), cfg)
    assert y.dtype == torch.float64 and y.shape == (14, 128)
    assert torch.equal(y, y_ref.double())


def test_fp8_linear_errors_and_cpu_module():
    cfg = FP8Config(precision="fp8")
    with pytest.raises(ValueError, match="must be divisible by activation_block_size"):
        _FP8W8A8Linear(nn.Linear(200, 64), WeightQuantizer(cfg), cfg, 128)
    lin = nn.Linear(256, 64)  # CPU module: buffers come back on the CPU
    mod = _FP8W8A8Linear(lin, WeightQuantizer(cfg), cfg, 128)
    assert mod.weight_fp8.device.type == "cpu"
    with pytest.raises(RuntimeError, match="not divisible by 128"):
        mod(torch.ones(2, 200))
    x = torch.randn(5, 256)
    y = mod(x)
    assert y.device.type == "cpu" and y.shape == (5, 64)
    _, _, y_ref = reference_forward(lin, x, cfg)
    assert torch.equal(y, y_ref.cpu())


def test_rollout_quantizer_patch_and_restore():
    torch.manual_seed(4)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.up = nn.Linear(256, 512)
            self.down = nn.Linear(512, 256)

        def forward(self, h):
            return h + self.down(F.silu(self.up(h)))

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.inp = nn.Linear(256, 256)
            self.blocks = nn.ModuleList([Block(), Block()])
            self.odd = nn.Linear(256, 100)
            self.head = nn.Linear(100, 64)  # in_features % 128 != 0: left as is

        def forward(self, x):
            h = self.inp(x)
            for b in self.blocks:
                h = b(h)
            return self.head(self.odd(h))

    net = Net().to(DEV, torch.bfloat16)
    x = torch.randn(4, 9, 256, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        y0 = net(x)
    off = FP8RolloutQuantizer(FP8Config(precision="bf16"))
    off.quantize_model(net)
    assert isinstance(net.inp, nn.Linear)
    cfg = FP8Config(precision="fp8", num_first_layers_in_bf16=1, num_last_layers_in_bf16=1)
    rq = FP8RolloutQuantizer(cfg, keep_leading_dims=True)  # this model feeds 3-D activations
    assert rq.should_skip_layer("x", 0, 7) and rq.should_skip_layer("x", 6, 7)
    assert not rq.should_skip_layer("x", 1, 7) and not rq.should_skip_layer("x", 5, 7)
    originals = dict(net.named_modules())
    rq.quantize_model(net)
    kinds = {n: type(m).__name__ for n, m in net.named_modules() if n}
    # linears in module order: inp, blocks.0.up, blocks.0.down, blocks.1.up,
    # blocks.1.down, odd, head -> first and last stay, head's in_features fail anyway
    assert kinds["inp"] == "Linear" and kinds["head"] == "Linear"
    for n in ("blocks.0.up", "blocks.0.down", "blocks.1.up", "blocks.1.down", "odd"):
        assert kinds[n] == "_FP8W8A8Linear", n
    with torch.no_grad():
        y1 = net(x)
    assert y1.dtype == torch.bfloat16 and torch.isfinite(y1).all()
    rel = (y1.float() - y0.float()).norm() / y0.float().norm()
    assert float(rel) < 0.1
    rq.restore_model(net)
    for n in ("blocks.0.up", "odd"):
        assert net.get_submodule(n) is originals[n]
    with torch.no_grad():
        assert torch.equal(net(x), y0)


def test_quantize_model_skips_a_failing_layer_and_patches_the_rest(caplog):
    """One weight that cannot be quantized (a meta tensor) makes the grouped
    batch raise; quantize_model then quantizes layer by layer, so that layer is
    skipped with the reference's warning (fp8_rollout.py:130-136) and every
    other eligible linear is patched with the reference's buffers."""
    torch.manual_seed(11)
    net = nn.Sequential(nn.Linear(256, 384), nn.Linear(384, 256), nn.Linear(256, 512)).to(DEV, torch.bfloat16)
    net[1] = nn.Linear(384, 256, device="meta", dtype=torch.bfloat16)
    rq = FP8RolloutQuantizer(FP8Config(precision="fp8"))
    with caplog.at_level("WARNING"):
        rq.quantize_model(net)
    assert any("Failed to FP8-wrap 1" in r.getMessage() for r in caplog.records)
    assert isinstance(net[1], nn.Linear)
    for i in (0, 2):
        m = net[i]
        assert isinstance(m, _FP8W8A8Linear), i
        q, s = T.quantize_tensor(rq._originals[str(i)].weight.data.cpu().float(), 128, False)
        assert torch.equal(m.weight_fp8.cpu().view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(m.weight_scale.cpu().view(torch.int16), s.to(torch.bfloat16).view(torch.int16))


def test_quantize_model_grouped_weights_equal_the_reference_ops():
    """quantize_model's grouped launches give every patched module the buffers of
    the reference's per-layer quantize_tensor (float32 upcast, bf16 scales), for
    bf16, fp16, fp32 and float64 weights and a CPU-resident linear."""
    torch.manual_seed(6)
    shapes = [(384, 256), (128, 512), (1024, 256), (256, 1024), (640, 384)] * 5
    net = nn.Sequential(*[nn.Linear(i, o, bias=(k % 2 == 0)) for k, (o, i) in enumerate(shapes)])
    net = net.to(DEV, torch.bfloat16)
    net[3].to(torch.float16)
    net[7].to(torch.float32)
    net[11].to(torch.float64)
    cpu_lin = nn.Linear(256, 128)
    net.append(cpu_lin)
    want = {}
    for name, m in net.named_modules():
        if isinstance(m, nn.Linear):
            q, s = T.quantize_tensor(m.weight.data.cpu().float(), 128, False)
            want[name] = (q.view(torch.uint8), s.to(torch.bfloat16).view(torch.int16))
    rq = FP8RolloutQuantizer(FP8Config(precision="fp8"))
    rq.quantize_model(net)
    patched = {n: m for n, m in net.named_modules() if isinstance(m, _FP8W8A8Linear)}
    assert len(patched) == len(want)
    for name, m in patched.items():
        assert torch.equal(m.weight_fp8.cpu().view(torch.uint8), want[name][0]), name
        assert torch.equal(m.weight_scale.cpu().view(torch.int16), want[name][1]), name
    assert patched[str(len(shapes))].weight_fp8.device.type == "cpu"
    x = torch.randn(9, 256, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        y = net[0](x)
    assert y.shape == (9, 384)
