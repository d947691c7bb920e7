"""quantize_tensor on float64 tensors, on an MI355X: the float64 kernel against
the CPU oracle and the reference's torch op sequence, bit for bit.

The reference evaluates every op of weight_quantizer.py:59-71 in float64 for a
float64 tensor (float64 scales) and rounds each quotient to float32 before the
e4m3 cast.  Cases: random and edge blocks (zero, +-inf, NaN, float64
subnormals, huge values, scales clamped to 2^-1022, float32 ties after the
float64 division), 1xB and 2-D blocks, strided and batched views, pow2 scales,
the drop-in WeightQuantizer on device and host tensors, and one 4096 x 4096
float64 weight in full.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref as T
from lumenrl_amd.quantization import FP8Config, WeightQuantizer, ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
RNG = np.random.default_rng(6464)


def say(*a):
    print(*a, flush=True)


def edge64(rows=16, cols=384):
    x = RNG.normal(0, 0.02, (rows, cols))
    x[0, :128] = 0
    x[0, 5] = -0.0
    x[1, 3], x[1, 4], x[1, 5] = np.inf, -np.inf, -0.0
    x[2, 7] = np.nan
    x[2, 200] = -np.nan
    x[3, :128] = 5e-324
    x[3, 1], x[3, 2] = -1e-310, 2.2e-308
    x[4, :128] = RNG.normal(0, 1e-300, 128)
    x[5, 9], x[5, 10] = 1.7e308, -1.7e308
    x[6, 130], x[6, 131] = np.nan, -np.inf
    x[7, :128] = 1.0625 + 2.0 ** -40
    x[7, 0], x[7, 1] = 448.0, 1.0625 - 2.0 ** -40
    x[8, :128] = -np.nan
    x[9, :128] = RNG.normal(0, 1, 128) * 1e-320
    x[10, 128:256] = RNG.normal(0, 1, 128) * 2.0 ** -1030
    x[11, 256:384] = RNG.uniform(-1, 1, 128) * 448.0 * 2.0 ** 900
    return x


def check(xd: torch.Tensor, blk, pow2):
    c, s = ops.fp8_block_quant(xd, blk, native_arith=True, pow2=pow2)
    torch.cuda.synchronize()
    assert s.dtype == torch.float64
    xh = xd.cpu().numpy()
    x3 = xh.reshape((-1,) + xh.shape[-2:])
    oc, osc = O.fp8_block_quant(x3, "f64", "native", blk, pow2)
    assert np.array_equal(c.view(torch.uint8).cpu().numpy().reshape(oc.shape), oc)
    assert np.array_equal(s.cpu().numpy().view(np.uint64).reshape(-1), osc.view(np.uint64).reshape(-1))


@pytest.mark.parametrize("pow2", [False, True])
@pytest.mark.parametrize("blk", [(1, 128), (1, 32), (1, 64), (1, 256), (1, 512), (1, 1024), (1, 2048), (1, 96),
                                 (1, 384), (1, 2), (1, 3), (1, 45), (1, 100), (1, 1000), (1, 3000), (1, 4096),
                                 (1, 5), (1, 7), (1, 8), (1, 16), (1, 33), (1, 65), (1, 127),
                                 (1, 6000), (1, 8192), (1, 12288), (1, 16384), (1, 16386),
                                 (128, 128), (3, 40), (64, 96)])
@pytest.mark.parametrize("data", ["weights", "edge"])
def test_f64_blocks_vs_oracle(data, blk, pow2):
    say("f64", data, blk, pow2)
    cols = blk[1] * 2 if blk[1] >= 512 else blk[1] * -(-384 // blk[1])
    if data == "weights":
        x = RNG.normal(0, 0.02, (200, cols))
        x.flat[RNG.integers(0, x.size, 80)] *= 150
    else:
        x = edge64(cols=cols)
    check(torch.from_numpy(x).to(DEV), blk, pow2)


@pytest.mark.parametrize("pow2", [False, True])
def test_f64_views_and_batches(pow2):
    base = torch.from_numpy(edge64(48, 640)).to(DEV)
    check(base[:, 64:448], (1, 128), pow2)          # row stride 640, offset view
    check(base[::3, :512], (1, 128), pow2)          # row stride 1920
    check(base[::2, :512], (1, 512), pow2)          # row stride 1280, one block per row
    check(base[:, 3:603], (1, 100), pow2)           # wide rows: row stride 640, 8 bytes off 16
    check(base[:, 1:46], (1, 45), pow2)             # odd width: the last chunk overlaps
    check(base[:40].reshape(5, 8, 640), (1, 64), pow2)  # batched matrices
    check(base.reshape(3, 16, 640)[:, :, :384], (8, 128), pow2)  # strided batch, 2-D blocks
    e = torch.empty(0, 128, dtype=torch.float64, device=DEV)
    c, s = ops.fp8_block_quant(e, (1, 128), native_arith=True)
    assert c.shape == (0, 128) and s.shape == (0, 1) and s.dtype == torch.float64


def test_f64_needs_float64_arithmetic():
    x = torch.zeros(4, 128, dtype=torch.float64, device=DEV)
    with pytest.raises(ValueError, match="float64 arithmetic"):
        ops.fp8_block_quant(x, (1, 128))
    with pytest.raises(TypeError):
        ops.quantize_mxfp8(x)


@pytest.mark.parametrize("pow2", [False, True])
def test_dropin_quantize_tensor_f64_vs_reference_ops(pow2):
    """WeightQuantizer.quantize_tensor on float64, device and host tensors, against
    the reference's torch ops on the CPU (non-NaN data: no loop-position rule)."""
    wq = WeightQuantizer(FP8Config(use_weight_pow2_scale=pow2))
    x = RNG.normal(0, 0.02, (6, 64, 512))
    x[0, 0, :128] = 0.0
    x[1, 3, 7] = np.inf
    x[2, 5, 128:256] = 1e-310
    x[3, 9, :128] = 1.0625 + 2.0 ** -40
    x[3, 9, 0] = 448.0
    t = torch.from_numpy(x)
    want_q, want_s = T.quantize_tensor(t, 128, pow2)
    for src in (t, t.to(DEV)):
        q, s = wq.quantize_tensor(src, 128)
        assert q.device == src.device and s.device == src.device
        assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float64
        assert tuple(s.shape) == (6, 64, 4)
        assert torch.equal(q.cpu().view(torch.uint8), want_q.view(torch.uint8))
        assert np.array_equal(s.cpu().numpy().view(np.uint64), want_s.numpy().view(np.uint64))
    if pow2:
        # a pow2 scale rounded down lets |x/s| reach 448*sqrt(2), which the
        # non-saturating e4m3fn cast turns into NaN in the reference too
        return
    # the reference's own unit contract (test_weight_quantizer.py:9-16), in float64
    w = torch.randn(64, 256, dtype=torch.float64, device=DEV)
    q, s = wq.quantize_tensor(w, 128)
    err = (wq.dequantize_tensor(q, s, 128).double() - w).abs().max().item()
    assert err < 0.25


def test_f64_full_4096x4096_vs_oracle():
    say("f64 4096x4096")
    x = RNG.normal(0, 0.02, (4096, 4096))
    x.flat[RNG.choice(x.size, x.size // 1000, replace=False)] = RNG.uniform(0.5, 4.0, x.size // 1000)
    xd = torch.from_numpy(x).to(DEV)
    c, s = ops.fp8_block_quant(xd, (1, 128), native_arith=True)
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(x, "f64", "native", (1, 128), False, nthreads=16)
    assert np.array_equal(s.cpu().numpy().view(np.uint64).reshape(-1), osc.view(np.uint64).reshape(-1))
    assert np.array_equal(c.view(torch.uint8).cpu().numpy(), oc[0])


def _e4m3_values() -> np.ndarray:
    """All positive finite float8_e4m3fn values, ascending."""
    codes = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn)
    return codes.float().numpy().astype(np.float64)


def _division_regimes(n_blocks: int, rng) -> dict:
    """float64 [n_blocks, 128] inputs whose quotients x/s stress the per-element division."""
    out = {}
    # (a) block amax anywhere in float64's range, elements 2^U(-80, 0) below it
    amax = 2.0 ** rng.uniform(-1000, 1000, (n_blocks, 1))
    x = amax * 2.0 ** rng.uniform(-80, 0, (n_blocks, 128)) * rng.choice([-1.0, 1.0], (n_blocks, 128))
    x[:, 0] = amax[:, 0]
    out["wide"] = x
    # (b) quotients planted on e4m3 ties and float32 rounding boundaries, then nudged
    v = _e4m3_values()
    ties = (v[:-1] + v[1:]) / 2
    s = 2.0 ** rng.uniform(-300, 300, (n_blocks, 1)) * rng.uniform(1, 2, (n_blocks, 1))
    t = rng.choice(np.concatenate([ties, v]), (n_blocks, 128))
    f32_half_ulp = np.ldexp(1.0, np.frexp(t)[1] - 25)
    nudge = rng.choice([-2, -1, 0, 1, 2], (n_blocks, 128)) * rng.choice([1e-16, 1e-12, 1.0], (n_blocks, 128))
    t = t + nudge * np.where(nudge == 0, 0, f32_half_ulp) * rng.uniform(0.5, 1.5, (n_blocks, 128))
    x = t * s * rng.choice([-1.0, 1.0], (n_blocks, 128))
    x[:, 0] = 448.0 * s[:, 0]
    out["ties"] = x
    # (c) tiny elements: near float64's underflow, subnormal, signed zeros, in blocks of any amax
    amax = 2.0 ** rng.uniform(-1000, 1000, (n_blocks, 1))
    x = 2.0 ** rng.uniform(-1074, -900, (n_blocks, 128)) * rng.choice([-1.0, 1.0], (n_blocks, 128))
    x[:, 1::9] = rng.choice([0.0, -0.0], x[:, 1::9].shape)
    x[:, 0] = amax[:, 0]
    out["tiny"] = x
    # (d) scales on both sides of 2^-900 (the kernel's Markstein / IEEE-division
    # cut per block): quotients on e4m3 values and ties and around the
    # subnormal edge (2^-13 ... 2^-9), nudged, and quotients below 2^-12
    s = 2.0 ** rng.uniform(-902, -898, (n_blocks, 1)) * rng.uniform(1, 2, (n_blocks, 1))
    edge = 2.0 ** rng.uniform(-13, -9, 4096)
    t = rng.choice(np.concatenate([ties, v, edge, edge * 2.0 ** -20]), (n_blocks, 128))
    nudge = rng.choice([-2, -1, 0, 1, 2], (n_blocks, 128)) * rng.choice([1e-16, 1e-12, 1.0], (n_blocks, 128))
    t = t + nudge * np.where(nudge == 0, 0, np.ldexp(1.0, np.frexp(t)[1] - 25))
    x = t * s * rng.choice([-1.0, 1.0], (n_blocks, 128))
    x[:, 0] = 448.0 * s[:, 0]
    out["guard"] = x
    return out


@pytest.mark.parametrize("pow2,blk", [(False, 128), (True, 128), (False, 32), (False, 64),
                                      (False, 256), (False, 512), (False, 8), (True, 16)])
def test_f64_row_kernel_division_sweep_vs_oracle(pow2, blk):
    """The 1xB float64 kernel (Markstein's correction in blocks with s >= 2^-900,
    the IEEE division below) against the oracle's IEEE division, bit for bit, on
    4 x 64 K rows of adversarial quotients.  The same rows read as 1x32, 1x64,
    1x256 and 1x512 blocks take the layouts whose scales reach each lane from
    other lanes (shuffles within a block's lanes, or readlane); 1x8 and 1x16
    blocks take the padded-group kernel (4 and 8 lanes per block)."""
    rng = np.random.default_rng(1717 + int(pow2))
    for name, x in _division_regimes(1 << 16, rng).items():
        say("f64 division sweep", name, pow2, blk)
        x = x.reshape(-1, blk)
        xd = torch.from_numpy(x).to(DEV)
        c, s = ops.fp8_block_quant(xd, (1, blk), native_arith=True, pow2=pow2)
        torch.cuda.synchronize()
        oc, osc = O.fp8_block_quant(x, "f64", "native", (1, blk), pow2, nthreads=16)
        got_s = s.cpu().numpy().view(np.uint64).reshape(-1)
        assert np.array_equal(got_s, osc.view(np.uint64).reshape(-1)), name
        got_c = c.view(torch.uint8).cpu().numpy()
        bad = np.flatnonzero(got_c.reshape(-1) != oc.reshape(-1))
        assert bad.size == 0, (name, bad[:8], x.reshape(-1)[bad[:8]])


def _grouped_inputs(shapes, rng):
    xs = []
    for shape in shapes:
        x = rng.normal(0.0, 0.02, shape) * 2.0 ** rng.uniform(-40, 40)
        flat = x.reshape(-1)
        flat[rng.integers(0, flat.size, 4)] = rng.uniform(0.5, 4.0, 4)
        xs.append(x)
    xs[0].reshape(-1)[:40] = 0.0
    xs[1].reshape(-1)[7] = np.inf
    xs[-1].reshape(-1)[-3] = np.nan
    return xs


@pytest.mark.parametrize("blk,pow2", [((1, 128), False), ((1, 128), True), ((1, 32), False),
                                      ((1, 512), False), ((128, 128), False), ((3, 40), False)])
def test_f64_grouped_plan_vs_oracle(blk, pow2):
    """float64 weights through one grouped launch (QuantPlan, float64 arithmetic):
    the 1xB row kernel for dense 1xB blocks, the generic kernel otherwise; run
    twice, the second time on new tensors (run(inputs=...))."""
    say("f64 grouped plan", blk, pow2)
    rng = np.random.default_rng(4242 + blk[1] + int(pow2))
    if blk[0] == 1:
        shapes = [(256, 1024), (1, 1024), (3, 64, 512), (640, 2048)]
    else:
        shapes = [(256, 384), (1, 200), (3, 130, 270), (640, 128)]
    plan = None
    for step in range(2):
        xs = _grouped_inputs(shapes, rng)
        ts = [torch.from_numpy(x).to(DEV) for x in xs]
        if plan is None:
            plan = ops.QuantPlan(ts, "fp8_block", blk, native_arith=True, use_pow2_scale=pow2)
            outs = plan.run()
        else:
            outs = plan.run(inputs=ts)
        torch.cuda.synchronize()
        for x, (c, s) in zip(xs, outs):
            assert s.dtype == torch.float64
            oc, osc = O.fp8_block_quant(x, "f64", "native", blk, pow2, nthreads=16)
            got_c = c.view(torch.uint8).cpu().numpy().reshape(oc.shape)
            got_s = s.cpu().numpy().view(np.uint64).reshape(osc.shape)
            assert np.array_equal(got_s, osc.view(np.uint64)), (blk, x.shape, step)
            assert np.array_equal(got_c, oc), (blk, x.shape, step)


def test_f64_plan_rules():
    x = torch.zeros(128, 256, dtype=torch.float64, device=DEV)
    with pytest.raises(ValueError, match="float64"):
        ops.QuantPlan([x], "fp8_block", (1, 128))
    with pytest.raises(ValueError, match="float64"):
        ops.QuantPlan([x], "mxfp8", (1, 32), native_arith=True)
