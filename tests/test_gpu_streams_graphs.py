"""Execution properties callers rely on, on an MI355X.

- Stream ordering: launches go to the caller's current stream.
- HIP graph replay: grouped launches captured once, replayed after the inputs
  change, each replay bit-exact with the oracle.
- A seeded sweep of random shapes, strides, blocks and dtypes through every
  kernel family, compared with the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from lumenrl_amd.quantization import QuantPlan, TensorScalePlan, act_qdq, ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def say(*a):
    print(*a, flush=True)


def host_in(t: torch.Tensor, dt: str) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.numpy() if dt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def f32bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


def _layer(gen):
    shapes = [(512, 1024), (128, 1024), (1024, 512)]
    return [(torch.randn(s, generator=gen, device=DEV) * 0.02).to(torch.bfloat16) for s in shapes]


def _check_fp8_tiles(ws, outs):
    for w, (c, s) in zip(ws, outs):
        oc, osc = O.fp8_block_quant(host_in(w, "bf16"), "bf16", "f32", (128, 128))
        assert np.array_equal(u8(c), oc[0])
        assert np.array_equal(f32bits(s), osc[0].view(np.uint32))


def test_plan_runs_on_the_current_stream():
    gen = torch.Generator(device=DEV).manual_seed(3)
    ws = _layer(gen)
    plan = QuantPlan(ws, "fp8_block", (128, 128))
    side = torch.cuda.Stream()
    main = torch.cuda.current_stream()
    for w in ws:  # new values written on the main stream ...
        w.normal_(0.0, 0.05, generator=gen)
    side.wait_stream(main)
    with torch.cuda.stream(side):  # ... quantized on the side stream after them
        outs = plan.run()
    main.wait_stream(side)
    torch.cuda.synchronize()
    _check_fp8_tiles(ws, outs)


@pytest.mark.parametrize("split", [False, True])
def test_graph_replay_of_grouped_launches(split, monkeypatch):
    """Captured grouped launches (one table, or a plan split into a launch per
    tensor) replay against the eager result after the inputs change."""
    gen = torch.Generator(device=DEV).manual_seed(4)
    ws = _layer(gen)
    if split:
        monkeypatch.setattr(ops, "GROUP_LAUNCH_BYTES", 64 << 10)
    plan = QuantPlan(ws, "fp8_block", (128, 128))
    assert len(plan._launch.parts) == (len(ws) if split else 1)
    scales = TensorScalePlan(ws)
    xa = (torch.randn(256, 1024, generator=gen, device=DEV)).to(torch.bfloat16)
    act_out = torch.empty(256, 1024, dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        plan.run()
        scales.run()
        act_qdq(xa, 128, out=act_out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
        scales.run()
        act_qdq(xa, 128, out=act_out)
    for rep in range(3):
        for w in ws:  # eager work between replays
            w.copy_((torch.randn(w.shape, generator=gen, device=DEV) * (0.01 * (rep + 1))).to(w.dtype))
        xa.copy_(torch.randn(xa.shape, generator=gen, device=DEV).to(xa.dtype))
        ws[1][5, 7] = float("inf") if rep == 1 else 0.25
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say("graph replay", rep)
        _check_fp8_tiles(ws, plan.outputs)
        got = f32bits(scales.scales)
        for i, w in enumerate(ws):
            assert got[i] == O.tensor_scale(host_in(w, "bf16"), "bf16"), (rep, i)
        assert np.array_equal(f32bits(act_out), O.act_qdq(host_in(xa, "bf16"), "bf16", 128).view(np.uint32))


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused capture records nothing
def test_plan_built_under_capture_is_refused():
    """A plan's table upload inside a capture would replay from a host buffer
    the plan frees; building one there raises before any device work."""
    w = torch.zeros(256, 256, dtype=torch.bfloat16, device=DEV)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="before HIP graph capture"):
        with torch.cuda.graph(graph):
            QuantPlan([w], "fp8_block", (128, 128))
    torch.cuda.synchronize()
    plan = QuantPlan([w], "fp8_block", (128, 128))  # outside a capture it builds and runs
    plan.run()
    torch.cuda.synchronize()
    assert torch.all(plan.outputs[0][0].view(torch.uint8) == 0)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_rebind_after_capture_is_refused():
    """A captured run keeps the plan's descriptor table (the graph holds its
    address).  Moving an input to other storage afterwards raises instead of
    replacing and freeing that table; the stale graph is never replayed on the
    moved input, and it still replays correctly on the planned inputs.  The
    same holds for a transfer bucket's pass-through copy table."""
    from lumenrl_amd.quantization import QuantizedBucketWriter

    gen = torch.Generator(device=DEV).manual_seed(8)
    ws = _layer(gen)
    plan = QuantPlan(ws, "fp8_block", (128, 128))
    norm = torch.ones(1024, dtype=torch.bfloat16, device=DEV)
    named = [("l.q_proj.weight", ws[0]), ("l.input_layernorm.weight", norm)]
    writer = QuantizedBucketWriter(named, bucket_bytes=4 << 20, fmt="fp8_block")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        plan.run()
        for b in writer:
            b.fill()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
        for b in writer:
            b.fill()
    table = plan._launch
    moved = ws[1].clone()  # the same values in other storage
    with pytest.raises(RuntimeError, match="captured into a HIP graph"):
        plan.run([ws[0], moved, ws[2]])
    assert plan._launch is table and plan.inputs[1] is ws[1]
    norm.data = torch.full((1024,), 0.5, dtype=torch.bfloat16, device=DEV)  # a p.data swap
    bucket = next(iter(writer))
    with pytest.raises(RuntimeError, match="captured into a HIP graph"):
        bucket.fill()
    torch.cuda.synchronize()
    for w in ws:
        w.copy_((torch.randn(w.shape, generator=gen, device=DEV) * 0.03).to(w.dtype))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    _check_fp8_tiles(ws, plan.outputs)


def test_random_shape_sweep():
    """Seeded random shapes, strides, dtypes and blocks through every kernel family."""
    rng = np.random.default_rng(2026)
    for case in range(40):
        dt = ["bf16", "f16", "f32"][rng.integers(0, 3)]
        rows = int(rng.integers(1, 300))
        cols = int(rng.choice([32, 64, 96, 128, 160, 256, 384, 520, 1024]))
        pad = int(rng.choice([0, 0, 4, 8, 64]))
        x = torch.from_numpy((rng.standard_t(5, (rows, cols + pad)) * 0.05).astype(np.float32))
        if rng.random() < 0.2:
            x[int(rng.integers(0, rows)), int(rng.integers(0, cols))] = float(rng.choice([np.inf, -np.inf, np.nan]))
        xd = x.to(DT[dt]).to(DEV)[:, :cols]
        xh = host_in(xd, dt)
        kind = rng.integers(0, 4)
        say("sweep", case, dt, rows, cols, pad, int(kind))
        if kind == 0:
            blk = [(128, 128), (1, 128), (1, 32), (64, 96), (3, 40)][rng.integers(0, 5)]
            native = bool(rng.integers(0, 2)) and dt != "f32"
            pow2 = bool(rng.integers(0, 2))
            c, s = ops.fp8_block_quant(xd, blk, native_arith=native, pow2=pow2)
            oc, osc = O.fp8_block_quant(xh, dt, "native" if native else "f32", blk, pow2)
            assert np.array_equal(u8(c), oc[0]), case
            sh = s.detach().cpu().contiguous()
            sb = sh.numpy().view(np.uint32) if sh.dtype == torch.float32 else \
                sh.view(torch.int16).numpy().view(np.uint16)
            ob = osc[0].reshape(-1)
            ob = ob.view(np.uint32) if ob.dtype == np.float32 else ob
            assert np.array_equal(sb.reshape(-1), ob), case
        elif kind == 1:
            if cols % 32:
                continue
            fmt = int(rng.choice([8, 4]))
            c, s = ops.quantize_mxfp8(xd) if fmt == 8 else ops.quantize_mxfp4(xd)
            oc, osc = O.mx_quant(xh, dt, fmt)
            assert np.array_equal(u8(c), oc) and np.array_equal(u8(s), osc), case
        elif kind == 2:
            blk = int(rng.choice([32, 64, 128, 256]))
            if cols % blk:
                continue
            pow2 = bool(rng.integers(0, 2))
            out = act_qdq(xd, blk, pow2=pow2)
            assert np.array_equal(f32bits(out), O.act_qdq(xh, dt, blk, pow2).view(np.uint32)), case
        else:
            sc = TensorScalePlan([xd]).run()
            assert f32bits(sc)[0] == O.tensor_scale(xh, dt), case
