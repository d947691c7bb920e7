"""lrq_tensor_scale_grouped_static (the entry point that allocates nothing) on an
MI355X: called through the C ABI, its scales must equal those of
lrq_tensor_scale_grouped (caller workspace) bit for bit, on consecutive calls
that share the library's static workspace, the second with a smaller input."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from lumenrl_amd import _lib
from lumenrl_amd.quantization import TensorScalePlan

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
RNG = np.random.default_rng(7070)


def say(*a):
    print(*a, flush=True)


def weights(shapes, dtype, specials=True):
    out = []
    for i, shape in enumerate(shapes):
        x = (RNG.standard_normal(shape) * 0.02).astype(np.float32)
        x.flat[RNG.integers(0, x.size)] = RNG.choice([-1.0, 1.0]) * RNG.uniform(0.5, 4.0)
        if specials and i % 5 == 1:
            x[:] = 0.0
        elif specials and i % 5 == 2:
            x.flat[x.size // 3] = -np.inf
        elif specials and i % 5 == 3:
            x.flat[x.size - 5] = np.nan
        elif specials and i % 5 == 4:
            x[:] = 1e-40
        out.append(torch.from_numpy(x).to(dtype).to(DEV))
    return out


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int32).numpy().view(np.uint32)


def both(ws):
    """Scales from the static-workspace entry point, then from the caller-workspace one."""
    plan = TensorScalePlan(ws)
    assert plan._launch.workspace_bytes() <= _lib.STATIC_WORKSPACE_BYTES
    plan.scales.fill_(-1.0)
    static = bits(plan.run_static())
    plan.scales.fill_(-2.0)
    plan.workspace.fill_(0xA5)
    ref = bits(plan.run())
    torch.cuda.synchronize()
    return static, ref, plan


def test_static_matches_caller_workspace_on_consecutive_calls():
    # call 1: the q/k/v projections of 4 Qwen3-8B layers, with zero/inf/NaN/tiny tensors
    big = weights([(4096, 4096), (1024, 4096), (1024, 4096)] * 4, torch.bfloat16)
    say("[no_alloc] call 1: 12 bf16 tensors")
    s1, r1, p1 = both(big)
    assert np.array_equal(s1, r1)
    units1 = p1.units
    # the oracle agrees too (the checker, on a few tensors)
    for i in (0, 1, 2, 3, 4):
        x = big[i].cpu().view(torch.int16).numpy().view(np.uint16)
        assert int(s1[i]) == int(O.tensor_scale(x, "bf16"))
    del big, p1
    # call 2: fewer, smaller tensors; the static workspace still holds call 1's partials
    small = weights([(256, 512), (128, 1024), (64, 4096)], torch.bfloat16)
    say("[no_alloc] call 2: 3 small bf16 tensors")
    s2, r2, p2 = both(small)
    assert p2.units < units1
    assert np.array_equal(s2, r2)
    # call 3: float32 and strided views through the same static workspace
    base = weights([(512, 1024)], torch.float32, specials=False)[0]
    f32 = [base[:, :768], base[::2], weights([(96, 640)], torch.float32)[0]]
    say("[no_alloc] call 3: float32 views")
    s3, r3, _ = both(f32)
    assert np.array_equal(s3, r3)


def test_static_rejects_oversized_table_before_device_work():
    L = _lib.lib()
    fake = 1 << 20
    t = (_lib.LrqTensor * 1)()
    rows, cols = 1 << 20, 8192  # 8 G bf16 elements: more partials than the static workspace holds
    t[0].in_, t[0].codes, t[0].scales = fake, None, fake
    t[0].batch, t[0].rows, t[0].cols, t[0].ld, t[0].batch_stride = 1, rows, cols, cols, rows * cols
    need = L.lrq_group_table_bytes(_lib.FMT_TENSOR_SCALE, t, 1, _lib.DTYPE_BF16, 1, 1, 0)
    assert need > 0
    host = (ctypes.c_uint8 * need)()
    assert L.lrq_group_pack(_lib.FMT_TENSOR_SCALE, t, 1, _lib.DTYPE_BF16, 1, 1, 0, host, need) == 0
    assert L.lrq_group_workspace_bytes(host) > _lib.STATIC_WORKSPACE_BYTES
    rc = L.lrq_tensor_scale_grouped_static(host, ctypes.c_void_p(fake), None)
    assert rc == _lib.ERR_CAPACITY and "static workspace" in _lib.last_error()


def test_static_entry_point_under_graph_capture():
    """The use case the entry point exists for: a HIP graph that captures it.
    The static workspace's address is looked up when the plan's table is set up
    (lrq_group_build_map), so the capture records only the two launches; the
    graph is replayed after eager changes to the weights, each replay checked
    bit for bit against the caller-workspace entry point run eagerly."""
    ws = weights([(1024, 4096), (256, 4096), (512, 2048)], torch.bfloat16, specials=False)
    plan = TensorScalePlan(ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    say("[no_alloc] capture run_static")
    with torch.cuda.graph(graph):  # no eager run_static before: capture is its first call here
        plan.run_static()
    for rep in range(3):
        for i, w in enumerate(ws):
            w.copy_(torch.from_numpy((RNG.standard_normal(tuple(w.shape)) * 0.01 * (rep + i + 1))
                                     .astype(np.float32)).to(w.dtype).to(DEV))
        if rep == 1:
            ws[2][7, 9] = float("nan")
        plan.scales.fill_(-1.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = bits(plan.scales).copy()
        plan.scales.fill_(-2.0)
        ref = bits(plan.run())
        torch.cuda.synchronize()
        say("[no_alloc] replay", rep)
        assert np.array_equal(got, ref), rep
