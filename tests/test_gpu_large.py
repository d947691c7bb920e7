"""Tensors past 2^31 elements on an MI355X: every kernel family, bit for bit.

A [65664, 32768] tensor holds 2,151,677,952 elements (4.3 GB in bf16): element
offsets pass 2^31 and byte offsets pass 2^32, where any 32-bit index arithmetic
would wrap.  The tensor is a random [384, 32768] base repeated 171 times, so
each output must equal the oracle's result on the base, repeated the same way;
the comparison runs on the device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
BASE_ROWS, COLS, TIMES = 384, 32768, 171
assert BASE_ROWS * TIMES * COLS > 1 << 31


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def base():
    rng = np.random.default_rng(31337)
    x = rng.normal(0.0, 0.02, (BASE_ROWS, COLS)).astype(np.float32)
    x.flat[rng.choice(x.size, 4096, replace=False)] = rng.uniform(0.5, 4.0, 4096)
    x[5, 256:384] = 0.0  # one zero block (and tile column) per repetition
    return torch.from_numpy(x).to(torch.bfloat16)  # CPU


def big_of(base: torch.Tensor, dtype=None) -> torch.Tensor:
    b = base.to(DEV)
    if dtype is not None:
        b = b.to(dtype)
    return b.repeat(TIMES, 1)


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def same(got: torch.Tensor, small_expected: np.ndarray | torch.Tensor, what: str) -> None:
    exp = torch.as_tensor(small_expected).to(DEV)
    exp = exp.reshape(-1, *got.shape[1:]) if got.dim() > 1 else exp
    reps = got.shape[0] // exp.shape[0]
    assert reps * exp.shape[0] == got.shape[0], what
    ints = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}
    g = got.view(ints[got.element_size()])
    e = exp.view(g.dtype)
    ok = torch.equal(g, e.repeat(reps, *([1] * (e.dim() - 1))))
    assert ok, what


@pytest.mark.parametrize("blk", [(128, 128), (1, 128)])
def test_fp8_blocks(base, blk):
    say("large fp8", blk)
    x = big_of(base)
    c, s = ops.fp8_block_quant(x, blk)
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(bf16_np(base), "bf16", "f32", blk, nthreads=16)
    same(c, oc.reshape(BASE_ROWS, COLS), f"codes {blk}")
    same(s, osc.view(np.int32).reshape(-1, s.shape[1]), f"scales {blk}")


@pytest.mark.parametrize("fmt", [8, 4])
def test_mx(base, fmt):
    say("large mx", fmt)
    x = big_of(base)
    c, s = (ops.quantize_mxfp8 if fmt == 8 else ops.quantize_mxfp4)(x)
    torch.cuda.synchronize()
    oc, osc = O.mx_quant(bf16_np(base), "bf16", fmt, nthreads=16)
    same(c, oc.reshape(BASE_ROWS, -1), f"mx{fmt} codes")
    same(s, osc.reshape(BASE_ROWS, -1), f"mx{fmt} scales")


@pytest.mark.parametrize("blk", [(1, 36), (1, 4096), (1, 32768)])
def test_fp8_row_widths(base, blk):
    """1x36 (padded lane groups, the last chunk overlapped) over the first 32760
    columns of each row, a strided view of 2.15 G elements; 1x4096 and 1x32768
    (whole rows: the wide-row kernel with one and with eight waves per block)
    over the whole tensor."""
    say("large fp8 rows", blk)
    x = big_of(base)
    cols = COLS - COLS % blk[1]
    c, s = ops.fp8_block_quant(x[:, :cols], blk)
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(np.ascontiguousarray(bf16_np(base)[:, :cols]), "bf16", "f32", blk, nthreads=16)
    same(c, oc.reshape(BASE_ROWS, cols), f"codes {blk}")
    same(s, osc.view(np.int32).reshape(-1, s.shape[1]), f"scales {blk}")


def test_mx_float32_input(base):
    say("large mx float32")
    x = big_of(base, torch.float32)
    c, s = ops.quantize_mxfp8(x)
    torch.cuda.synchronize()
    oc, osc = O.mx_quant(base.float().numpy(), "f32", 8, nthreads=16)
    same(c, oc.reshape(BASE_ROWS, -1), "mx8 f32 codes")
    same(s, osc.reshape(BASE_ROWS, -1), "mx8 f32 scales")


def test_fp8_dequant_to_bf16(base):
    say("large dequant")
    x = big_of(base)
    c, s = ops.fp8_block_quant(x, (1, 128), scale_dtype=torch.bfloat16)
    del x
    out = ops.fp8_block_dequant(c, s, (1, 128), torch.bfloat16)
    torch.cuda.synchronize()
    qc, qs = torch_ref.quantize_tensor(base.float(), 128)
    want = torch_ref.dequantize_tensor(qc, qs.to(torch.bfloat16), 128).to(torch.bfloat16)
    same(out, want.view(torch.int16), "dequant bf16")


def test_float64_rows(base):
    say("large float64 1x128")
    x = big_of(base, torch.float64)
    c, s = ops.fp8_block_quant(x, (1, 128), native_arith=True)
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(base.double().numpy(), "f64", "native", (1, 128), False, nthreads=16)
    same(c, oc.reshape(BASE_ROWS, COLS), "f64 codes")
    same(s, osc.view(np.int64).reshape(BASE_ROWS, -1), "f64 scales")


def test_unscaled_cast_copy_and_tensor_scale(base):
    say("large cast / copy / tensor scale")
    x = big_of(base)
    (q,) = ops.CastPlan([x]).run()
    dst = torch.empty_like(x)
    ops.CopyPlan([(dst, x)]).run()
    sc = ops.TensorScalePlan([x]).run()[0]
    torch.cuda.synchronize()
    same(q, base.to(torch.float8_e4m3fn).view(torch.uint8), "cast")
    assert torch.equal(dst.view(torch.int16), x.view(torch.int16))
    assert sc.cpu().view(torch.int32).item() == torch_ref.kv_scale(base).view(torch.int32).item()


def test_activation_fake_quant(base):
    say("large act_qdq")
    x = big_of(base)
    out = ops.act_qdq(x, 128)
    torch.cuda.synchronize()
    want = torch_ref.act_qdq(base, 128)
    same(out, want.view(torch.int32), "act_qdq")
