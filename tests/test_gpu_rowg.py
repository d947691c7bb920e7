"""1xB blocks of widths that are not 32..512 powers of two, on an MI355X.

``quantize_tensor(tensor, block_size=B)`` takes any B dividing the last dim
(weight_quantizer.py:40-77).  Widths 8..512 run on the row kernel with 1- or
2-lane groups (8, 16) or ceil(B/8) chunks in lane groups padded to the next
power of two (the last lanes of each group idle); when 8 does not divide B
(12, 36, 100, 500) the last chunk overlaps its neighbour.  1024 and 2048 run on
the row kernel with a block spanning 2 or 4 wave instructions; other widths up
to 65536 on the wide-row kernel: one wave per block up to 4096 (640, 1000,
1032, 1536, 3001, 4096), two or four up to 16384 (4104, 9999, 12288, 16384),
a work-group of 8 or 16 waves beyond (16392, 18944, 29568, 65536); the rest
(5, 7, 65544) on the generic kernel.  Every code and scale bit is compared
with the oracle, and the drop-in with the reference's torch op sequence.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref as TR
from lumenrl_amd.quantization import FP8Config, WeightQuantizer, ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
WIDTHS = [40, 48, 96, 120, 200, 248, 504, 8, 16, 24, 36, 1024, 2048, 1536,
          640, 1032, 4096, 4104, 12288, 16384, 16392, 12, 100, 500, 1000, 3001, 9999, 5, 7,
          3072, 4090, 6144, 7000, 8192, 18944, 29568, 65536, 65544]
# (rows, blocks per row, row pitch padding, pow2, bf16 scales when arith is f32)
CASES = [(1, 1, 0, False, False), (37, 3, 0, True, False), (200, 5, 16, False, True),
         (513, 2, 0, False, False), (64, 11, 8, True, False)]
CASES_WIDE = [(1, 1, 0, False, False), (37, 3, 0, True, False), (90, 1, 16, False, True),
              (129, 2, 0, False, False), (16, 5, 8, True, False)]


def host(t: torch.Tensor, dt: str) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.numpy() if dt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def weights(rng, rows, cols, ld, dt):
    x = (rng.standard_t(4, (rows, ld)) * 10.0 ** rng.uniform(-3, 0)).astype(np.float32)
    for _ in range(3):
        x[rng.integers(0, rows), rng.integers(0, cols)] = rng.choice([np.inf, -np.inf, np.nan, 0.0, 1e-30, 6e4])
    x[rng.integers(0, rows), :] = 0.0
    t = torch.from_numpy(x).to(DT[dt]).to(DEV)
    return t[:, :cols] if ld != cols else t


@pytest.mark.parametrize("B", WIDTHS)
@pytest.mark.parametrize("dt,arith", [("bf16", "f32"), ("bf16", "native"), ("f16", "native"),
                                      ("f16", "f32"), ("f32", "f32")])
def test_width_vs_oracle(B, dt, arith):
    print("rowg", B, dt, arith, flush=True)
    rng = np.random.default_rng(B * 7 + len(dt) + len(arith))
    for rows, mult, pitch, pow2, sbf16 in CASES if B <= 2048 else CASES_WIDE:
        sbf16 = sbf16 and arith == "f32"
        cols = B * mult
        ld = cols + pitch
        if DT[dt].itemsize * ld % 16:
            ld = cols
        t = weights(rng, rows, cols, ld, dt)
        c, s = ops.fp8_block_quant(t, (1, B), native_arith=arith == "native", pow2=pow2,
                                   scale_dtype=torch.bfloat16 if sbf16 else None)
        torch.cuda.synchronize()
        oc, osc = O.fp8_block_quant(host(t, dt), dt, arith, (1, B), pow2)
        assert np.array_equal(c.view(torch.uint8).cpu().numpy(), oc[0]), (B, rows, cols, ld)
        want = O.bf16_from_f32(osc[0]) if sbf16 else osc[0]
        want = want.view(np.uint32) if want.dtype == np.float32 else want
        got = s.cpu().contiguous()
        got = got.numpy().view(np.uint32) if got.dtype == torch.float32 else got.view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got.reshape(-1), want.reshape(-1)), (B, rows, cols, ld)


@pytest.mark.parametrize("B", [96, 40, 200, 8, 1536, 4104, 36, 1000, 3001, 7000])
def test_grouped_plan_and_expert_stacks(B):
    print("rowg grouped", B, flush=True)
    rng = np.random.default_rng(B)
    ts = [weights(rng, r, B * m, B * m, "bf16") for r, m in [(100, 3), (1, 7), (333, 1), (64, 16)]]
    ts.append(torch.from_numpy(rng.normal(0, 0.02, (3, 50, B * 2)).astype(np.float32)).to(torch.bfloat16).to(DEV))
    plan = ops.QuantPlan(ts, "fp8_block", (1, B), scale_dtype=torch.bfloat16)
    for step in range(2):
        outs = plan.run()
        torch.cuda.synchronize()
        for t, (c, s) in zip(ts, outs):
            x = host(t, "bf16")
            oc, osc = O.fp8_block_quant(x.reshape(-1, x.shape[-1]), "bf16", "f32", (1, B), False)
            assert np.array_equal(c.view(torch.uint8).cpu().numpy().reshape(-1), oc.reshape(-1)), (B, step)
            want = O.bf16_from_f32(osc.reshape(-1))
            assert np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1), want), (B, step)


@pytest.mark.parametrize("block", [96, 36, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dropin_quantize_tensor_odd_blocks_match_reference_ops(dtype, block):
    torch.manual_seed(5)
    w = (torch.randn(300, 9000 if block == 1000 else 2880) * 0.02).to(dtype)
    wq = WeightQuantizer(FP8Config())
    q, s = wq.quantize_tensor(w.to(DEV), block_size=block)
    rq, rs = TR.quantize_tensor(w, block)
    assert q.shape == rq.shape and s.shape == rs.shape and s.dtype == rs.dtype
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu().view(torch.int16 if s.element_size() == 2 else torch.int32),
                       rs.view(torch.int16 if rs.element_size() == 2 else torch.int32))


def test_tiny_blocks_past_one_launch():
    """1x5 blocks of a [8192, 16400] weight: 26.9 M blocks on the generic kernel
    (one work-group each) exceed one launch's 2^32 threads, so the entry point
    splits the tensor into bands of rows, one launch each."""
    print("rowg 1x5 past one launch", flush=True)
    rng = np.random.default_rng(55)
    x = torch.from_numpy(rng.normal(0, 0.02, (8192, 16400)).astype(np.float32)).to(torch.bfloat16)
    x[77, 5:10] = 0.0
    x[4000, 12] = float("inf")
    c, s = ops.fp8_block_quant(x.to(DEV), (1, 5))
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(host(x, "bf16"), "bf16", "f32", (1, 5), nthreads=16)
    assert np.array_equal(c.view(torch.uint8).cpu().numpy(), oc[0])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), osc[0].view(np.uint32))


@pytest.mark.parametrize("B", [8, 12, 36, 96, 100, 1000])
@pytest.mark.parametrize("odt", [torch.float32, torch.bfloat16])
def test_dequant_widths_vs_reference_ops(B, odt):
    """dequantize_tensor (weight_quantizer.py:79-89) at widths the lane-chunks
    fit differently: 8 codes per chunk (bf16 out, 8 | B), 4 (float32 out, or
    bf16 out with 4 | B but not 8: 12, 36, 100), the per-element kernel
    otherwise; the bf16 output is the reference's float32 result cast, as
    dequantize_state_dict does (:133).  Codes also read from a view 3 bytes
    into its storage."""
    print("rowg dequant", B, odt, flush=True)
    g = torch.Generator().manual_seed(B)
    w = (torch.randn(97, B * 7, generator=g) * 0.05).to(torch.bfloat16)
    w[3, :B] = 0.0
    w[5, 2] = float("inf")
    w[9, 1] = float("nan")
    q, s = TR.quantize_tensor(w, B)
    want = TR.dequantize_tensor(q, s, B).to(odt)
    got = ops.fp8_block_dequant(q.to(DEV), s.to(DEV), (1, B), odt)
    buf = torch.zeros(q.numel() + 16, dtype=torch.uint8, device=DEV)
    buf[3:3 + q.numel()] = q.view(torch.uint8).reshape(-1).to(DEV)
    got_view = ops.fp8_block_dequant(buf[3:3 + q.numel()].view(q.shape), s.to(DEV), (1, B), odt)
    torch.cuda.synchronize()
    ints = torch.int32 if odt == torch.float32 else torch.int16
    for g_ in (got, got_view):
        g_ = g_.cpu()
        nan = torch.isnan(g_)
        assert torch.equal(nan, torch.isnan(want))
        assert torch.equal(g_[~nan].view(ints), want[~nan].view(ints))
