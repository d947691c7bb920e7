"""Alignment on an MI355X: inputs off their 16-byte boundaries take the vector
kernels, and outputs off a code chunk's alignment take the generic paths.

torch guarantees element alignment only: a view at an odd element offset, or a
row pitch that is not a multiple of 8 elements, starts its rows on 2-byte (or
4-byte, float32; 8-byte, float64) boundaries.  Under the HSA ABI the hardware
runs in unaligned-access mode, so the kernels' 16-byte loads take such
addresses directly; every code, scale and output bit is compared with the
oracle for each kernel family.  The generic kernels and the cast's element walk
still serve code outputs that are not aligned to a lane's chunk of codes; they
are reached here through the C ABI with offset output pointers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from lumenrl_amd import _lib
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "f64": torch.float64}
ABI_DT = {"bf16": _lib.DTYPE_BF16, "f16": _lib.DTYPE_F16, "f32": _lib.DTYPE_F32}


def say(*a):
    print(*a, flush=True)


def host(t: torch.Tensor, dt: str) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.numpy() if dt in ("f32", "f64") else t.view(torch.int16).numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def offset_view(rng, rows, cols, ld, off, dt):
    """[rows, cols] with row pitch ld, starting `off` elements into a fresh allocation."""
    x = rng.standard_t(4, rows * ld + off + 64) * 0.05
    for _ in range(4):
        x[rng.integers(off, off + rows * ld)] = rng.choice([np.inf, -np.inf, np.nan, 0.0, 1e-30, 300.0])
    x[off + ld * int(rng.integers(0, rows)):][:cols] = 0.0  # one zero row
    t = torch.from_numpy(x.astype(np.float64 if dt == "f64" else np.float32)).to(DT[dt]).to(DEV)
    return t[off:off + rows * ld].view(rows, ld)[:, :cols]


CASES = [(300, 1536, 1536, 1), (257, 1536, 1543, 3), (64, 4608, 4613, 5), (1, 3072, 3072, 7)]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_offset_inputs_match_the_oracle(dt, case):
    rows, cols, ld, off = CASES[case]
    rng = np.random.default_rng(100 * case + len(dt))
    x = offset_view(rng, rows, cols, ld, off, dt)
    assert x.data_ptr() % 16 != 0 or ld % 8 != 0
    xh = host(x, dt)
    say("alignment", dt, CASES[case])
    for blk in ((128, 128), (1, 128), (1, 96), (1, 1536), (1, 16)):
        for arith in ("f32",) if dt == "f32" else ("f32", "native"):
            c, s = ops.fp8_block_quant(x, blk, native_arith=arith == "native")
            torch.cuda.synchronize()
            oc, osc = O.fp8_block_quant(xh, dt, arith, blk)
            assert np.array_equal(u8(c), oc[0]), (blk, arith)
            want = osc[0].view(np.uint32) if osc.dtype == np.float32 else osc[0]
            got = s.cpu().numpy().view(np.uint32) if s.dtype == torch.float32 else s.cpu().view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(got.reshape(want.shape), want), (blk, arith)
    for fmt, fn in ((8, ops.quantize_mxfp8), (4, ops.quantize_mxfp4)):
        c, s = fn(x)
        torch.cuda.synchronize()
        oc, osc = O.mx_quant(xh, dt, fmt)
        assert np.array_equal(u8(c), oc) and np.array_equal(u8(s), osc), fmt
    a = ops.act_qdq(x, 128)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy().view(np.uint32), O.act_qdq(xh, dt, 128).view(np.uint32))
    sc = ops.TensorScalePlan([x]).run()
    assert int(sc.cpu().view(torch.int32).item()) & 0xFFFFFFFF == int(O.tensor_scale(xh, dt))
    flat = x.reshape(-1) if ld == cols else x[0]  # one contiguous run at the same offset
    q = ops.cast_e4m3(flat)
    torch.cuda.synchronize()
    assert np.array_equal(u8(q), O.cast_e4m3(host(flat, dt).reshape(-1), dt))


@pytest.mark.parametrize("blk", [(1, 128), (128, 128), (1, 512)])
def test_offset_float64_inputs(blk):
    rng = np.random.default_rng(blk[0] + blk[1])
    say("alignment float64", blk)
    for rows, cols, ld, off in ((200, 1024, 1024, 1), (130, 1024, 1031, 3)):
        x = offset_view(rng, rows, cols, ld, off, "f64")
        assert x.data_ptr() % 16 == 8
        c, s = ops.fp8_block_quant(x, blk, native_arith=True)
        torch.cuda.synchronize()
        oc, osc = O.fp8_block_quant(host(x, "f64"), "f64", "native", blk)
        assert np.array_equal(u8(c), oc[0]), (blk, rows, ld)
        assert np.array_equal(s.cpu().numpy().view(np.uint64).reshape(-1), osc[0].view(np.uint64).reshape(-1))


def _odd(n: int) -> torch.Tensor:
    """n bytes starting one byte past a fresh allocation."""
    return torch.zeros(n + 64, dtype=torch.uint8, device=DEV)[1:1 + n]


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_unaligned_codes_take_the_generic_paths(dt):
    rng = np.random.default_rng(7 + len(dt))
    rows, cols = 200, 768
    x = offset_view(rng, rows, cols, cols, 0, dt)
    xh = host(x, dt)
    stream = ops._stream(DEV)
    L = _lib.lib()
    say("unaligned codes", dt)
    # FP8 blocks: codes one byte off -> k_generic
    for blk in ((1, 128), (128, 128)):
        codes = _odd(rows * cols)
        scales = torch.zeros(-(-rows // blk[0]) * (cols // blk[1]), dtype=torch.float32, device=DEV)
        rc = L.lrq_fp8_block_quant(x.data_ptr(), ABI_DT[dt], 1, rows, cols, cols, rows * cols, blk[0], blk[1],
                                   codes.data_ptr(), scales.data_ptr(), 0, stream)
        _lib.check(rc, "lrq_fp8_block_quant")
        torch.cuda.synchronize()
        oc, osc = O.fp8_block_quant(xh, dt, "f32", blk)
        assert np.array_equal(codes.cpu().numpy(), oc[0].reshape(-1)), blk
        assert np.array_equal(scales.cpu().numpy().view(np.uint32), osc[0].view(np.uint32).reshape(-1)), blk
    # MX: codes one byte off -> k_mx_generic
    for fmt, fn in ((8, L.lrq_mxfp8_quant), (4, L.lrq_mxfp4_quant)):
        codes = _odd(rows * (cols if fmt == 8 else cols // 2))
        scales = torch.zeros(rows * cols // 32, dtype=torch.uint8, device=DEV)
        _lib.check(fn(x.data_ptr(), ABI_DT[dt], rows, cols, cols, codes.data_ptr(), scales.data_ptr(), stream),
                   "mx quant")
        torch.cuda.synchronize()
        oc, osc = O.mx_quant(xh, dt, fmt)
        assert np.array_equal(codes.cpu().numpy(), oc.reshape(-1)) and np.array_equal(
            scales.cpu().numpy(), osc.reshape(-1)), fmt
    # unscaled cast: codes one byte off -> the element walk
    n = rows * cols - 5
    codes = _odd(n)
    _lib.check(L.lrq_cast_e4m3(x.data_ptr(), ABI_DT[dt], n, codes.data_ptr(), stream), "lrq_cast_e4m3")
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), O.cast_e4m3(xh.reshape(-1)[:n], dt))
