"""MX dequantization (MXFP8 / MXFP4 codes + E8M0 -> bf16 / fp32) on an MI355X.

Oracle: oracle/torch_ref.mx_dequant (torch's own decode and product on the CPU),
pinned in test_oracle.py to the closed form element * 2^(E-127).  Bit-exact,
NaN payloads included (tensor sizes keep torch's loop in its vectorized body).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torch_ref as T
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)


def say(*a):
    print(*a, flush=True)


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy().view(np.uint32)


def every_pair(fmt: int):
    """Codes and scales covering every (code byte, E8M0) pair of ``fmt``."""
    e = np.repeat(np.arange(256, dtype=np.uint8), 8)[:, None]
    if fmt == 8:
        codes = np.tile(np.arange(256, dtype=np.uint8), (2048, 7))          # 1792 elements a row
    else:
        codes = np.tile(np.arange(256, dtype=np.uint8), (2048, 1))          # 512 elements a row
    groups = codes.shape[1] * (1 if fmt == 8 else 2) // 32
    return codes, np.repeat(e, groups, axis=1)


@pytest.mark.parametrize("fmt", [8, 4])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float32])
def test_every_code_and_scale(fmt, odt):
    say("mx dequant every pair", fmt, odt)
    codes, scales = every_pair(fmt)
    cd, sd = torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV)
    fn = ops.dequantize_mxfp8 if fmt == 8 else ops.dequantize_mxfp4
    got = fn(cd, sd, odt)
    want = T.mx_dequant(torch.from_numpy(codes), torch.from_numpy(scales), fmt, odt)
    assert got.dtype == odt and tuple(got.shape) == tuple(want.shape)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [8, 4])
def test_round_trip_of_quantized_weights(fmt):
    """quantize -> dequantize (bf16) equals the oracle, and quantizing the result
    again gives back the same codes and scales."""
    say("mx round trip", fmt)
    g = torch.Generator(device=DEV).manual_seed(11)
    x = (torch.randn(1024, 4096, generator=g, device=DEV) * 0.02)
    x[::97] *= torch.exp(torch.randn(x[::97].shape, generator=g, device=DEV) * 2)
    x = x.to(torch.bfloat16)
    x[5, 64:96] = 0.0
    x[9, 7] = float("inf")
    q, s = (ops.quantize_mxfp8 if fmt == 8 else ops.quantize_mxfp4)(x)
    dq = (ops.dequantize_mxfp8 if fmt == 8 else ops.dequantize_mxfp4)(q, s)
    assert np.array_equal(bits(dq), bits(T.mx_dequant(q, s, fmt, torch.bfloat16)))
    finite = torch.isfinite(dq).all(dim=-1)
    q2, s2 = (ops.quantize_mxfp8 if fmt == 8 else ops.quantize_mxfp4)(dq[finite])
    assert torch.equal(q2.view(torch.uint8), q[finite].view(torch.uint8))
    assert torch.equal(s2, s[finite])


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_grouped_plan_and_misaligned_codes(fmt):
    say("mx dequant plan", fmt)
    g = torch.Generator(device=DEV).manual_seed(12)
    shapes = [(8, 96, 2048), (3, 64), (1, 32), (257, 1024)]
    quant = ops.quantize_mxfp8 if fmt == "mxfp8" else ops.quantize_mxfp4
    pairs = [quant((torch.randn(s, generator=g, device=DEV) * 0.3).to(torch.bfloat16)) for s in shapes]
    for odt in (torch.bfloat16, torch.float32):
        plan = ops.DequantPlan(pairs, (1, 32), odt, fmt=fmt)
        outs = plan.run()
        torch.cuda.synchronize()
        for (q, s), o in zip(pairs, outs):
            want = T.mx_dequant(q, s, 8 if fmt == "mxfp8" else 4, odt)
            assert np.array_equal(bits(o), bits(want.reshape(o.shape)))
    # a code view starting 2 bytes into its storage is read in place
    q, s = pairs[3]
    qv, sv = q.view(torch.uint8).reshape(-1)[2:].reshape(-1)[: 64 * q.shape[-1]].reshape(64, -1), s[:64]
    qv = qv if fmt == "mxfp4" else qv.view(torch.float8_e4m3fn)
    dq = (ops.dequantize_mxfp8 if fmt == "mxfp8" else ops.dequantize_mxfp4)(qv, sv, torch.float32)
    want = T.mx_dequant(qv, sv, 8 if fmt == "mxfp8" else 4, torch.float32)
    assert np.array_equal(bits(dq), bits(want))
