"""Seeded random sweep of grouped launches against the oracle, on an MI355X.

Each case is one plan over 1-12 tensors of random shape, dtype, row stride and
magnitude (Student-t values, planted +-inf/NaN/zero/tiny/huge entries, zero
rows): 128x128, 1x128 and odd-block FP8 (float32 or native arithmetic, pow2
and bf16 scale options), float64 FP8 in float64 arithmetic (dense 1xB rows or
any block over strided tensors, magnitudes across float64's range), MXFP8,
MXFP4, the unscaled cast, per-tensor KV scales, FP8
dequant of the 1x128 results and MX dequant of the MX results, to float32 and
bf16.  Every code, scale and output bit is compared with the oracle (MX dequant
with the torch restatement, NaN payloads aside: they depend on torch's loop
split, which a dedicated test pins).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref as TR
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
KINDS = ["tile", "row", "mx8", "mx4", "cast", "kv", "deq", "mxdeq", "blk", "f64"]
F64_BLOCKS = [(1, 32), (1, 128), (1, 512), (128, 128), (3, 40), (1, 96), (1, 1024), (1, 45), (1, 3000)]
BLOCKS = [(1, 32), (1, 64), (1, 256), (1, 512), (3, 40), (64, 96), (128, 64), (2, 128), (1, 96), (1, 40), (1, 16),
          (1, 1024), (1, 8), (1, 1536), (1, 4104), (1, 36), (1, 100), (1, 12)]


def host(t: torch.Tensor, dt: str) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.numpy() if dt in ("f32", "f64") else t.view(torch.int16).numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def fbits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.numpy().view(np.uint32) if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def _tensor(rng, rows, cols, dt, strided):
    ld = cols + (8 * int(rng.integers(1, 9)) if strided else 0)
    x = (rng.standard_t(4, (rows, ld)) * 10.0 ** rng.uniform(-4, 1)).astype(np.float32)
    for _ in range(int(rng.integers(0, 3))):
        x[rng.integers(0, rows), rng.integers(0, ld)] = rng.choice([np.inf, -np.inf, np.nan, 0.0, 1e-30, 6e4])
    if rng.random() < 0.1:
        r0 = int(rng.integers(0, rows))
        x[r0:r0 + 3, :] = 0.0
    t = torch.from_numpy(x).to(DT[dt]).to(DEV)
    return t[:, :cols] if strided else t


def _tensor64(rng, rows, cols, strided, pitch_step=1):
    ld = cols + (pitch_step * int(rng.integers(1, 9)) if strided else 0)
    x = rng.standard_t(4, (rows, ld)) * 2.0 ** rng.uniform(-1000, 1000)
    for _ in range(int(rng.integers(0, 4))):
        x[rng.integers(0, rows), rng.integers(0, ld)] = rng.choice(
            [np.inf, -np.inf, np.nan, 0.0, -0.0, 5e-324, -2.5e-310, 1e300])
    t = torch.from_numpy(x).to(DEV)
    return t[:, :cols] if strided else t


def _shape(rng, kind):
    if kind == "tile":
        return int(rng.integers(1, 600)), 8 * int(rng.integers(1, 120))
    if kind in ("row", "deq"):
        return int(rng.integers(1, 300)), 128 * int(rng.integers(1, 8))
    if kind == "blk":
        return int(rng.integers(1, 200)), 8 * int(rng.integers(1, 80))
    if kind in ("mx8", "mx4", "mxdeq"):
        return int(rng.integers(1, 300)), 32 * int(rng.integers(1, 30))
    return 1, int(rng.integers(1, 70000))


def _same_or_both_nan(got: torch.Tensor, want: torch.Tensor) -> bool:
    g, w = got.detach().cpu().float(), want.float()
    nan = torch.isnan(g)
    return bool(torch.equal(nan, torch.isnan(w))) and np.array_equal(fbits(got.cpu()[~nan]), fbits(want[~nan]))


@pytest.mark.parametrize("seed", [101, 202, 303])
def test_grouped_plans_random_sweep(seed):
    rng = np.random.default_rng(seed)
    for case in range(60):
        kind = KINDS[rng.integers(0, len(KINDS))]
        if kind == "f64":
            _f64_case(rng, seed, case)
            continue
        dt = ["bf16", "f16", "f32"][rng.integers(0, 3)]
        native = kind in ("tile", "row", "blk") and dt != "f32" and rng.random() < 0.3
        pow2 = kind in ("tile", "row", "blk") and rng.random() < 0.3
        blk = BLOCKS[rng.integers(0, len(BLOCKS))] if kind == "blk" else (128, 128) if kind == "tile" else (1, 128)
        sbf16 = kind == "row" and not native and rng.random() < 0.3
        ts = []
        blk_cols = _shape(rng, "blk")[1]  # one width per odd-block plan: one kernel for all
        if kind == "blk" and blk[0] == 1 and rng.random() < 0.7:
            blk_cols = blk[1] * int(rng.integers(1, 8))  # whole 1xB blocks: the row kernels
        for _ in range(int(rng.integers(1, 13))):
            rows, cols = _shape(rng, kind)
            cols = blk_cols if kind == "blk" else cols
            strided = kind not in ("cast", "kv") and rng.random() < 0.3
            ts.append(_tensor(rng, rows, cols, dt, strided))
        mxf = int(rng.choice([8, 4])) if kind == "mxdeq" else (8 if kind == "mx8" else 4)
        print("group sweep", seed, case, kind, dt, native, pow2, sbf16, [tuple(t.shape) for t in ts], flush=True)
        if kind in ("tile", "row", "deq", "blk"):
            outs = ops.QuantPlan(ts, "fp8_block", blk, native_arith=native, use_pow2_scale=pow2,
                                 scale_dtype=torch.bfloat16 if sbf16 else torch.float32).run()
        elif kind in ("mx8", "mx4", "mxdeq"):
            outs = ops.QuantPlan(ts, "mxfp8" if mxf == 8 else "mxfp4", (1, 32)).run()
        elif kind == "cast":
            outs = ops.CastPlan([t.reshape(-1) for t in ts]).run()
        else:
            scales = ops.TensorScalePlan(ts).run()
        torch.cuda.synchronize()
        for i, t in enumerate(ts):
            xh = host(t, dt)
            if kind in ("tile", "row", "deq", "blk"):
                oc, osc = O.fp8_block_quant(xh, dt, "native" if native else "f32", blk, pow2)
                assert np.array_equal(u8(outs[i][0]), oc[0]), (case, i)
                want_s = O.bf16_from_f32(osc[0]) if sbf16 else osc[0]
                want_s = want_s.view(np.uint32) if want_s.dtype == np.float32 else want_s
                assert np.array_equal(fbits(outs[i][1]).reshape(-1), want_s.reshape(-1)), (case, i)
            elif kind in ("mx8", "mx4", "mxdeq"):
                oc, osc = O.mx_quant(xh, dt, mxf)
                assert np.array_equal(u8(outs[i][0]), oc) and np.array_equal(u8(outs[i][1]), osc), (case, i)
            elif kind == "cast":
                assert np.array_equal(u8(outs[i]), O.cast_e4m3(xh.reshape(-1), dt)), (case, i)
            else:
                assert fbits(scales)[i] == O.tensor_scale(xh, dt), (case, i)
        if kind == "mxdeq":
            for odt in (torch.float32, torch.bfloat16):
                back = ops.DequantPlan(outs, (1, 32), odt, fmt="mxfp8" if mxf == 8 else "mxfp4").run()
                torch.cuda.synchronize()
                for i, (c, s) in enumerate(outs):
                    assert _same_or_both_nan(back[i], TR.mx_dequant(c.cpu(), s.cpu(), mxf, odt)), (case, i, odt)
        if kind == "deq":
            pairs = [(c.reshape(c.shape[0], -1), s) for c, s in outs]
            for odt, oname in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
                back = ops.DequantPlan(pairs, (1, 128), odt).run()
                torch.cuda.synchronize()
                for i, (c, s) in enumerate(pairs):
                    want = O.fp8_block_dequant(u8(c), fbits(s).view(np.float32).reshape(s.shape), "f32",
                                               (1, 128), oname)[0]
                    assert np.array_equal(fbits(back[i]), want.view(np.uint32) if oname == "f32" else want), \
                        (case, i, oname)


def _f64_case(rng, seed, case):
    """One grouped float64 plan: 1xB rows over widths that B divides (the row
    kernel for powers of two, the wide-row kernel for other B), possibly
    strided; 128x128 tiles over even widths (the tile kernel) or odd widths
    (the generic kernel); 1xB blocks over widths B does not divide, and 2-D
    blocks (the generic kernel).  One kernel per plan, as a grouped table
    requires."""
    blk = F64_BLOCKS[rng.integers(0, len(F64_BLOCKS))]
    row = blk[0] == 1 and rng.random() < 0.7  # whole blocks: row or wide-row kernel
    even = blk == (128, 128) and rng.random() < 0.6
    pow2 = bool(rng.random() < 0.3)
    ts = []
    for _ in range(int(rng.integers(1, 9))):
        rows = int(rng.integers(1, 300))
        if row:
            cols = blk[1] * int(rng.integers(1, 9 if blk[1] <= 512 else 3))
        elif blk == (128, 128):
            cols = 2 * int(rng.integers(1, 200)) + (0 if even else 1)
        else:
            cols = int(rng.integers(1, 400))
            if blk[0] == 1 and cols % blk[1] == 0:
                cols += 1  # a partial last block: the generic kernel
        ts.append(_tensor64(rng, rows, cols, strided=rng.random() < 0.3, pitch_step=2 if even else 1))
    print("group sweep", seed, case, "f64", blk, pow2, [tuple(t.shape) for t in ts], flush=True)
    outs = ops.QuantPlan(ts, "fp8_block", blk, native_arith=True, use_pow2_scale=pow2).run()
    torch.cuda.synchronize()
    for i, t in enumerate(ts):
        oc, osc = O.fp8_block_quant(host(t, "f64"), "f64", "native", blk, pow2)
        assert np.array_equal(u8(outs[i][0]), oc[0]), (case, i)
        got_s = outs[i][1].cpu().numpy().view(np.uint64).reshape(-1)
        assert np.array_equal(got_s, osc[0].view(np.uint64).reshape(-1)), (case, i)


@pytest.mark.parametrize("seed", [7, 8])
def test_split_plans_equal_one_launch(seed, monkeypatch):
    """Plans split into many launches of consecutive tensors (a ~256 KiB limit
    instead of ~3 GiB) write every byte a one-launch plan writes: FP8 128x128
    and 1x128, MXFP8, MXFP4 and the FP8 / MX dequant plans, on ragged strided
    tensors; a re-bind to new storage keeps the split."""
    rng = np.random.default_rng(seed)
    ts = [_tensor(rng, int(rng.integers(1, 400)), 128 * int(rng.integers(1, 6)), "bf16", rng.random() < 0.3)
          for _ in range(24)]

    def plans(limit):
        monkeypatch.setattr(ops, "GROUP_LAUNCH_BYTES", limit)
        out = {"tile": ops.QuantPlan(ts, "fp8_block", (128, 128)),
               "row": ops.QuantPlan(ts, "fp8_block", (1, 128), scale_dtype=torch.bfloat16),
               "mx8": ops.QuantPlan(ts, "mxfp8", (1, 32)),
               "mx4": ops.QuantPlan(ts, "mxfp4", (1, 32))}
        for p in out.values():
            p.run()
        out["deq"] = ops.DequantPlan([(c, s) for c, s in out["row"].outputs], (1, 128), torch.bfloat16)
        out["mxdeq"] = ops.DequantPlan(list(out["mx8"].outputs), (1, 32), torch.float32, fmt="mxfp8")
        out["deq"].run()
        out["mxdeq"].run()
        torch.cuda.synchronize()
        return out

    one, split = plans(3 << 30), plans(256 << 10)
    assert all(len(p._launch.parts) == 1 for p in one.values())
    assert all(len(p._launch.parts) > 2 for p in split.values())
    for k in ("tile", "row", "mx8", "mx4"):
        for (c1, s1), (c2, s2) in zip(one[k].outputs, split[k].outputs):
            assert np.array_equal(u8(c1), u8(c2)), k
            assert np.array_equal(u8(s1), u8(s2)), k
    for k in ("deq", "mxdeq"):
        for o1, o2 in zip(one[k].outputs, split[k].outputs):
            assert np.array_equal(u8(o1), u8(o2)), k
    # new storage for every input: the split plan re-binds each of its launches
    moved = [t.clone() for t in ts]
    split["tile"].run(inputs=moved)
    torch.cuda.synchronize()
    for (c1, s1), (c2, s2) in zip(one["tile"].outputs, split["tile"].outputs):
        assert np.array_equal(u8(c1), u8(c2)) and np.array_equal(u8(s1), u8(s2))
