"""Parity of the HIP kernels with the CPU oracle (bit-exact), on an MI355X.

Sizes: golden fixtures and random cases at oracle-friendly sizes, BASELINE
config 1 ([4096, 4096]) in full, one full Qwen3-8B layer through the grouped
launch, exhaustive (x, amax) pairs over every bf16 value, and every float32
bit pattern through the hardware e4m3 encoder.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import ROOT, load_golden
from oracle import oracle as O
from lumenrl_amd import _lib
from lumenrl_amd.quantization import ops

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)

DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
RNG = np.random.default_rng(1234)


def say(*a):
    print(*a, flush=True)


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def dev_from_bits(x: np.ndarray, dt: str) -> torch.Tensor:
    if dt == "f32":
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV)
    if dt == "f64":
        return torch.from_numpy(np.ascontiguousarray(x, np.float64)).to(DEV)
    t = torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16))
    return t.view(DT[dt]).to(DEV)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def scale_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    if t.dtype == torch.float64:
        return t.numpy().view(np.uint64)
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def weights(shape, outlier_frac=1e-3, dt="bf16"):
    x = RNG.normal(0.0, 0.02, shape).astype(np.float32)
    n = max(1, int(x.size * outlier_frac))
    idx = RNG.choice(x.size, n, replace=False)
    x.flat[idx] = RNG.choice([-1.0, 1.0], n) * RNG.uniform(0.5, 4.0, n)
    t = torch.from_numpy(x).to(DT[dt])
    return t


def assert_fp8_matches_oracle(xd, blk, arith="f32", pow2=False, scale_dtype=None):
    dt = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[xd.dtype]
    c, s = ops.fp8_block_quant(xd, blk, native_arith=arith == "native", pow2=pow2,
                               scale_dtype=scale_dtype)
    torch.cuda.synchronize()
    xh = host_bits(xd)
    shape = xh.shape
    x3 = xh.reshape((-1,) + shape[-2:]) if xh.ndim >= 2 else xh.reshape(1, 1, -1)
    oc, osc = O.fp8_block_quant(x3, dt, arith, blk, pow2)
    assert np.array_equal(u8(c).reshape(oc.shape), oc)
    got = scale_bits(s).reshape(-1)
    if scale_dtype == torch.bfloat16 and osc.dtype == np.float32:
        osc = O.bf16_from_f32(osc)
        want = osc.reshape(-1)
    else:
        want = osc.view(np.uint32).reshape(-1) if osc.dtype == np.float32 else osc.reshape(-1)
    assert np.array_equal(got, want)


# ----------------------------------------------------------------------------
# hardware encoders
# ----------------------------------------------------------------------------
@pytest.mark.slow
def test_hw_e4m3_encoder_all_float32_patterns():
    """v_cvt_pk_fp8_f32 vs the oracle's encoder on all 2^32 float32 patterns.

    Identical on every non-NaN input (finite, subnormal, +-inf).  On NaN input
    the hardware writes 0xFF whatever the sign (torch keeps the sign); the
    kernels never feed it a NaN -- inf/NaN blocks take special_code().
    """
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.uint8, device=DEV)
    bad_non_nan = 0
    nan_codes = set()
    for k in range((1 << 32) // chunk):
        start = k * chunk
        rc = _lib.lib().lrq_diag_e4m3_bits(start, chunk, out.data_ptr(), None)
        _lib.check(rc, "lrq_diag_e4m3_bits")
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = O.e4m3_from_f32_bits_range(start, chunk)
        bits = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32)
        isnan = (bits & 0x7FFFFFFF) > 0x7F800000
        diff = got != want
        nb = int((diff & ~isnan).sum())
        if nb:
            w = np.argwhere(diff & ~isnan)[:4].ravel()
            say("e4m3 mismatch", [(hex(start + int(i)), hex(got[i]), hex(want[i])) for i in w])
        bad_non_nan += nb
        if isnan.any():
            nan_codes |= set(np.unique(got[isnan]).tolist())
    assert bad_non_nan == 0
    assert nan_codes <= {0x7F, 0xFF}


@pytest.mark.slow
def test_hw_bf16_encoder_all_float32_patterns():
    """v_cvt_pk_bf16_f32 (dequant's bf16 output) vs the oracle's RNE on every
    non-NaN float32 pattern; NaN results never reach it (the kernel routes NaN
    codes and NaN/inf/zero scales through the explicit rules)."""
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int16, device=DEV)
    bad = 0
    for k in range((1 << 32) // chunk):
        start = k * chunk
        _lib.check(_lib.lib().lrq_diag_bf16_bits(start, chunk, out.data_ptr(), None), "diag")
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16)
        bits = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32)
        want = O.bf16_from_f32(bits.view(np.float32))
        isnan = (bits & 0x7FFFFFFF) > 0x7F800000
        nb = int(((got != want) & ~isnan).sum())
        if nb:
            w = np.argwhere((got != want) & ~isnan)[:4].ravel()
            say("bf16 mismatch", [(hex(start + int(i)), hex(got[i]), hex(want[i])) for i in w])
        bad += nb
    assert bad == 0


@pytest.mark.parametrize("fmt", [8, 4])
def test_mx_element_path_every_bf16_and_scale(fmt):
    """The MX kernels' element encoder on every finite bf16 x under every E8M0
    the format can produce (E4M3: 0..246, E2M1: 0..252) vs the oracle's
    element rule: x * 2^(127-E), E4M3 clamp +-448 / E2M1 saturation, RNE."""
    b = np.arange(0, 1 << 16, dtype=np.uint32)
    xb = (b << 16).view(np.float32)
    xb = xb[np.isfinite(xb)]
    if xb.size % 2:
        xb = xb[:-1]
    emax_byte = 246 if fmt == 8 else 252
    es = np.arange(0, emax_byte + 1, dtype=np.uint8)
    x = np.tile(xb, es.size)
    e_pair = np.repeat(es, xb.size // 2)
    e_elem = np.repeat(es, xb.size).astype(np.int64)
    with np.errstate(over="ignore", under="ignore"):
        v = np.ldexp(x.astype(np.float64), 127 - e_elem)
    if fmt == 8:
        want = O.e4m3_from_f32(np.clip(v, -448.0, 448.0).astype(np.float32))
    else:
        want = O.e2m1_from_f32(np.clip(v, -6.0, 6.0).astype(np.float32))
    xd = torch.from_numpy(x).to(DEV)
    ed = torch.from_numpy(e_pair).to(DEV)
    out = torch.empty(x.size, dtype=torch.uint8, device=DEV)
    rc = _lib.lib().lrq_diag_mx_encode(_lib.FMT_MXFP8 if fmt == 8 else _lib.FMT_MXFP4,
                                       xd.data_ptr(), ed.data_ptr(), out.data_ptr(), x.size, None)
    _lib.check(rc, "lrq_diag_mx_encode")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    bad = np.argwhere(got != want).ravel()
    if bad.size:
        say("mx encode mismatch", [(float(x[i]), int(e_elem[i]), hex(got[i]), hex(want[i])) for i in bad[:6]])
    assert bad.size == 0


# ----------------------------------------------------------------------------
# golden fixtures
# ----------------------------------------------------------------------------
FP8_GOLDEN = sorted(f for f in os.listdir(os.path.join(ROOT, "tests", "golden"))
                    if f.startswith("fp8_") and f != "fp8_dequant.npz")


@pytest.mark.parametrize("name", FP8_GOLDEN)
def test_fp8_golden_on_device(name):
    g = load_golden(name)
    dt, arith, pow2 = str(g["meta"][0]), str(g["meta"][1]), bool(int(g["meta"][2]))
    blk = tuple(int(v) for v in g["block"])
    say("golden", name, g["x"].shape)
    xd = dev_from_bits(g["x"], dt)
    c, s = ops.fp8_block_quant(xd, blk, native_arith=arith == "native", pow2=pow2)
    torch.cuda.synchronize()
    assert np.array_equal(u8(c).reshape(g["codes"].shape), g["codes"])
    want = g["scales"]
    got = scale_bits(s).reshape(want.shape)
    wbits = {np.dtype(np.float32): np.uint32, np.dtype(np.float64): np.uint64}.get(want.dtype)
    assert np.array_equal(got, want.view(wbits) if wbits else want)
    if "scales_bf16" in g:
        c2, s2 = ops.fp8_block_quant(xd, blk, pow2=pow2, scale_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert np.array_equal(scale_bits(s2).reshape(g["scales_bf16"].shape), g["scales_bf16"])
        assert np.array_equal(u8(c2), u8(c))


@pytest.mark.parametrize("name", ["mxfp8_bf16.npz", "mxfp4_bf16.npz", "mxfp8_f32.npz", "mxfp4_f32.npz"])
def test_mx_golden_on_device(name):
    g = load_golden(name)
    dt = "bf16" if "bf16" in name else "f32"
    xd = dev_from_bits(g["x"], dt)
    fn = ops.quantize_mxfp8 if name.startswith("mxfp8") else ops.quantize_mxfp4
    c, s = fn(xd)
    torch.cuda.synchronize()
    assert np.array_equal(u8(s), g["scales"])
    assert np.array_equal(u8(c), g["codes"])


def test_dequant_golden_on_device():
    g = load_golden("fp8_dequant.npz")
    c = torch.from_numpy(g["codes"]).to(DEV).view(torch.float8_e4m3fn)
    s = torch.from_numpy(g["scales"]).to(DEV)
    out = ops.fp8_block_dequant(c, s, (1, 128), torch.float32)
    sb = dev_from_bits(g["scales_bf16"], "bf16")
    outb = ops.fp8_block_dequant(c, sb, (1, 128), torch.bfloat16)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), g["out_f32"].view(np.uint32))
    assert np.array_equal(host_bits(outb), g["out_bf16"])


# ----------------------------------------------------------------------------
# random parity, every kernel path
# ----------------------------------------------------------------------------
def test_config1_full_tile128_and_row128():
    """[4096, 4096] bf16, 128x128 (32x32 scales) and 1x128."""
    x = weights((4096, 4096)).to(DEV)
    say("config1 tile")
    assert_fp8_matches_oracle(x, (128, 128))
    say("config1 row")
    assert_fp8_matches_oracle(x, (1, 128))
    assert_fp8_matches_oracle(x, (1, 128), scale_dtype=torch.bfloat16)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("arith", ["f32", "native"])
@pytest.mark.parametrize("pow2", [False, True])
def test_tile_and_row_kernels_dtypes(dt, arith, pow2):
    x = weights((384, 768), dt=dt)
    x[0, :5] = 0.0
    x[130:140, 300] = 0.0
    xd = x.to(DEV)
    assert_fp8_matches_oracle(xd, (128, 128), arith, pow2)
    assert_fp8_matches_oracle(xd, (1, 128), arith, pow2)


@pytest.mark.parametrize("bc", [32, 64, 256, 512])
def test_row_kernel_block_sizes(bc):
    xd = weights((96, 2048)).to(DEV)
    assert_fp8_matches_oracle(xd, (1, bc))


@pytest.mark.parametrize("blk", [(1, 96), (64, 64), (1, 8), (256, 128), (128, 256), (3, 40)])
def test_generic_kernel_odd_blocks(blk):
    xd = weights((200, 480)).to(DEV)
    assert_fp8_matches_oracle(xd, blk)


def test_ragged_tiles_and_strided_views():
    big = weights((520, 1100)).to(DEV)
    say("ragged tiles")
    assert_fp8_matches_oracle(big[:300, :392], (128, 128))        # strided (ld=1100), fast path
    assert_fp8_matches_oracle(big[:300, 1:393], (128, 128))       # 2-byte aligned rows, tile kernel
    assert_fp8_matches_oracle(big[:256, 8:520], (1, 128))         # strided rows, fast path
    assert_fp8_matches_oracle(big[:256, 3:515], (1, 128))         # 2-byte aligned rows, row kernel
    c1, s1 = ops.fp8_block_quant(big[:256, 8:520], (1, 128))
    c2, s2 = ops.fp8_block_quant(big[:256, 8:520].contiguous(), (1, 128))
    assert torch.equal(u8t(c1), u8t(c2)) and torch.equal(s1, s2)


def test_tiles_across_tensors_batches_and_edges():
    """128x128 tiles of a strided batch and of grouped launches whose tensors
    end in ragged edge tiles (rows or columns short of 128) and hold an inf
    and a zero row: every tile must match the oracle."""
    say("tiles: strided batch with ragged tiles")
    base = weights((3, 256, 272)).to(DEV)
    assert_fp8_matches_oracle(base[:, :200, :264], (128, 128))    # batch stride != rows * ld
    say("tiles: grouped ragged tensors")
    shapes = [(1000, 8), (130, 136), (2, 128, 128), (257, 384), (3, 136, 264), (129, 1032)]
    ws = [(weights(s) if s[0] else torch.zeros(s, dtype=torch.bfloat16)).to(DEV) for s in shapes]
    ws[1][129, 135] = float("inf")
    ws[3][256, :] = 0.0
    for n in (1, 2, 3, len(ws)):                                   # 8 .. 60 tiles per launch
        plan = ops.QuantPlan(ws[:n], "fp8_block", (128, 128))
        plan.run()
        torch.cuda.synchronize()
        for w, (c, s) in zip(ws[:n], plan.outputs):
            xh = host_bits(w)
            oc, osc = O.fp8_block_quant(xh.reshape((-1,) + xh.shape[-2:]), "bf16", "f32", (128, 128))
            assert np.array_equal(u8(c).reshape(oc.shape), oc)
            assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))


def u8t(c):
    return c.view(torch.uint8)


def test_expert_stacks_one_launch():
    """Config-3 shapes (fewer experts): [E,768,2048] and [E,2048,768] with a zero and an inf tile."""
    E = 8
    gu = weights((E, 768, 2048))
    dn = weights((E, 2048, 768))
    gu[3, 128:256, 512:640] = 0.0
    dn[5, 1024 + 7, 256 + 9] = float("inf")
    for t in (gu, dn):
        assert_fp8_matches_oracle(t.to(DEV), (128, 128))


def test_edge_blocks_fp8():
    x = weights((8, 512))
    x[0, :128] = 0.0
    x[0, 5] = -0.0
    x[1, 3], x[1, 4] = float("inf"), -float("inf")
    x[2, 7] = float("nan")
    x[3, :128] = 1e-40
    x[4, :128] = torch.randn(128) * 1e-30
    x[5, 9] = 3.3e38
    x[6, 130], x[6, 131] = float("nan"), -float("inf")
    x[7, 256:384] = 1e-38
    xd = x.to(DEV)
    # small tensor: native-bf16 and pow2 NaN rules are the vectorized-body ones
    for blk in ((1, 128), (1, 64), (8, 128), (1, 96)):
        for arith in ("f32", "native"):
            for pow2 in (False, True):
                assert_fp8_matches_oracle(xd, blk, arith, pow2)
    xf = x.float().to(DEV)
    for pow2 in (False, True):
        assert_fp8_matches_oracle(xf, (1, 128), "f32", pow2)
        assert_fp8_matches_oracle(xf, (128, 128), "f32", pow2)


@pytest.mark.parametrize("fmt", [8, 4])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_mx_random_and_strided(fmt, dt):
    x = weights((256, 1024), dt=dt)
    x = x * torch.exp(torch.empty(256, 1).uniform_(np.log(0.25), np.log(4.0))).to(x.dtype)
    x[0, :32] = 0.0
    x[1, 40] = float("nan")
    x[2, 70] = -float("inf")
    x[3, 96:128] = 1e-40 if dt != "f16" else 1e-7
    fn = ops.quantize_mxfp8 if fmt == 8 else ops.quantize_mxfp4
    for xd, tag in ((x.to(DEV), "contig"), (torch.cat([x, x], 1).to(DEV)[:, 512:1536 - 0][:, :1024], "strided")):
        c, s = fn(xd)
        torch.cuda.synchronize()
        oc, osc = O.mx_quant(host_bits(xd.contiguous()), dt, fmt)
        assert np.array_equal(u8(s), osc), tag
        assert np.array_equal(u8(c), oc), tag
    # a view off its 16-byte alignment (2-byte aligned rows): the vector MX kernel
    big = torch.cat([x, x], 1).to(DEV)
    xv = big[:, 1:1025 - 0][:, :992]
    c, s = fn(xv)
    torch.cuda.synchronize()
    oc, osc = O.mx_quant(host_bits(xv.contiguous()), dt, fmt)
    assert np.array_equal(u8(s), osc) and np.array_equal(u8(c), oc)


def test_empty_tensors():
    for shape in ((0, 256), (4, 0), (0,)):
        x = torch.zeros(shape, dtype=torch.bfloat16, device=DEV)
        c, s = ops.fp8_block_quant(x, (1, 128))
        assert c.shape == x.shape
    c, s = ops.quantize_mxfp8(torch.zeros((0, 64), dtype=torch.bfloat16, device=DEV))
    assert c.shape == (0, 64) and s.shape == (0, 2)


# ----------------------------------------------------------------------------
# grouped launches
# ----------------------------------------------------------------------------
QWEN3_8B_LAYER = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096),
                  (12288, 4096), (12288, 4096), (4096, 12288)]


@pytest.mark.parametrize("fmt,blk", [("fp8_block", (128, 128)), ("fp8_block", (1, 128)),
                                     ("mxfp8", None), ("mxfp4", None)])
def test_grouped_qwen3_layer_matches_oracle(fmt, blk):
    say("grouped layer", fmt, blk)
    ws = [weights(s).to(DEV) for s in QWEN3_8B_LAYER]
    plan = ops.QuantPlan(ws, fmt, blk or (1, 32))
    plan.run()
    torch.cuda.synchronize()
    for w, (c, s) in zip(ws, plan.outputs):
        xh = host_bits(w)
        if fmt == "fp8_block":
            oc, osc = O.fp8_block_quant(xh, "bf16", "f32", blk)
            assert np.array_equal(u8(c).reshape(oc.shape), oc)
            assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))
        else:
            oc, osc = O.mx_quant(xh, "bf16", 8 if fmt == "mxfp8" else 4)
            assert np.array_equal(u8(c), oc) and np.array_equal(u8(s), osc)
    # re-running after the inputs change re-quantizes the new values
    ws[0].mul_(2)
    plan.run()
    torch.cuda.synchronize()
    if fmt == "fp8_block":
        oc, osc = O.fp8_block_quant(host_bits(ws[0]), "bf16", "f32", blk)
        assert np.array_equal(u8(plan.outputs[0][0]).reshape(oc.shape), oc)


def test_device_built_work_group_map():
    """lrq_group_build_map writes map[w] = the tensor owning work-group w, empty
    tensors (first, between, last) owning none, as a host loop over the
    descriptors' [unit0, unit0 + units) ranges would."""
    shapes = [(0, 4096), (256, 4096), (0, 128), (0, 4096), (4096, 4096), (128, 128), (0, 128)]
    ws = [(weights(s) if s[0] else torch.zeros(s, dtype=torch.bfloat16)).to(DEV) for s in shapes]
    say("device map", shapes)
    L = _lib.lib()
    descs = (_lib.LrqTensor * len(ws))()
    outs = []
    for i, w in enumerate(ws):
        c = torch.empty(w.shape, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty((-(-w.shape[0] // 128), w.shape[1] // 128), dtype=torch.float32, device=DEV)
        outs.append((c, s))
        descs[i].in_, descs[i].codes, descs[i].scales = w.data_ptr(), c.data_ptr(), s.data_ptr()
        descs[i].batch, descs[i].rows, descs[i].cols = 1, w.shape[0], w.shape[1]
        descs[i].ld, descs[i].batch_stride = w.shape[1], w.numel()
    launch = ops._GroupLaunch("fp8_block", descs, len(ws), _lib.DTYPE_BF16, (128, 128), 0, DEV)
    tiles = [(r // 128) * (c // 128) for r, c in shapes]
    assert launch.units == sum(tiles)
    host_bytes = launch.host.numel()
    torch.cuda.synchronize()
    wmap = launch.dev[host_bytes:].cpu().numpy().view(np.uint32)
    assert np.array_equal(wmap, np.repeat(np.arange(len(shapes), dtype=np.uint32), tiles))
    launch.run()
    torch.cuda.synchronize()
    for w, (c, s) in zip(ws, outs):
        if w.numel():
            oc, osc = O.fp8_block_quant(host_bits(w), "bf16", "f32", (128, 128))
            assert np.array_equal(u8(c).reshape(oc.shape), oc)
            assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))


def test_grouped_expert_stacks_single_launch():
    gu = weights((16, 1536, 2048))
    dn = weights((16, 2048, 768))
    gu[2, :128, :128] = 0.0
    dn[9, 300, 400] = float("inf")
    ws = [gu.to(DEV), dn.to(DEV)]
    plan = ops.QuantPlan(ws, "fp8_block", (128, 128))
    assert plan.units == 16 * 12 * 16 + 16 * 16 * 6
    plan.run()
    torch.cuda.synchronize()
    for w, (c, s) in zip(ws, plan.outputs):
        oc, osc = O.fp8_block_quant(host_bits(w), "bf16", "f32", (128, 128))
        assert np.array_equal(u8(c).reshape(oc.shape), oc)
        assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))


def test_plan_mixing_kernels_raises_wherever_launches_split(monkeypatch):
    """A plan whose tensors take different kernels (128x128 tiles with K % 8
    != 0 take the generic kernel) raises ValueError whether the two tensors
    share a launch or not."""
    ws = [weights((256, 256)).to(DEV), weights((256, 300)).to(DEV)]
    for limit in (ops.GROUP_LAUNCH_BYTES, 1):  # one launch; one launch per tensor
        monkeypatch.setattr(ops, "GROUP_LAUNCH_BYTES", limit)
        with pytest.raises(ValueError, match="tensor 1 needs a different kernel than tensor 0"):
            ops.QuantPlan(ws, "fp8_block", (128, 128))
    # each kind alone still plans and runs, split or not
    plan = ops.QuantPlan([ws[0], weights((300, 512)).to(DEV)], "fp8_block", (128, 128))
    assert len(plan._launch.parts) == 2
    plan.run()
    torch.cuda.synchronize()
    for w, (c, s) in zip(plan.inputs, plan.outputs):
        oc, osc = O.fp8_block_quant(host_bits(w)[None], "bf16", "f32", (128, 128))
        assert np.array_equal(u8(c).reshape(oc.shape), oc)
        assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))


def test_tile_xcd_runs_at_odd_offsets_and_tails():
    """The tile kernel remaps each tensor's tiles in runs of 4 (rows of a
    multiple of 8 KiB) or 8 (other pitches), within the tensor: tensors that
    start at work-groups off a run-chunk boundary, whole chunks followed by a
    partial one, and a strided view whose pitch (not width) sets the run must
    all match the oracle tile for tile."""
    wide = weights((600, 4096))
    shapes = [(300, 1000),        # 24 tiles, pitch 2000 B: runs of 8, all in the partial chunk
              (1100, 2048),       # 144 tiles from work-group 24: 2 chunks of 64 + 16
              (640, 4096),        # 160 tiles from 168 (168 % 32 = 8), runs of 4: 5 chunks
              (2, 700, 768)]      # 72 tiles from 328: 1 chunk + 8
    ws = [weights(s) for s in shapes]
    ws[1][1000, 2000] = float("inf")
    ws[3][1, 128:256, 384:512] = 0.0
    views = [w.to(DEV) for w in ws]
    views.append(wide.to(DEV)[:, 64:2112])  # 80 tiles, cols 2048 on 8 KiB rows: runs of 4
    plan = ops.QuantPlan(views, "fp8_block", (128, 128))
    assert plan.units == 24 + 144 + 160 + 72 + 80
    plan.run()
    torch.cuda.synchronize()
    say("tile runs: grouped")
    for w, (c, s) in zip(views, plan.outputs):
        xh = host_bits(w)
        oc, osc = O.fp8_block_quant(xh.reshape((-1,) + xh.shape[-2:]), "bf16", "f32", (128, 128))
        assert np.array_equal(u8(c).reshape(oc.shape), oc)
        assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))
    say("tile runs: single launches")
    assert_fp8_matches_oracle(weights((1300, 1536)).to(DEV), (128, 128))  # 132 tiles: 2 chunks + 4
    assert_fp8_matches_oracle(views[4], (128, 128))


# ----------------------------------------------------------------------------
# exhaustive (x, amax): every bf16 x against every finite bf16 amax
# ----------------------------------------------------------------------------
def exhaustive_blocks(per_block: int, dt: str = "bf16") -> np.ndarray:
    """Rows of `per_block` bf16 (or fp16) patterns: slot 0 holds amax a, the
    rest every x with |x| <= a (both signs), for every finite positive a."""
    rows = []
    for a in range(1, 0x7F80 if dt == "bf16" else 0x7C00):
        xs = np.concatenate([np.arange(0, a + 1, dtype=np.uint16),
                             np.arange(0x8000, 0x8000 + a + 1, dtype=np.uint16)])
        k = per_block - 1
        nb = -(-xs.size // k)
        pad = np.full(nb * k - xs.size, a, np.uint16)
        blk = np.concatenate([xs, pad]).reshape(nb, k)
        rows.append(np.concatenate([np.full((nb, 1), a, np.uint16), blk], axis=1))
    return np.concatenate(rows)


@pytest.mark.slow
@pytest.mark.parametrize("arith", ["f32", "native"])
def test_exhaustive_pairs_row_kernel(arith):
    xb = exhaustive_blocks(128)
    say("exhaustive row", arith, xb.shape)
    xd = dev_from_bits(xb, "bf16")
    c, s = ops.fp8_block_quant(xd, (1, 128), native_arith=arith == "native")
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(xb, "bf16", arith, (1, 128))
    got = u8(c)
    bad = int((got.reshape(oc.shape) != oc).sum())
    assert bad == 0
    sb = scale_bits(s).reshape(-1)
    want = osc.view(np.uint32).reshape(-1) if osc.dtype == np.float32 else osc.reshape(-1)
    assert np.array_equal(sb, want)


@pytest.mark.slow
@pytest.mark.parametrize("arith", ["f32", "native"])
def test_exhaustive_pairs_f16_row_and_tile_kernels(arith):
    """Every fp16 x against every finite fp16 amax (1.0 G pairs) through the 1x128
    row kernel and the 128x128 tile kernel: the Markstein quotient, rounded to
    fp16 in native arithmetic, equals the oracle's IEEE division everywhere."""
    for blk in ((1, 128), (128, 128)):
        xb = exhaustive_blocks(blk[0] * 128, "f16").reshape(-1, 128)
        say("exhaustive f16", arith, blk, xb.shape)
        xd = dev_from_bits(xb, "f16")
        c, s = ops.fp8_block_quant(xd, blk, native_arith=arith == "native")
        torch.cuda.synchronize()
        oc, osc = O.fp8_block_quant(xb, "f16", arith, blk)
        assert int((u8(c).reshape(oc.shape) != oc).sum()) == 0, blk
        sb = scale_bits(s).reshape(-1)
        want = osc.view(np.uint32).reshape(-1) if osc.dtype == np.float32 else osc.reshape(-1)
        assert np.array_equal(sb, want), blk
        del xb, xd, c, s, oc, osc


def _e4m3_midpoints() -> np.ndarray:
    """The 126 rounding boundaries between consecutive non-negative e4m3 values."""
    c = np.arange(0, 127)
    e, m = c >> 3, c & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    return (v[:-1] + v[1:]) / 2.0


@pytest.mark.parametrize("blk", [(1, 128), (128, 128)])
def test_float32_quotients_next_to_e4m3_midpoints(blk):
    """Float32 weights have no exhaustive sweep, so aim at the inputs where the
    kernels' Markstein quotient could round differently from IEEE x/s: for
    2000 scales across float32's range (and on both sides of the 2^-80 amax
    guard), every x within 2 ulps of m*s for each e4m3 rounding boundary m,
    both signs.  Codes and scales must equal the oracle's (IEEE division)."""
    rng = np.random.default_rng(2024)
    mids = _e4m3_midpoints()
    amaxes = np.concatenate([2.0 ** rng.uniform(-120, 120, 1990),
                             2.0 ** -80 * np.array([0.5, 0.999, 1.0, 1.001, 2.0]),
                             np.array([448.0, 1.0, 3.0e38, 1.2e-38, 7.0])]).astype(np.float32)
    per = blk[0] * 128
    blocks = []
    for a in amaxes:
        s = np.float32(a) / np.float32(448.0)  # what the kernel derives (checked against the oracle's scales)
        xs = (mids * np.float64(s)).astype(np.float32)
        up1 = np.nextafter(xs, np.float32(np.inf))
        dn1 = np.nextafter(xs, np.float32(0))
        x = np.concatenate([xs, up1, np.nextafter(up1, np.float32(np.inf)),
                            dn1, np.nextafter(dn1, np.float32(0))])
        x = x[np.abs(x) <= a]
        x = np.concatenate([x, -x])
        take = np.zeros(per, np.float32)
        n = min(per - 1, x.size)
        take[0] = a
        take[1:1 + n] = x[:n]
        blocks.append(take.reshape(blk[0], 128))
        for rest in range(per - 1, x.size, per - 1):  # the values that did not fit
            more = np.zeros(per, np.float32)
            chunk = x[rest:rest + per - 1]
            more[0] = a
            more[1:1 + chunk.size] = chunk
            blocks.append(more.reshape(blk[0], 128))
    xb = np.concatenate(blocks).astype(np.float32)
    say("float32 midpoint neighbours", blk, xb.shape)
    xd = torch.from_numpy(xb).to(DEV)
    c, sc = ops.fp8_block_quant(xd, blk)
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(xb[None], "f32", "f32", blk)
    got = u8(c).reshape(oc.shape)
    bad = np.argwhere(got != oc)
    if bad.size:
        say("mismatches", bad.shape[0], [(float(xb.reshape(-1)[i]), hex(got.reshape(-1)[i]), hex(oc.reshape(-1)[i]))
                                        for i in np.flatnonzero(got.reshape(-1) != oc.reshape(-1))[:6]])
    assert bad.size == 0
    assert np.array_equal(scale_bits(sc).reshape(-1), osc.view(np.uint32).reshape(-1))


@pytest.mark.slow
def test_exhaustive_pairs_tile_kernel():
    xb = exhaustive_blocks(128 * 128).reshape(-1, 128)
    say("exhaustive tile", xb.shape)
    xd = dev_from_bits(xb, "bf16")
    c, s = ops.fp8_block_quant(xd, (128, 128))
    torch.cuda.synchronize()
    oc, osc = O.fp8_block_quant(xb, "bf16", "f32", (128, 128))
    assert np.array_equal(u8(c).reshape(oc.shape), oc)
    assert np.array_equal(scale_bits(s).reshape(-1), osc.view(np.uint32).reshape(-1))


# ----------------------------------------------------------------------------
# dequant (weight_quantizer.py:79-89, :133) and quantize-into-bucket
# ----------------------------------------------------------------------------
def _codes_and_scales(shape, blk, sdt):
    rows, cols = shape[-2], shape[-1]
    lead = shape[:-2]
    codes = RNG.integers(0, 256, shape, dtype=np.uint8)
    sshape = lead + (-(-rows // blk[0]), -(-cols // blk[1]))
    sc = (RNG.normal(0, 1e-3, sshape)).astype(np.float32)
    flat = sc.reshape(-1)
    flat[:4] = [0.0, np.inf, np.nan, -np.inf]
    if sdt == "f32":
        return codes, flat.reshape(sshape), flat.reshape(sshape)
    t = torch.from_numpy(flat).to(DT[sdt])
    bits16 = t.view(torch.int16).numpy().view(np.uint16).reshape(sshape)
    return codes, bits16, t.reshape(sshape)


@pytest.mark.parametrize("blk", [(1, 128), (128, 128), (1, 64), (1, 40), (64, 48)])
@pytest.mark.parametrize("sdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("odt", ["f32", "bf16"])
def test_dequant_paths_match_oracle(blk, sdt, odt):
    shape = (3, 200, 480) if blk[1] % 16 == 0 else (200, 480)
    codes, sbits, st = _codes_and_scales(shape, blk, sdt)
    cd = torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn)
    sd = st.to(DEV) if isinstance(st, torch.Tensor) else torch.from_numpy(st).to(DEV)
    out = ops.fp8_block_dequant(cd, sd, blk, torch.float32 if odt == "f32" else torch.bfloat16)
    torch.cuda.synchronize()
    c3 = codes.reshape((-1,) + shape[-2:])
    want = O.fp8_block_dequant(c3, sbits, sdt, blk, odt)
    got = out.cpu().contiguous()
    got = got.numpy().view(np.uint32) if odt == "f32" else got.view(torch.int16).numpy().view(np.uint16)
    w = want.view(np.uint32) if odt == "f32" else want
    assert np.array_equal(got.reshape(w.shape), w)


def test_grouped_dequant_plan_matches_oracle():
    pairs, host = [], []
    for rows, cols in QWEN3_8B_LAYER[:4]:
        codes, sbits, st = _codes_and_scales((rows, cols), (1, 128), "bf16")
        pairs.append((torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn), st.to(DEV)))
        host.append((codes, sbits))
    plan = ops.DequantPlan(pairs, (1, 128), torch.bfloat16)
    outs = plan.run()
    torch.cuda.synchronize()
    for (codes, sbits), o in zip(host, outs):
        want = O.fp8_block_dequant(codes, sbits, "bf16", (1, 128), "bf16")[0]
        assert np.array_equal(o.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("fmt", ["fp8_block", "mxfp8", "mxfp4"])
def test_bucket_writer_matches_oracle(fmt):
    from lumenrl_amd.quantization import QuantizedBucketWriter

    named = [("model.embed_tokens.weight", weights((512, 256)).to(DEV)),
             ("layers.0.self_attn.q_proj.weight", weights((512, 512)).to(DEV)),
             ("layers.0.input_layernorm.weight", torch.ones(512, dtype=torch.bfloat16, device=DEV)),
             ("layers.0.mlp.down_proj.weight", weights((256, 1024)).to(DEV)),
             ("layers.0.mlp.experts.w13", weights((4, 256, 384)).to(DEV)),
             ("lm_head.weight", weights((512, 256)).to(DEV))]
    writer = QuantizedBucketWriter(named, bucket_bytes=700_000, fmt=fmt)
    assert len(writer) >= 2
    src = dict(named)
    seen = set()
    for bucket in writer:
        bucket.fill()
        torch.cuda.synchronize()
        meta = bucket.bucket_meta()
        assert [e["name"] for e in bucket.rdma_entries()] == list(meta)
        views = dict(bucket.views())
        for name, t in views.items():
            seen.add(name)
            base = name[: -len("_scale_inv")] if name.endswith("_scale_inv") else name
            w = src[base]
            if base == name and t.dtype == w.dtype:       # pass-through
                assert torch.equal(t, w)
                continue
            xh = host_bits(w)
            if fmt == "fp8_block":
                oc, osc = O.fp8_block_quant(xh.reshape((-1,) + xh.shape[-2:]), "bf16", "f32", (128, 128))
                want = oc if name == base else osc
                got = u8(t) if name == base else scale_bits(t)
                assert np.array_equal(got.reshape(-1), (want if name == base else want.view(np.uint32)).reshape(-1))
            else:
                oc, osc = O.mx_quant(xh.reshape(-1, xh.shape[-1]), "bf16", 8 if fmt == "mxfp8" else 4)
                want = oc if name == base else osc
                assert np.array_equal(u8(t).reshape(-1), want.reshape(-1))
    assert seen == {n for n, _ in named} | {n + "_scale_inv" for n, _ in named
                                             if "embed" not in n and "lm_head" not in n and "norm" not in n}


def test_grouped_copy_plan_odd_sizes():
    """Grouped byte copies of sizes around the 4 KiB unit and 16-byte tails."""
    from lumenrl_amd.quantization import CopyPlan

    g = torch.Generator(device=DEV).manual_seed(8)
    sizes = [1, 15, 16, 200, 4095, 4096, 4097, 4096 * 7 + 9, 16385, 3 << 20]
    srcs = [torch.randint(0, 256, (n,), generator=g, device=DEV, dtype=torch.uint8) for n in sizes]
    dsts = [torch.full((n,), 0xAB, device=DEV, dtype=torch.uint8) for n in sizes]
    plan = CopyPlan(list(zip(dsts, srcs)))
    plan.run()
    torch.cuda.synchronize()
    for n, d, s in zip(sizes, dsts, srcs):
        assert torch.equal(d, s), n
    # any dtype: bf16 weights copied bytewise into uint8 views
    w = torch.randn(300, 130, generator=g, device=DEV).to(torch.bfloat16)
    out = torch.empty(300 * 130 * 2, dtype=torch.uint8, device=DEV)
    CopyPlan([(out, w.reshape(-1).view(torch.uint8))]).run()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.bfloat16).view(300, 130), w)
