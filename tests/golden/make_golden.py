"""Write the golden fixtures under tests/golden/ (run from the repo root).

FP8 blockwise fixtures are produced by the reference's op sequence evaluated
with torch on this x86 CPU (oracle/torch_ref.py restates
lumenrl/quantization/weight_quantizer.py op for op).  MX fixtures are produced
by the independent numpy restatement of OCP MX v1.0 below (float64 exact
scaling, torch's float8_e4m3fn cast for E4M3, nearest-even grid search for
E2M1) -- not by the C oracle, which the tests check against these files.

    python tests/golden/make_golden.py        (all fixtures)
    python tests/golden/make_golden.py f64    (the float64 ones only)
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import torch_ref  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def weights(rng: np.random.Generator, shape, outlier_frac=1e-3) -> np.ndarray:
    """N(0, 0.02^2) with a fraction of entries replaced by +-U(0.5, 4)."""
    x = rng.normal(0.0, 0.02, shape).astype(np.float32)
    n = max(1, int(x.size * outlier_frac))
    idx = rng.choice(x.size, n, replace=False)
    x.flat[idx] = rng.choice([-1.0, 1.0], n) * rng.uniform(0.5, 4.0, n)
    return x


def plant_edges_rows(x: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    """Edge 1x128 blocks in the first rows of a [R, K>=256] array."""
    x = x.copy()
    x[0, :128] = 0.0
    x[0, 5] = -0.0
    x[0, 128:256] = -0.0
    x[1, 3], x[1, 4], x[1, 5] = np.inf, -np.inf, -0.0
    x[2, 7] = np.nan
    x[2, 128 + 9] = -np.nan
    x[3, :128] = np.float32(1e-40)
    x[3, 1], x[3, 2] = -np.float32(2e-39), np.float32(1.2e-38)
    x[4, :128] = rng.normal(0.0, 1e-30, 128)
    x[5, 9], x[5, 10] = 3.3e38, -3.3e38
    x[6, 130], x[6, 131] = np.nan, -np.inf
    x[7, 128:256] = rng.normal(0.0, 1e-36, 128)
    return x


def fp8_row_case(name, x_bf16_or_f, dtype_name, native, pow2, rows_edge=True):
    t = x_bf16_or_f
    tin = t if native else t.float()
    q, s = torch_ref.quantize_tensor(tin, 128, pow2)
    rec = {"codes": q.view(torch.uint8).numpy(), "block": np.array([1, 128])}
    if dtype_name in ("f32", "f64"):
        rec["x"] = t.numpy()
    elif dtype_name == "f16":
        rec["x"] = t.view(torch.int16).numpy().view(np.uint16)
    else:
        rec["x"] = bits16(t)
    if s.dtype == torch.float32:
        rec["scales"] = s.numpy()
        rec["scales_bf16"] = bits16(s.to(torch.bfloat16))
    elif s.dtype == torch.float64:
        rec["scales"] = s.numpy()
    else:
        rec["scales"] = s.view(torch.int16).numpy().view(np.uint16)
    rec["meta"] = np.array([dtype_name, "native" if native else "f32", int(pow2)], dtype="U8")
    np.savez_compressed(os.path.join(OUT, name), **rec)


def fp8_tile_case(name, t, pow2=False):
    q, s = torch_ref.quantize_tensor_tiles(t.float(), (128, 128), pow2)
    np.savez_compressed(os.path.join(OUT, name), x=bits16(t), codes=q.view(torch.uint8).numpy(),
                        scales=s.numpy(), block=np.array([128, 128]),
                        meta=np.array(["bf16", "f32", int(pow2)], dtype="U8"))


def f64_edges(rng: np.random.Generator, rows: int = 24, cols: int = 384) -> np.ndarray:
    """float64 weights with edge 1x128 blocks in the first rows."""
    x = rng.normal(0.0, 0.02, (rows, cols))
    idx = rng.choice(x.size, 10, replace=False)
    x.flat[idx] = rng.choice([-1.0, 1.0], 10) * rng.uniform(0.5, 4.0, 10)
    x[0, :128] = 0.0
    x[0, 5] = -0.0
    x[1, 3], x[1, 4], x[1, 5] = np.inf, -np.inf, -0.0
    x[2, 7] = np.nan
    x[2, 128 + 9] = -np.nan
    x[3, :128] = 5e-324                       # float64 subnormals
    x[3, 1], x[3, 2] = -1e-310, 2.2e-308
    x[4, :128] = rng.normal(0.0, 1e-300, 128)
    x[5, 9], x[5, 10] = 1.7e308, -1.7e308
    x[6, 130], x[6, 131] = np.nan, -np.inf
    # s == 1 exactly (amax 448): 1.0625 +- 2^-40 round to the float32 1.0625, an
    # e4m3 tie that goes to even (1.0); a single rounding would give 1.125
    x[7, :128] = 1.0625 + 2.0 ** -40
    x[7, 0], x[7, 1], x[7, 2] = 448.0, 1.0625 - 2.0 ** -40, -(1.1875 + 2.0 ** -35)
    x[8, :128] = rng.normal(0.0, 1.0, 128) * 2.0 ** -1030   # scale clamps to 2^-1022
    x[9, :128] = rng.normal(0.0, 1.0, 128) * 1e-320
    return x


def write_f64_fixtures() -> None:
    """quantize_tensor on float64 tensors: float64 arithmetic and scales."""
    rng = np.random.default_rng(20261202)
    x = f64_edges(rng)
    fp8_row_case("fp8_row_f64.npz", torch.from_numpy(x), "f64", native=True, pow2=False)
    # pow2: the NaN scale of a pow2 block depends on torch's loop position, so no
    # NaN here (tests/test_oracle.py pins that rule on a large tensor)
    xp = x.copy()
    xp[2, 7], xp[2, 128 + 9], xp[6, 130] = 0.3, -0.2, 0.1
    fp8_row_case("fp8_row_f64_pow2.npz", torch.from_numpy(xp), "f64", native=True, pow2=True)
    xt = rng.normal(0.0, 0.02, (256, 320))
    xt[0:128, 0:128] = 0.0
    xt[0:128, 128:256][5, 7] = np.inf
    xt[128:256, 0:128][9, 1] = np.nan
    xt[128:256, 128:256] = rng.normal(0.0, 1.0, (128, 128)) * 1e-310
    q, s = torch_ref.quantize_tensor_tiles(torch.from_numpy(xt), (128, 128), False)
    np.savez_compressed(os.path.join(OUT, "fp8_tile_f64.npz"), x=xt, codes=q.view(torch.uint8).numpy(),
                        scales=s.numpy(), block=np.array([128, 128]),
                        meta=np.array(["f64", "native", 0], dtype="U8"))


# ---------------------------------------------------------------- MX (numpy)
def mx_reference(xf: np.ndarray, fmt: int) -> tuple[np.ndarray, np.ndarray]:
    """Independent OCP MX v1.0 restatement; xf float32 [R, K] (K % 32 == 0)."""
    R, K = xf.shape
    g = xf.astype(np.float64).reshape(R, K // 32, 32)
    emax = 8 if fmt == 8 else 2
    a = np.abs(g)
    nonfinite = ~np.isfinite(g).all(axis=2)
    amax = np.where(np.isnan(a), 0, a).max(axis=2)
    m, e = np.frexp(np.where(nonfinite | (amax == 0), 1.0, amax))
    floor_log2 = e - 1  # amax = m*2^e, m in [0.5, 1)
    e8 = np.clip(floor_log2 - emax + 127, 0, 254)
    e8 = np.where(amax == 0, 0, e8)
    e8 = np.where(nonfinite, 255, e8).astype(np.uint8)
    scale = np.ldexp(1.0, np.where(nonfinite, 0, e8.astype(np.int64) - 127))
    v = g / scale[..., None]  # exact: power-of-two scaling in float64
    sign = np.signbit(g)
    if fmt == 8:
        vc = np.clip(np.where(np.isfinite(v), v, 0.0), -448.0, 448.0).astype(np.float32)
        codes = torch.from_numpy(vc).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
        special = np.where(~np.isfinite(g), 0x7F, 0).astype(np.uint8) | np.where(sign, 0x80, 0).astype(np.uint8)
        codes = np.where(nonfinite[..., None], special, codes)
        return codes.reshape(R, K), e8
    av = np.minimum(np.abs(np.where(np.isfinite(v), v, 0.0)), 6.0)
    d = np.abs(av[..., None] - E2M1_GRID)
    best = d.min(axis=-1, keepdims=True)
    cand = d == best
    idx = np.where(cand[..., ::2].any(axis=-1),
                   np.argmax(cand & (np.arange(8) % 2 == 0), axis=-1),
                   np.argmax(cand, axis=-1))
    nib = idx.astype(np.uint8) | np.where(sign, 8, 0).astype(np.uint8)
    nib = np.where(nonfinite[..., None], np.where(sign, 8, 0).astype(np.uint8), nib)
    nib = nib.reshape(R, K)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return packed, e8


def mx_inputs(rng: np.random.Generator) -> np.ndarray:
    R, K = 48, 512
    t = rng.standard_t(4, (R, K)) * (0.02 / np.sqrt(2.0))
    mult = np.exp(rng.uniform(np.log(0.25), np.log(4.0), (R, 1)))
    x = (t * mult).astype(np.float32)
    x[0, :32] = 0.0
    x[0, 3] = -0.0
    x[1, 32:64] = np.float32(1e-40)
    x[1, 40] = -np.float32(3e-39)
    x[2, 5] = np.nan
    x[2, 64 + 7] = -np.inf
    x[2, 128 + 1] = np.inf
    x[3, :32] = rng.normal(0, 1e-30, 32)
    x[4, 0:32] = rng.uniform(-3e38, 3e38, 32)
    x[5, :32] = np.linspace(-6.5, 6.5, 32)  # E2M1 ties and saturation at scale 1
    x[6, :32] = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0] * 4) * 4.0
    x[7, :32] = np.array([448.0, 464.0, 480.0, 500.0, 256.0, 300.0, 0.0, -1.0] * 4)
    return x


def main() -> None:
    rng = np.random.default_rng(20261201)
    # FP8 1x128, bf16 input, float32 arithmetic (quantize_state_dict path)
    x = plant_edges_rows(weights(rng, (64, 512)), rng)
    fp8_row_case("fp8_row_bf16_f32.npz", bf16(x), "bf16", native=False, pow2=False)
    fp8_row_case("fp8_row_bf16_f32_pow2.npz", bf16(x), "bf16", native=False, pow2=True)
    # bf16 arithmetic (quantize_tensor on a bf16 tensor); no NaN blocks: torch's
    # NaN bits there depend on vector vs scalar loop position
    xn = weights(rng, (64, 512))
    xn[0, :128] = 0.0
    xn[1, 3] = np.inf
    xn[3, :128] = np.float32(1e-40)
    fp8_row_case("fp8_row_bf16_native.npz", bf16(xn), "bf16", native=True, pow2=False)
    fp8_row_case("fp8_row_bf16_native_pow2.npz", bf16(xn), "bf16", native=True, pow2=True)
    # float32 input
    xf = plant_edges_rows(weights(rng, (32, 256)), rng)
    fp8_row_case("fp8_row_f32.npz", torch.from_numpy(xf), "f32", native=False, pow2=False)
    fp8_row_case("fp8_row_f32_pow2.npz", torch.from_numpy(xf), "f32", native=False, pow2=True)
    # float16 input, float32 and fp16 arithmetic
    xh = weights(rng, (32, 256))
    xh[0, :128] = 0.0
    xh[1, 3] = np.inf
    xh[2, 200] = np.nan
    xh[3, :128] = np.float32(1e-7)
    th = torch.from_numpy(xh).half()
    fp8_row_case("fp8_row_f16_f32.npz", th, "f16", native=False, pow2=False)
    fp8_row_case("fp8_row_f16_native.npz", th, "f16", native=True, pow2=False)

    # FP8 128x128 tiles, float32 arithmetic
    x = weights(rng, (384, 640))
    x[0:128, 0:128] = 0.0                      # zero tile
    x[0:128, 128:256][5, 7] = np.inf           # inf tile
    x[128:256, 0:128][9, 1] = np.nan           # NaN tile
    x[128:256, 128:256] = rng.normal(0, 1e-38, (128, 128))  # subnormal tile
    x[256:384, 512:640] *= 1e4                 # large tile
    fp8_tile_case("fp8_tile_bf16.npz", bf16(x))
    # pow2 of a NaN scale depends on torch's loop position (15 tiles are all
    # scalar tail); the NaN rule under pow2 is pinned by the 1x128 fixture
    xp = x.copy()
    xp[128:256, 0:128][9, 1] = 0.5
    fp8_tile_case("fp8_tile_bf16_pow2.npz", bf16(xp), pow2=True)
    fp8_tile_case("fp8_tile_ragged_bf16.npz", bf16(weights(rng, (200, 328))))
    # MoE expert stack [E, N, K] with a zero tile and an inf tile
    xe = weights(rng, (4, 256, 384))
    xe[1, 128:256, 0:128] = 0.0
    xe[2, 0:128, 256:384][17, 33] = np.inf
    fp8_tile_case("fp8_tile_experts_bf16.npz", bf16(xe))

    # dequant: every code, with f32 / bf16 scales incl. zero, inf, NaN
    codes = np.tile(np.arange(256, dtype=np.uint8), 4).reshape(8, 128)
    sc = np.array([[0.5], [1.0 / 448], [3.0e-3], [0.0], [np.inf], [np.nan], [1e-38], [2.0 ** 100]],
                  np.float32)
    qt = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    d32 = torch_ref.dequantize_tensor(qt, torch.from_numpy(sc), 128)
    sb = torch.from_numpy(sc).to(torch.bfloat16)
    dbf = torch_ref.dequantize_tensor(qt, sb, 128).to(torch.bfloat16)
    np.savez_compressed(os.path.join(OUT, "fp8_dequant.npz"), codes=codes, scales=sc,
                        scales_bf16=bits16(sb), out_f32=d32.numpy(), out_bf16=bits16(dbf))

    # MX
    xm = mx_inputs(rng)
    tb = bf16(xm)
    xmf = tb.float().numpy()
    for fmt, name in ((8, "mxfp8_bf16.npz"), (4, "mxfp4_bf16.npz")):
        c, s = mx_reference(xmf, fmt)
        np.savez_compressed(os.path.join(OUT, name), x=bits16(tb), codes=c, scales=s)
    xm32 = mx_inputs(rng)
    for fmt, name in ((8, "mxfp8_f32.npz"), (4, "mxfp4_f32.npz")):
        c, s = mx_reference(xm32, fmt)
        np.savez_compressed(os.path.join(OUT, name), x=xm32, codes=c, scales=s)
    write_f64_fixtures()
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))


if __name__ == "__main__":
    if sys.argv[1:] == ["f64"]:
        write_f64_fixtures()
    else:
        main()
