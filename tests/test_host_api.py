"""Host-side mirror of lumenrl/quantization (no GPU): config, validation, loud failure."""

from __future__ import annotations

import pytest
import torch

from lumenrl_amd import _lib
from lumenrl_amd.quantization import (
    FP8Config,
    QuantizationConfig,
    TrainingQuantConfig,
    WeightQuantizer,
    fp8_e4m3_max,
)


# tests/unit/quantization/test_fp8_config.py:7-29, against the mirror
def test_default_values():
    cfg = FP8Config()
    assert cfg.precision == "bf16"
    assert cfg.recipe == "blockwise"
    assert cfg.use_deep_gemm is True
    assert cfg.use_weight_pow2_scale is False
    assert cfg.is_fp8_enabled() is False


def test_from_config():
    q = QuantizationConfig()
    q.rollout.precision = "bf16"
    q.training = TrainingQuantConfig(fp8="e4m3", fp8_recipe="tensorwise")
    cfg = FP8Config.from_config(q)
    assert cfg.precision == "e4m3"
    assert cfg.recipe == "tensorwise"
    assert cfg.is_fp8_enabled() is True
    assert cfg.use_weight_pow2_scale is False


def test_is_fp8_enabled():
    assert FP8Config(precision="fp8").is_fp8_enabled() is True
    assert FP8Config(precision="hybrid_fp8").is_fp8_enabled() is True
    assert FP8Config(precision="bf16").is_fp8_enabled() is False
    assert FP8Config(precision=" E4M3 ").is_fp8_enabled() is True


def test_from_config_rejects_other_types():
    with pytest.raises(TypeError, match="QuantizationConfig"):
        FP8Config.from_config({"rollout": None})


def test_fp8_max():
    assert fp8_e4m3_max() == 448.0


def test_validation_errors_match_reference_texts():
    wq = WeightQuantizer(FP8Config())
    with pytest.raises(ValueError, match=r"quantize_tensor expects tensor.dim\(\) >= 1"):
        wq.quantize_tensor(torch.tensor(1.0))
    with pytest.raises(ValueError, match=r"Last dim 100 must be divisible by block_size=128"):
        wq.quantize_tensor(torch.zeros(2, 100))
    with pytest.raises(ZeroDivisionError):
        wq.quantize_tensor(torch.zeros(2, 100), block_size=0)


def _raised(fn):
    try:
        fn()
    except Exception as e:  # noqa: BLE001 - the type and text are what is compared
        return type(e), str(e)
    return None


@pytest.mark.parametrize("shape", [(4, 0), (0,), (0, 0), (2, 3, 0)])
@pytest.mark.parametrize("block_size", [128, 64, -128, 0])
def test_zero_width_rows_raise_as_the_reference(shape, block_size):
    """Zero-width rows pass the divisibility check and then reach the
    reference's ``unfold`` (weight_quantizer.py:51-59, :85-86), which raises
    RuntimeError; the drop-in raises the same error before any staging or
    device call (so this runs without a device).  ``[0, K]`` stays valid."""
    from oracle import torch_ref

    wq = WeightQuantizer(FP8Config())
    x = torch.zeros(shape)
    want = _raised(lambda: torch_ref.quantize_tensor(x, block_size))
    assert want is not None and want[0] in (RuntimeError, ZeroDivisionError)
    assert _raised(lambda: wq.quantize_tensor(x, block_size)) == want
    q = torch.zeros(shape, dtype=torch.float8_e4m3fn)
    s = torch.zeros(shape[:-1] + (0,))
    want = _raised(lambda: torch_ref.dequantize_tensor(q, s, block_size))
    assert want is not None and want[0] is RuntimeError
    assert _raised(lambda: wq.dequantize_tensor(q, s, block_size)) == want


def test_zero_width_state_dict_entry_raises_as_the_reference():
    """A [N, 0] float weight passes quantize_state_dict's `in_features % 128`
    rule (:105) and raises in quantize_tensor (:109); a [N, 0] codes entry with
    its sidecar raises in dequantize_tensor (:132).  Both before any device work."""
    from oracle import torch_ref

    wq = WeightQuantizer(FP8Config())
    sd = {"step": 1, "w": torch.zeros(4, 0)}
    want = _raised(lambda: torch_ref.quantize_state_dict(sd))
    assert want is not None and want[0] is RuntimeError
    assert _raised(lambda: wq.quantize_state_dict(sd)) == want
    qsd = {"w": torch.zeros(4, 0, dtype=torch.float8_e4m3fn), "w_fp8_scales": torch.zeros(4, 0)}
    want = _raised(lambda: torch_ref.dequantize_state_dict(qsd))
    assert want is not None and want[0] is RuntimeError
    assert _raised(lambda: wq.dequantize_state_dict(qsd)) == want


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device failure")
def test_zero_rows_stay_valid_without_reaching_unfold_errors():
    """[0, K] is a valid input in the reference; the drop-in gets past the
    unfold checks to its device requirement (no device here)."""
    wq = WeightQuantizer(FP8Config())
    with pytest.raises(RuntimeError, match="HIP device"):
        wq.quantize_tensor(torch.zeros(0, 256))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device failure")
def test_no_device_fails_loudly():
    wq = WeightQuantizer(FP8Config())
    with pytest.raises(RuntimeError, match="HIP device"):
        wq.quantize_tensor(torch.zeros(2, 128))
    with pytest.raises(RuntimeError, match="HIP device"):
        wq.quantize_state_dict({"w": torch.zeros(4, 128)})


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/liblrq.so")
    with pytest.raises(_lib.LrqError, match="no non-HIP fallback"):
        _lib.lib()


def test_state_dict_passthrough_rules_without_device():
    """Entries the reference passes through never touch the device (:95-108)."""
    wq = WeightQuantizer(FP8Config())
    sd = {"step": 3, "ids": torch.arange(4), "bias": torch.zeros(128), "odd": torch.zeros(4, 100)}
    out = wq.quantize_state_dict(sd)
    assert list(out) == list(sd)
    for k in sd:
        assert out[k] is sd[k]


# matrix_view: the stride analysis every launch relies on (CPU tensors, no device)
from hypothesis import given, settings, strategies as st  # noqa: E402

from lumenrl_amd.quantization.ops import matrix_view  # noqa: E402


@st.composite
def _views(draw):
    """Random views of a random buffer: slices, steps, transposes, expands, 1-3 dims."""
    ndim = draw(st.integers(1, 3))
    shape = [draw(st.integers(1, 9)) for _ in range(ndim)]
    base = torch.arange(1, 1 + 4 * 9 * 9 * 9, dtype=torch.float32)
    pads = [draw(st.integers(0, 3)) for _ in range(ndim)]
    full = [s + p for s, p in zip(shape, pads)]
    t = base[: int(torch.tensor(full).prod())].view(*full)
    idx = tuple(slice(draw(st.integers(0, p)), None) for p in pads)
    t = t[idx]
    t = t[tuple(slice(0, s) for s in shape)]
    if ndim >= 2 and draw(st.booleans()):
        t = t.transpose(-1, -2)
    if draw(st.booleans()):
        t = t.unsqueeze(0).expand(draw(st.integers(1, 3)), *t.shape)
    return t


@settings(max_examples=300, deadline=None)
@given(_views())
def test_matrix_view_addresses_exactly_the_tensor(t):
    xb, batch, rows, cols, ld, bstride = matrix_view(t)
    want = t.reshape(-1, t.shape[-1])
    lead = 1
    for d in t.shape[:-2]:
        lead *= d
    assert (batch, rows, cols) == (lead, t.shape[-2] if t.dim() >= 2 else 1, t.shape[-1])
    # rebuild every element from (pointer, batch, rows, cols, ld, bstride) over xb's storage
    flat = xb.reshape(-1) if xb.data_ptr() != t.data_ptr() else None
    esz = t.element_size()
    got = torch.empty(batch, rows, cols)
    if flat is None:
        # in place: offsets relative to t's first element inside its storage
        storage = torch.as_strided(t, (t.untyped_storage().nbytes() // esz - t.storage_offset(),), (1,))
        assert cols == 1 or xb.stride(-1) == 1
        for b in range(batch):
            for r in range(rows):
                o = b * bstride + r * ld
                got[b, r] = storage[o:o + cols]
    else:
        # a dense copy: ld == cols, bstride == rows * cols
        assert ld == cols and bstride == rows * cols
        got = flat.view(batch, rows, cols)
    assert torch.equal(got.reshape(-1, cols), want.reshape(-1, cols))
    # matrices never overlap and rows never overlap
    assert rows == 1 or ld >= cols
    assert batch == 1 or bstride >= (rows - 1) * ld + cols


# transfer-bucket layout (pure host arithmetic)
from lumenrl_amd.quantization.bucket import entry_sizes, plan_layout  # noqa: E402


@st.composite
def _weight_lists(draw):
    fmt = draw(st.sampled_from(["fp8_block", "mxfp8", "mxfp4"]))
    n = draw(st.integers(1, 12))
    ws = []
    for i in range(n):
        q = draw(st.booleans())
        if q:
            lead = tuple(draw(st.lists(st.integers(1, 3), max_size=1)))
            shape = lead + (draw(st.integers(1, 300)), 32 * draw(st.integers(1, 40)))
        else:
            shape = tuple(draw(st.lists(st.integers(1, 300), min_size=1, max_size=2)))
        ws.append((f"w{i}", shape, draw(st.sampled_from([torch.bfloat16, torch.float32])), q))
    return fmt, ws


@settings(max_examples=300, deadline=None)
@given(_weight_lists(), st.integers(1 << 12, 1 << 20))
def test_bucket_layout_properties(fw, bucket_bytes):
    fmt, ws = fw
    need = {n: sum((e[2] + 255) // 256 * 256 for e in entry_sizes(s, d, q, fmt, (128, 128)))
            for n, s, d, q in ws}
    if max(need.values()) > bucket_bytes:
        with pytest.raises(ValueError, match="more than the bucket"):
            plan_layout(ws, bucket_bytes, fmt)
        return
    layouts = plan_layout(ws, bucket_bytes, fmt)
    # every weight once, in order; quantized ones bring their scale entry
    assert [n for lay in layouts for n, _ in lay.items] == [n for n, *_ in ws]
    for lay in layouts:
        assert lay.nbytes <= bucket_bytes
        end = 0
        for e in lay.entries:
            assert e.offset % 256 == 0 and e.offset >= end  # aligned, in order, no overlap
            end = e.offset + e.nbytes
        assert end <= lay.nbytes
        names = [e.name for e in lay.entries]
        for n, q in lay.items:
            assert (n + "_scale_inv" in names) == q
    # greedy: a bucket closes only when the next weight would not fit
    for a, b in zip(layouts, layouts[1:]):
        assert a.nbytes + need[b.items[0][0]] > bucket_bytes
    # codes/scale sizes of each format
    for n, s, d, q in ws:
        if not q:
            continue
        (cs, cdt, cn), (ss, sdt, sn) = entry_sizes(s, d, True, fmt, (128, 128))
        rows, cols = s[-2], s[-1]
        lead = 1
        for x in s[:-2]:
            lead *= x
        if fmt == "fp8_block":
            assert cn == lead * rows * cols and sn == 4 * lead * -(-rows // 128) * -(-cols // 128)
        else:
            assert cn == lead * rows * (cols if fmt == "mxfp8" else cols // 2)
            assert sn == lead * rows * (cols // 32) and sdt == torch.uint8


from lumenrl_amd.quantization.ops import launch_chunks  # noqa: E402


@given(st.integers(min_value=0, max_value=1000))
@settings(max_examples=60, deadline=None)
def test_launch_chunks_cover_every_item_once_in_order(n):
    """The drop-ins' launch slices: 8, 16, 32, then 64 items, in order, none lost."""
    items = list(range(n))
    chunks = list(launch_chunks(items))
    assert [x for c in chunks for x in c] == items
    sizes = [len(c) for c in chunks]
    want = []
    left, k = n, 8
    while left > 0:
        want.append(min(k, left))
        left -= k
        k = min(2 * k, 64)
    assert sizes == want


from lumenrl_amd.quantization.ops import GROUP_LAUNCH_BYTES, launch_ranges  # noqa: E402


@given(st.lists(st.integers(min_value=0, max_value=5000), max_size=60), st.integers(min_value=1, max_value=6000))
@settings(max_examples=200, deadline=None)
def test_launch_ranges_split_plans_into_maximal_runs(sizes, limit):
    """A grouped plan's launches: consecutive runs of whole tensors covering
    every tensor once, in order; each run within the byte limit unless it is a
    single larger tensor, and no run could take the next tensor too."""
    rs = launch_ranges(sizes, limit)
    assert [k for i, j in rs for k in range(i, j)] == list(range(len(sizes)))
    for n, (i, j) in enumerate(rs):
        assert j > i
        assert sum(sizes[i:j]) <= limit or j - i == 1
        if n + 1 < len(rs):
            assert sum(sizes[i:j + 1]) > limit


def test_launch_ranges_of_the_qwen3_8b_set():
    """The 252 Qwen3-8B linears (128x128 FP8: 3 bytes per element plus scales)
    split into 7 launches of consecutive tensors under the default limit."""
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096),
              (4096, 12288)] * 36
    sizes = [3 * r * c + 4 * (r // 128) * (c // 128) for r, c in shapes]
    rs = launch_ranges(sizes)
    assert len(rs) == 7 and all(sum(sizes[i:j]) <= GROUP_LAUNCH_BYTES for i, j in rs)


from lumenrl_amd.quantization.ops import ChunkedLaunches  # noqa: E402


def test_chunked_launches_schedule_and_results():
    """Groups launch 8, 16, 32, then 64 items each, as soon as a chunk is full;
    results map every name to its own output; groups never mix."""
    calls = []

    def run(items):
        calls.append(list(items))
        return [x * 10 for x in items]

    cl = ChunkedLaunches(run)
    for i in range(150):
        cl.add("a" if i % 3 else "b", f"n{i}", i)
        if i == 30:
            assert [len(c) for c in calls] == [8, 8]  # a: 8 of 20 so far; b: 8 of 11
    res = cl.flush()
    assert res == {f"n{i}": i * 10 for i in range(150)}
    a_sizes = [len(c) for c in calls if c[0] % 3]
    b_sizes = [len(c) for c in calls if c[0] % 3 == 0]
    assert a_sizes == [8, 16, 32, 44] and b_sizes == [8, 16, 26]
    assert all(len({x % 3 == 0 for x in c}) == 1 for c in calls)


def test_host_windows_split_in_order_and_keep_big_items_whole():
    from lumenrl_amd.quantization.ops import _windows

    t = {n: torch.empty(n, dtype=torch.uint8) for n in (10, 30, 60, 100, 5, 5)}
    items = [(f"k{i}", (t[n],)) for i, n in enumerate([30, 60, 10, 100, 5, 5, 60, 30])]
    wins = [[k for k, _ in w] for w in _windows(items, 100)]
    assert wins == [["k0", "k1", "k2"], ["k3"], ["k4", "k5", "k6", "k7"]]
    assert [k for w in wins for k in w] == [k for k, _ in items]
    # an item larger than the window is a window of its own
    big = [("a", (t[5],)), ("b", (torch.empty(500, dtype=torch.uint8),)), ("c", (t[5],))]
    assert [[k for k, _ in w] for w in _windows(big, 100)] == [["a"], ["b"], ["c"]]
    # several inputs per item count together
    pairs = [("p", (t[60], t[30])), ("q", (t[10], t[5]))]
    assert [[k for k, _ in w] for w in _windows(pairs, 100)] == [["p"], ["q"]]


def test_host_items_split_rows_and_map_outputs():
    from lumenrl_amd.quantization.ops import host_items

    x = torch.zeros(1000, 64, dtype=torch.bfloat16)          # 128,000 bytes
    codes = torch.zeros(1000, 64, dtype=torch.uint8)
    sc = torch.zeros(1000, 1, dtype=torch.bfloat16)
    whole = host_items("w", (x,), (codes, sc), window_bytes=1 << 20)
    assert len(whole) == 1 and whole[0][0] == "w" and whole[0][2][0] is codes
    parts = host_items("w", (x,), (codes, sc), window_bytes=16_000)  # 125 rows per window
    assert [k for k, _, _ in parts] == [("w", r) for r in range(0, 1000, 125)]
    for (_, r0), ins, outs in parts:
        n = ins[0].shape[0]
        assert n == min(125, 1000 - r0)
        assert ins[0].data_ptr() == x[r0].data_ptr()
        assert outs[0].data_ptr() == codes[r0].data_ptr() and outs[0].shape[0] == n
        assert outs[1].data_ptr() == sc[r0].data_ptr() and outs[1].shape[0] == n
    # 128-row tiles: chunks of whole tile rows; scales have ceil(rows / 128) rows
    t = torch.zeros(1000, 256, dtype=torch.bfloat16)          # 512 bytes per row
    tc = torch.zeros(1000, 256, dtype=torch.uint8)
    ts = torch.zeros(8, 2, dtype=torch.float32)
    parts = host_items("t", (t,), (tc, ts), window_bytes=300 * 512, multiple=128, out_div=(1, 128))
    assert [k[1] for k, _, _ in parts] == [0, 256, 512, 768]
    assert [o[1].shape[0] for _, _, o in parts] == [2, 2, 2, 2]
    assert [i[0].shape[0] for _, i, _ in parts] == [256, 256, 256, 232]
    assert parts[-1][2][1].data_ptr() == ts[6].data_ptr()
    with pytest.raises(ValueError):
        host_items("t", (t,), (tc, ts), window_bytes=300 * 512, multiple=100, out_div=(1, 128))
