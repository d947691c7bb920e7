"""The C-ABI library (no GPU needed): loads, exports include/lrq.h, host-side logic.

Only calls that return before touching the HIP runtime are made here:
argument validation and the grouped-table packer, which works on host memory.
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT
from lumenrl_amd import _lib

HEADER = os.path.join(ROOT, "include", "lrq.h")


def declared_functions() -> list[str]:
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(lrq_[a-z0-9_]+)\s*\(", txt)))


def test_library_built_and_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() / make -C lumen-rl_amd"
    L = ctypes.CDLL(_lib.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing
    # the Python binding declares a signature for each of them
    assert sorted(_lib.SIGNATURES) == names


def test_library_targets_gfx950_only():
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert other not in blob


def test_version():
    assert _lib.version().startswith("lrq ") and "gfx950" in _lib.version()


def L():
    return _lib.lib()


def test_argument_errors_need_no_device():
    fake = ctypes.c_void_p(0x10000)
    # bad dtype
    rc = L().lrq_fp8_block_quant(fake, 7, 1, 4, 128, 128, 512, 1, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG and "dtype" in _lib.last_error()
    # negative extent
    rc = L().lrq_fp8_block_quant(fake, 0, 1, -4, 128, 128, 512, 1, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG
    # ld < cols
    rc = L().lrq_fp8_block_quant(fake, 0, 1, 4, 128, 64, 512, 1, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG and "ld" in _lib.last_error()
    # null pointer with work to do
    rc = L().lrq_fp8_block_quant(None, 0, 1, 4, 128, 128, 512, 1, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG
    # bad block
    rc = L().lrq_fp8_block_quant(fake, 0, 1, 4, 128, 128, 512, 0, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG
    # MX needs cols % 32
    rc = L().lrq_mxfp8_quant(fake, 0, 4, 48, 48, fake, fake, None)
    assert rc == _lib.ERR_ARG and "32" in _lib.last_error()
    rc = L().lrq_mxfp4_quant(fake, 9, 4, 64, 64, fake, fake, None)
    assert rc == _lib.ERR_ARG
    # dequant dtypes
    rc = L().lrq_fp8_block_dequant(fake, fake, 5, 1, 4, 128, 1, 128, fake, 2, None)
    assert rc == _lib.ERR_ARG
    rc = L().lrq_fp8_block_dequant(fake, fake, 2, 1, 4, 128, 1, 128, fake, 1, None)
    assert rc == _lib.ERR_ARG
    # empty work is a no-op success (no launch)
    rc = L().lrq_fp8_block_quant(None, 0, 1, 0, 128, 128, 0, 1, 128, None, None, 0, None)
    assert rc == 0
    # diagnostics
    assert L().lrq_diag_e4m3_bits(0, 6, fake, None) == _lib.ERR_ARG


def _tensors(shapes, base=0x100000000, align=256):
    arr = (_lib.LrqTensor * len(shapes))()
    p = base
    for i, (b, r, c) in enumerate(shapes):
        arr[i].in_ = p
        p += b * r * c * 2 + align
        arr[i].codes = p
        p += b * r * c + align
        arr[i].scales = p
        p += b * r * c + align
        arr[i].batch, arr[i].rows, arr[i].cols = b, r, c
        arr[i].ld, arr[i].batch_stride = c, r * c
    return arr


QWEN3_8B_LAYER = [(1, 4096, 4096), (1, 1024, 4096), (1, 1024, 4096), (1, 4096, 4096),
                  (1, 12288, 4096), (1, 12288, 4096), (1, 4096, 12288)]


def _pack(fmt, shapes, blk=(128, 128), flags=0, dtype=0):
    ts = _tensors(shapes)
    need = L().lrq_group_table_bytes(fmt, ts, len(shapes), dtype, blk[0], blk[1], flags)
    assert need > 0, _lib.last_error()
    buf = np.zeros(need, np.uint8)
    rc = L().lrq_group_pack(fmt, ts, len(shapes), dtype, blk[0], blk[1], flags, buf.ctypes.data, need)
    assert rc == 0, _lib.last_error()
    return buf


def test_group_pack_tiles_qwen3_layer():
    buf = _pack(_lib.FMT_FP8_BLOCK, QWEN3_8B_LAYER)
    units = L().lrq_group_units(buf.ctypes.data)
    tiles = [(r // 128) * (c // 128) for _, r, c in QWEN3_8B_LAYER]
    assert units == sum(tiles)
    # host table: a 256-byte header, then one 112-byte descriptor per tensor whose
    # work-groups [unit0, unit0 + units) follow table order (the device map relies on it)
    assert buf.size == 256 + -(-7 * 112 // 256) * 256
    d = buf[256:256 + 7 * 112].view(np.int64).reshape(7, 14)
    assert np.array_equal(d[:, 8], np.cumsum([0] + tiles[:-1])) and np.array_equal(d[:, 9], tiles)
    # each tile descriptor carries the log2 of its XCD run: 4 tiles for rows of
    # a multiple of 8 KiB (every tensor here)
    assert np.all(d[:, 13] == 2)
    # the device table adds 4 bytes of work-group -> tensor map per work-group
    assert L().lrq_group_device_bytes(buf.ctypes.data) == buf.size + 4 * units
    assert L().lrq_group_device_bytes(None) == _lib.ERR_ARG
    assert L().lrq_group_build_map(None, None, None) == _lib.ERR_ARG
    # a device table off its 256-byte alignment is refused before any launch
    assert L().lrq_group_build_map(buf.ctypes.data, ctypes.c_void_p(0x1000 + 64), None) == _lib.ERR_ALIGN
    assert "256-byte" in _lib.last_error()


def test_group_pack_rows_and_mx_units():
    shapes = [(1, 256, 4096), (1, 64, 12288)]
    buf = _pack(_lib.FMT_FP8_BLOCK, shapes, (1, 128))
    blocks = 256 * 32 + 64 * 96
    # 1x128 rows: 16 lanes per block, 4 blocks per wave instruction, 64 blocks per work-group
    assert L().lrq_group_units(buf.ctypes.data) == -(-256 * 32 // 64) + -(-64 * 96 // 64)
    buf = _pack(_lib.FMT_MXFP4, shapes, (1, 32))
    # MX: 64 lanes of a wave, a quad per group, 2 groups per quad -> 128 groups per work-group
    assert L().lrq_group_units(buf.ctypes.data) == -(-256 * 128 // 128) + -(-64 * 384 // 128)
    del blocks
    # other widths: 1x8 and 1x16 take 1- and 2-lane groups, wider ones the next
    # power of two of B/8 lanes (4 at least); 4 waves x 4 instructions per work-group
    for B, lanes in ((8, 1), (16, 2), (24, 4), (40, 8), (96, 16), (200, 32), (504, 64),
                     (12, 2), (36, 8), (100, 16), (500, 64)):  # ceil(B/8) chunks when 8 does not divide B
        shapes = [(1, 256, 16 * B), (1, 63, 3 * B)]
        buf = _pack(_lib.FMT_FP8_BLOCK, shapes, (1, B))
        per_wg = 4 * 4 * (64 // lanes)
        assert L().lrq_group_units(buf.ctypes.data) == -(-256 * 16 // per_wg) + -(-63 * 3 // per_wg), B
    # wider blocks: 4 waves of 2 or 1 blocks (B <= 1024, 2048), blocks of 2
    # waves (B <= 4096) or 4 (B <= 16384), with 4 chunk slots per lane; with 8
    # slots, one wave per block at B = 4096 and 4 waves per block past 6144
    # (16-bit) or 8192; 1024 and 2048 stay on the row kernel
    for dt, cases in ((0, ((640, 8), (1032, 4), (1536, 4), (3072, 2), (4096, 4), (4104, 1), (6144, 1),
                           (8192, 1), (16384, 1), (1000, 8), (3001, 2), (9999, 1))),
                      (_lib.DTYPE_F32, ((640, 8), (1000, 8), (1536, 4), (3072, 2), (4096, 4),
                                        (4104, 1), (8192, 1), (8200, 1)))):
        for B, per_wg in cases:
            buf = _pack(_lib.FMT_FP8_BLOCK, [(1, 256, 16 * B), (1, 72, 3 * B)], (1, B), dtype=dt)
            assert L().lrq_group_units(buf.ctypes.data) == -(-256 * 16 // per_wg) + -(-72 * 3 // per_wg), B
    # past 16384, one block of 8 or 16 waves per work-group up to 65536
    for B in (16392, 18944, 32768, 65536):
        buf = _pack(_lib.FMT_FP8_BLOCK, [(1, 8, 2 * B), (1, 3, B)], (1, B))
        assert L().lrq_group_units(buf.ctypes.data) == 8 * 2 + 3, B
    # widths under 8 and past 65536 take the generic kernel: one work-group per block
    for B in (5, 7, 65544):
        buf = _pack(_lib.FMT_FP8_BLOCK, [(1, 4, 2 * B)], (1, B))
        assert L().lrq_group_units(buf.ctypes.data) == 4 * 2, B


def test_group_pack_expert_stack_single_descriptor():
    buf = _pack(_lib.FMT_FP8_BLOCK, [(128, 768, 2048), (128, 2048, 768)])
    assert L().lrq_group_units(buf.ctypes.data) == 128 * 6 * 16 + 128 * 16 * 6


def test_group_kernel_ids_tell_tables_apart():
    """lrq_group_kernel: equal ids for tables of the same kernel, different ids
    for the tile kernel and the generic one (K % 8 != 0); errors as the other
    table readers."""
    tile_a = _pack(_lib.FMT_FP8_BLOCK, [(1, 256, 256)])
    tile_b = _pack(_lib.FMT_FP8_BLOCK, [(2, 128, 4096), (1, 300, 1024)])
    generic = _pack(_lib.FMT_FP8_BLOCK, [(1, 256, 300)])
    rows = _pack(_lib.FMT_FP8_BLOCK, [(1, 256, 256)], (1, 128))
    ids = [L().lrq_group_kernel(b.ctypes.data) for b in (tile_a, tile_b, generic, rows)]
    assert min(ids) >= 0 and ids[0] == ids[1] and len({ids[0], ids[2], ids[3]}) == 3
    assert L().lrq_group_kernel(None) == _lib.ERR_ARG
    assert L().lrq_group_kernel(np.zeros(256, np.uint8).ctypes.data) == _lib.ERR_TABLE


def test_tile_xcd_run_follows_the_row_pitch():
    """k_tile128 descriptors: runs of 4 tiles (log2 2) when a row spans a
    multiple of 8 KiB of input, runs of 8 (log2 3) for any other pitch."""
    def runs(shapes, dtype=0, ld=None):
        ts = _tensors(shapes)
        if ld is not None:
            for t, l in zip(ts, ld):
                t.ld, t.batch_stride = l, t.rows * l
        need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, ts, len(shapes), dtype, 128, 128, 0)
        buf = np.zeros(need, np.uint8)
        assert L().lrq_group_pack(_lib.FMT_FP8_BLOCK, ts, len(shapes), dtype, 128, 128, 0,
                                  buf.ctypes.data, need) == 0, _lib.last_error()
        return list(buf[256:256 + len(shapes) * 112].view(np.int64).reshape(-1, 14)[:, 13])
    # bf16: 8 KiB (K = 4096), 24 KiB, 4 KiB (K = 2048), 1.5 KiB (K = 768), 2 KiB
    assert runs([(1, 256, 4096), (1, 256, 12288), (2, 256, 2048), (2, 256, 768), (1, 300, 1024)]) == [2, 2, 3, 3, 3]
    # float32 input: K = 2048 rows are 8 KiB
    assert runs([(1, 256, 2048), (1, 256, 768)], dtype=_lib.DTYPE_F32) == [2, 3]
    # the pitch counts, not the width: K = 2048 views of K = 4096 rows keep runs of 4
    assert runs([(1, 256, 2048), (1, 256, 2048)], ld=[4096, 3072]) == [2, 3]


def test_group_pack_rejects_mixed_kernels_and_small_buffers():
    ts = _tensors([(1, 256, 256), (1, 256, 256)])
    ts[1].in_ = ts[1].in_ + 2  # element-aligned, off 16 bytes: the same tile kernel
    assert L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, ts, 2, 0, 128, 128, 0) > 0, _lib.last_error()
    ts[1].codes = ts[1].codes + 1  # codes off a lane's 8-byte chunk: the generic kernel
    need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, ts, 2, 0, 128, 128, 0)
    assert need == _lib.ERR_ARG and "kernel" in _lib.last_error()
    ts = _tensors([(1, 256, 256)])
    need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, ts, 1, 0, 128, 128, 0)
    buf = np.zeros(need - 1, np.uint8)
    rc = L().lrq_group_pack(_lib.FMT_FP8_BLOCK, ts, 1, 0, 128, 128, 0, buf.ctypes.data, need - 1)
    assert rc == _lib.ERR_CAPACITY


def test_tensor_scale_tables():
    """Per-tensor scale tables: 8 KiB units (16-byte loads) or 8192-element units
    (element walk) in one table, no codes pointer, workspace of 4 B per unit."""
    qkv = [(1, 4096, 4096), (1, 1024, 4096), (1, 1024, 4096)]
    ts = _tensors(qkv + [(1, 300, 100)])
    for t in ts:
        t.codes = None
    ts[3].in_ = ts[3].in_ + 2  # 100 columns (not whole 16-byte chunks): element walk
    fmt = _lib.FMT_TENSOR_SCALE
    need = L().lrq_group_table_bytes(fmt, ts, 4, 0, 1, 1, 0)
    assert need > 0, _lib.last_error()
    buf = np.zeros(need, np.uint8)
    assert L().lrq_group_pack(fmt, ts, 4, 0, 1, 1, 0, buf.ctypes.data, need) == 0, _lib.last_error()
    units = [4096 * 4096 // 4096, 1024 * 4096 // 4096, 1024 * 4096 // 4096, -(-300 * 100 // 8192)]
    assert L().lrq_group_units(buf.ctypes.data) == sum(units)
    assert L().lrq_group_workspace_bytes(buf.ctypes.data) == 4 * sum(units)
    d = buf[256:256 + 4 * 112].view(np.int64).reshape(4, 14)
    assert np.array_equal(d[:, 8], np.cumsum([0] + units[:-1])) and np.array_equal(d[:, 9], units)
    assert L().lrq_group_device_bytes(buf.ctypes.data) == need + 4 * sum(units)
    # argument errors are reported before any device work
    assert L().lrq_quant_grouped(buf.ctypes.data, buf.ctypes.data, None) == _lib.ERR_ARG
    assert "workspace" in _lib.last_error()
    small = 4 * sum(units) - 4
    rc = L().lrq_tensor_scale_grouped(buf.ctypes.data, buf.ctypes.data, ctypes.c_void_p(0x1000), small, None)
    assert rc == _lib.ERR_CAPACITY
    rc = L().lrq_tensor_scale_grouped(buf.ctypes.data, buf.ctypes.data, None, 1 << 20, None)
    assert rc == _lib.ERR_ARG
    fp8 = _pack(_lib.FMT_FP8_BLOCK, qkv)
    assert L().lrq_group_workspace_bytes(fp8.ctypes.data) == 0
    rc = L().lrq_tensor_scale_grouped(fp8.ctypes.data, fp8.ctypes.data, ctypes.c_void_p(0x1000), 1 << 20, None)
    assert rc == _lib.ERR_ARG and "not a tensor-scale table" in _lib.last_error()
    # an empty tensor has no max (torch's max() raises)
    ts = _tensors([(1, 0, 128)])
    assert L().lrq_group_table_bytes(fmt, ts, 1, 0, 1, 1, 0) == _lib.ERR_ARG
    assert "empty" in _lib.last_error()


def test_huge_extents_rejected_before_any_device_work():
    big = ctypes.c_void_p(0x10000)
    rc = L().lrq_fp8_block_quant(big, 0, 1, 1 << 40, 1 << 20, 1 << 20, 1 << 60, 128, 128, big, big, 0, None)
    assert rc == _lib.ERR_ARG and "2^48" in _lib.last_error()
    rc = L().lrq_fp8_block_quant(big, 0, 1 << 30, 4096, 4096, 4096, 4096 * 4096, 128, 128, big, big, 0, None)
    assert rc == _lib.ERR_ARG
    rc = L().lrq_fp8_block_dequant(big, big, 2, 1, 1 << 62, 1 << 4, 1, 128, big, 2, None)
    assert rc == _lib.ERR_ARG
    rc = L().lrq_mxfp8_quant(big, 0, 1 << 62, 64, 1 << 3, big, big, None)
    assert rc == _lib.ERR_ARG
    rc = L().lrq_act_qdq(big, 0, 1 << 40, 1 << 20, 1 << 20, 128, 0, big, None)
    assert rc == _lib.ERR_ARG and "2^48" in _lib.last_error()


def test_c_caller_is_built_against_the_in_tree_libraries():
    import subprocess

    from conftest import ROOT

    binary = os.path.join(ROOT, "tests", "c_abi", "_build", "test_abi_c")
    if not os.path.exists(binary):
        pytest.skip("tests/c_abi not built (run __graft_entry__.build())")
    deps = subprocess.run(["ldd", binary], capture_output=True, text=True).stdout
    assert "lumen-rl_amd/lumenrl_amd/liblrq.so" in deps
    assert "oracle/_build/liblrq_oracle.so" in deps


def test_copy_tables():
    """Grouped byte copies: 4 KiB units, NULL scales allowed, alignment and
    single-run checks before any device work."""
    fmt = _lib.FMT_COPY
    sizes = [16384 * 3, 200, 16384 + 17, 1]
    ts = (_lib.LrqTensor * len(sizes))()
    base = 0x100000
    for i, n in enumerate(sizes):
        ts[i].in_, ts[i].codes, ts[i].scales = base, base + (1 << 24), None
        ts[i].batch, ts[i].rows, ts[i].cols, ts[i].ld, ts[i].batch_stride = 1, 1, n, n, n
        base += 1 << 20
    need = L().lrq_group_table_bytes(fmt, ts, len(sizes), 0, 1, 1, 0)
    assert need > 0, _lib.last_error()
    buf = np.zeros(need, np.uint8)
    assert L().lrq_group_pack(fmt, ts, len(sizes), 0, 1, 1, 0, buf.ctypes.data, need) == 0
    assert L().lrq_group_units(buf.ctypes.data) == sum(-(-n // 4096) for n in sizes)
    assert L().lrq_group_workspace_bytes(buf.ctypes.data) == 0
    ts[1].in_ = ts[1].in_ + 8
    assert L().lrq_group_table_bytes(fmt, ts, len(sizes), 0, 1, 1, 0) == _lib.ERR_ALIGN
    ts[1].in_ = ts[1].in_ - 8
    ts[2].rows = 2
    assert L().lrq_group_table_bytes(fmt, ts, len(sizes), 0, 1, 1, 0) == _lib.ERR_ARG


def test_group_units_rejects_null_and_foreign_tables():
    assert L().lrq_group_units(None) == _lib.ERR_ARG and "null" in _lib.last_error()
    junk = np.zeros(4096, np.uint8)
    assert L().lrq_group_units(junk.ctypes.data) == _lib.ERR_TABLE
    assert L().lrq_group_device_bytes(junk.ctypes.data) == _lib.ERR_TABLE
    assert L().lrq_group_build_map(junk.ctypes.data, ctypes.c_void_p(0x1000), None) == _lib.ERR_TABLE


def test_cast_tables():
    """Unscaled e4m3 cast tables: one contiguous run per tensor, 4096 elements
    per work-group; the vector path needs a 16-byte aligned input and codes
    aligned to one chunk (8 bytes for 16-bit input, 4 for float32)."""
    fmt = _lib.FMT_CAST_E4M3
    ts = _tensors([(1, 1, 10000), (1, 1, 4096), (1, 1, 7), (1, 1, 0)])
    for i, t in enumerate(ts):
        t.in_, t.codes, t.scales = 0x200000000 + i * 0x100000, 0x300000000 + i * 0x100000, None
    ts[1].codes = ts[1].codes + 4  # codes only 4-byte aligned: element walk for bf16
    need = L().lrq_group_table_bytes(fmt, ts, 4, 0, 1, 1, 0)
    assert need > 0, _lib.last_error()
    buf = np.zeros(need, np.uint8)
    assert L().lrq_group_pack(fmt, ts, 4, 0, 1, 1, 0, buf.ctypes.data, need) == 0, _lib.last_error()
    assert L().lrq_group_units(buf.ctypes.data) == 3 + 1 + 1 + 0
    descs = buf[256:256 + 4 * 112].view(np.int64).reshape(4, 14)  # 112-byte descriptors
    assert descs[:3, 10].tolist() == [1, 0, 1]  # vector-path flag (units_c)
    assert descs[:, 9].tolist() == [3, 1, 1, 0]   # work-groups per tensor
    # float32 input: 4-byte aligned codes are enough
    need32 = L().lrq_group_table_bytes(fmt, ts, 2, _lib.DTYPE_F32, 1, 1, 0)
    buf32 = np.zeros(need32, np.uint8)
    assert L().lrq_group_pack(fmt, ts, 2, _lib.DTYPE_F32, 1, 1, 0, buf32.ctypes.data, need32) == 0
    assert buf32[256:256 + 2 * 112].view(np.int64).reshape(2, 14)[:, 10].tolist() == [1, 1]
    # a cast entry is one run; the single-tensor call checks its arguments first
    ts2 = _tensors([(1, 4, 64)])
    assert L().lrq_group_table_bytes(fmt, ts2, 1, 0, 1, 1, 0) == _lib.ERR_ARG
    fake = ctypes.c_void_p(0x10000)
    assert L().lrq_cast_e4m3(fake, 0, -1, fake, None) == _lib.ERR_ARG
    assert L().lrq_cast_e4m3(None, 0, 16, fake, None) == _lib.ERR_ARG
    assert L().lrq_cast_e4m3(fake, 5, 16, fake, None) == _lib.ERR_ARG
    assert L().lrq_cast_e4m3(None, 0, 0, None, None) == 0  # nothing to do, no launch


def test_mx_dequant_tables():
    """MX dequant: dense [rows, cols] codes, 2 lane-chunks of 8 (bf16 out) or 4
    (fp32 out) elements per lane, 256 lanes per work-group; codes aligned to one
    lane-chunk of codes, output to 16 bytes."""
    ts = _tensors([(1, 64, 1024), (2, 32, 512)])
    for i, t in enumerate(ts):
        t.in_, t.codes, t.scales = 0x200000000 + i * 0x100000, 0x300000000 + i * 0x100000, 0x400000000
    for fmt in (_lib.FMT_MXFP8_DEQUANT, _lib.FMT_MXFP4_DEQUANT):
        for flags, cpc in ((_lib.FLAG_OUT_BF16, 8), (0, 4)):
            need = L().lrq_group_table_bytes(fmt, ts, 2, 0, 1, 32, flags)
            assert need > 0, _lib.last_error()
            buf = np.zeros(need, np.uint8)
            assert L().lrq_group_pack(fmt, ts, 2, 0, 1, 32, flags, buf.ctypes.data, need) == 0
            units = [-(-64 * 1024 // cpc // 512), -(-2 * 32 * 512 // cpc // 512)]
            assert L().lrq_group_units(buf.ctypes.data) == sum(units)
    ts[1].in_ = ts[1].in_ + 3  # codes at any byte offset
    assert L().lrq_group_table_bytes(_lib.FMT_MXFP8_DEQUANT, ts, 2, 0, 1, 32, 0) > 0, _lib.last_error()
    ts[1].codes = ts[1].codes + 8  # the output takes 16-byte stores
    assert L().lrq_group_table_bytes(_lib.FMT_MXFP8_DEQUANT, ts, 2, 0, 1, 32, 0) == _lib.ERR_ALIGN
    fake = ctypes.c_void_p(0x10000)
    assert L().lrq_mx_dequant(3, fake, fake, 4, 64, fake, 0, None) == _lib.ERR_ARG      # bad format
    assert L().lrq_mx_dequant(_lib.FMT_MXFP8, fake, fake, 4, 48, fake, 0, None) == _lib.ERR_ARG  # cols % 32
    assert L().lrq_mx_dequant(_lib.FMT_MXFP4, fake, fake, 4, 64, fake, 1, None) == _lib.ERR_ARG  # fp16 out
    assert L().lrq_mx_dequant(_lib.FMT_MXFP4, None, None, 0, 64, None, 0, None) == 0    # nothing to do


def test_grouped_rejects_foreign_table():
    junk = np.zeros(4096, np.uint8)
    rc = L().lrq_quant_grouped(junk.ctypes.data, ctypes.c_void_p(0x1000), None)
    assert rc == _lib.ERR_TABLE
    assert L().lrq_group_units(junk.ctypes.data) == _lib.ERR_TABLE


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_ARG, "x")
    with pytest.raises(_lib.LrqError):
        _lib.check(_lib.ERR_TABLE, "x")
    with pytest.raises(_lib.LrqError):
        _lib.check(1, "x")


from hypothesis import given, settings, strategies as st  # noqa: E402

_FMT_BLK = [(_lib.FMT_FP8_BLOCK, (128, 128)), (_lib.FMT_FP8_BLOCK, (1, 128)), (_lib.FMT_FP8_BLOCK, (3, 40)),
            (_lib.FMT_MXFP8, (1, 32)), (_lib.FMT_MXFP4, (1, 32)), (_lib.FMT_FP8_DEQUANT, (1, 128)),
            (_lib.FMT_TENSOR_SCALE, (1, 1)), (_lib.FMT_COPY, (1, 1)), (_lib.FMT_CAST_E4M3, (1, 1)),
            (_lib.FMT_MXFP8_DEQUANT, (1, 32)), (_lib.FMT_MXFP4_DEQUANT, (1, 32))]


@given(fmt_blk=st.sampled_from(_FMT_BLK),
       dims=st.lists(st.tuples(st.integers(-2, 4), st.integers(-2, 3000), st.integers(-2, 3000),
                               st.integers(-8, 64), st.integers(0, 7)), min_size=1, max_size=6),
       dtype=st.integers(-1, 3), flags=st.integers(0, 15))
@settings(max_examples=400, deadline=None)
def test_group_packer_never_crashes_and_is_consistent(fmt_blk, dims, dtype, flags):
    """Random (often invalid) extents, strides, pointer offsets, dtypes and flags through
    the table packer, host side only: every call returns 0 or an LRQ_ERR_* code, and a
    table that sizes also packs, with units matching lrq_group_units."""
    fmt, blk = fmt_blk
    arr = (_lib.LrqTensor * len(dims))()
    p = 0x100000000
    for i, (b, r, c, pad, off) in enumerate(dims):
        arr[i].in_, arr[i].codes, arr[i].scales = p + off, p + (1 << 32) + off, p + (2 << 32)
        arr[i].batch, arr[i].rows, arr[i].cols = b, r, c
        arr[i].ld, arr[i].batch_stride = c + pad, max(r, 0) * (c + pad)
        p += 3 << 32
    need = L().lrq_group_table_bytes(fmt, arr, len(dims), dtype, blk[0], blk[1], flags)
    errs = {_lib.ERR_ARG, _lib.ERR_ALIGN, _lib.ERR_CAPACITY, _lib.ERR_TABLE}
    if need < 0:
        assert need in errs and _lib.last_error()
        return
    buf = np.zeros(need, np.uint8)
    assert L().lrq_group_pack(fmt, arr, len(dims), dtype, blk[0], blk[1], flags, buf.ctypes.data, need) == 0
    units = L().lrq_group_units(buf.ctypes.data)
    assert units >= 0
    assert L().lrq_group_device_bytes(buf.ctypes.data) == need + 4 * units


def test_static_workspace_entry_rejects_oversized_table_before_any_hip_call():
    fake = 1 << 20
    t = (_lib.LrqTensor * 1)()
    rows, cols = 1 << 20, 8192  # 2 M partials: more than LRQ_STATIC_WORKSPACE_BYTES holds
    t[0].in_, t[0].codes, t[0].scales = fake, None, fake
    t[0].batch, t[0].rows, t[0].cols, t[0].ld, t[0].batch_stride = 1, rows, cols, cols, rows * cols
    need = L().lrq_group_table_bytes(_lib.FMT_TENSOR_SCALE, t, 1, _lib.DTYPE_BF16, 1, 1, 0)
    host = (ctypes.c_uint8 * need)()
    assert L().lrq_group_pack(_lib.FMT_TENSOR_SCALE, t, 1, _lib.DTYPE_BF16, 1, 1, 0, host, need) == 0
    assert L().lrq_group_workspace_bytes(host) == 4 * (rows * cols // 4096) > _lib.STATIC_WORKSPACE_BYTES
    rc = L().lrq_tensor_scale_grouped_static(host, ctypes.c_void_p(fake), None)
    assert rc == _lib.ERR_CAPACITY and "static workspace" in _lib.last_error()
    # a table of another format is refused the same way
    t[0].rows, t[0].codes = 128, fake
    need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, t, 1, _lib.DTYPE_BF16, 128, 128, 0)
    host = (ctypes.c_uint8 * need)()
    assert L().lrq_group_pack(_lib.FMT_FP8_BLOCK, t, 1, _lib.DTYPE_BF16, 128, 128, 0, host, need) == 0
    assert L().lrq_tensor_scale_grouped_static(host, ctypes.c_void_p(fake), None) == _lib.ERR_ARG


def test_tensor_scale_tensor_count_limit_follows_the_finishing_work_groups():
    """The finishing launch runs one 1024-thread work-group per tensor, so a
    tensor-scale table of 2^32 / 1024 tensors is refused before any HIP call."""
    n = 0xFFFFFFFF // 1024 + 1
    fake = 1 << 20
    arr = np.zeros((n, 8), np.int64)  # lrq_tensor: in, codes, scales, batch, rows, cols, ld, batch_stride
    arr[:, 0] = fake + 16 * np.arange(n, dtype=np.int64)
    arr[:, 2] = fake
    arr[:, 3:8] = (1, 1, 8, 8, 8)
    ts = arr.ctypes.data_as(ctypes.POINTER(_lib.LrqTensor))
    need = L().lrq_group_table_bytes(_lib.FMT_TENSOR_SCALE, ts, n, _lib.DTYPE_BF16, 1, 1, 0)
    assert need > 0, _lib.last_error()
    host = np.zeros(need, np.uint8)
    assert L().lrq_group_pack(_lib.FMT_TENSOR_SCALE, ts, n, _lib.DTYPE_BF16, 1, 1, 0,
                              host.ctypes.data, need) == 0, _lib.last_error()
    ws = L().lrq_group_workspace_bytes(host.ctypes.data)
    rc = L().lrq_tensor_scale_grouped(host.ctypes.data, ctypes.c_void_p(fake), ctypes.c_void_p(fake), ws, None)
    assert rc == _lib.ERR_ARG and "too many tensors" in _lib.last_error()
    del host, arr


def test_float64_input_needs_float64_arithmetic_and_the_fp8_block_format():
    fake = ctypes.c_void_p(0x10000)
    rc = L().lrq_fp8_block_quant(fake, _lib.DTYPE_F64, 1, 4, 128, 128, 512, 1, 128, fake, fake, 0, None)
    assert rc == _lib.ERR_ARG and "LRQ_FLAG_NATIVE_ARITH" in _lib.last_error()
    rc = L().lrq_mxfp8_quant(fake, _lib.DTYPE_F64, 4, 64, 64, fake, fake, None)
    assert rc == _lib.ERR_ARG
    # misaligned float64 input
    odd = ctypes.c_void_p(0x10004)
    rc = L().lrq_fp8_block_quant(odd, _lib.DTYPE_F64, 1, 4, 128, 128, 512, 1, 128, fake, fake,
                                 _lib.FLAG_NATIVE_ARITH, None)
    assert rc == _lib.ERR_ALIGN
    # tables pack (host memory only) with each float64 kernel's geometry: a dense
    # 1x128 tensor, dense or with a padded row pitch, takes the row kernel (4
    # waves x 4 instructions of 128 doubles of the element sequence per
    # work-group); blocks narrower than 128 the padded-group kernel (64/L blocks
    # per wave instruction for L = nextpow2(ceil(B/2)) lanes, 4 instructions, 4
    # waves); wider ones the wide-row kernel; a 2-D block the generic kernel
    # (one wave per block, four per work-group)
    def units(rows, cols, ld, blk=128, blk_r=1):
        t = (_lib.LrqTensor * 1)()
        t[0].in_, t[0].codes, t[0].scales = 0x10000, 0x20000, 0x30000
        t[0].batch, t[0].rows, t[0].cols, t[0].ld, t[0].batch_stride = 1, rows, cols, ld, rows * ld
        need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, t, 1, _lib.DTYPE_F64, blk_r, blk,
                                         _lib.FLAG_NATIVE_ARITH)
        host = (ctypes.c_uint8 * need)()
        assert L().lrq_group_pack(_lib.FMT_FP8_BLOCK, t, 1, _lib.DTYPE_F64, blk_r, blk,
                                  _lib.FLAG_NATIVE_ARITH, host, need) == 0
        return L().lrq_group_units(host)

    assert units(5, 256, 256) == 1
    assert units(40, 256, 256) == 5
    assert units(40, 256, 384) == 5
    assert units(5, 288, 288, 96) == -(-5 * 3 // 16)   # L = 64: one block per instruction
    assert units(5, 450, 450, 45) == -(-5 * 10 // 32)  # L = 32: two
    assert units(64, 80, 80, 5) == 64 * 16 // 256      # L = 4: sixteen
    assert units(7, 112, 120, 16) == -(-7 * 7 // 128)  # L = 8, padded row pitch
    assert units(50, 768, 800, 384) == -(-50 * 2 // 8)  # 2 blocks per wave
    assert units(9, 3000, 3000, 3000) == 9              # one block of 4 waves
    assert units(3, 24576, 24576, 12288) == 6           # one block of 16 waves
    assert units(8, 16386, 16386, 16386) == 2           # past 16384: generic, 4 blocks per work-group
    assert units(5, 288, 288, 96, 2) == (3 * 3 + 3) // 4  # 2-D blocks: generic


def test_fp8_dequant_chunk_per_width():
    """FP8 dequant lane-chunks: 8 codes for bf16 output when 8 divides the block
    width and every row, else 4 (a 4-code bf16 chunk stores 8 bytes); 512
    chunks per work-group; widths 4 does not divide take the per-element kernel
    (256 elements per work-group)."""
    def units(cols, blk_c, out_bf16, rows=64):
        flags = _lib.FLAG_OUT_BF16 if out_bf16 else 0
        return L().lrq_group_units(_pack(_lib.FMT_FP8_DEQUANT, [(1, rows, cols)], (1, blk_c), flags).ctypes.data)

    n = 64 * 1152
    assert units(1152, 128, True) == -(-n // 8 // 512)
    assert units(1152, 36, True) == -(-n // 4 // 512)
    assert units(1152, 128, False) == -(-n // 4 // 512)
    assert units(1152, 36, False) == -(-n // 4 // 512)
    assert units(1152, 6, True) == -(-n // 256)


@pytest.mark.parametrize("dtype,blk_c,threads", [(0, 32768, 512), (0, 65536, 1024), (2, 65536, 1024),
                                                 (3, 8192, 512), (3, 16384, 1024), (0, 16384, 256)])
def test_group_limit_counts_the_wide_kernels_work_group_size(dtype, blk_c, threads):
    """HIP takes a launch's thread count as 32 bits.  k_row_wide runs 512- or
    1024-thread work-groups for its widest 1xB blocks (one block each) and
    k_row_wide_f64 for float64 blocks past 4096, so a grouped table may hold at
    most 0xFFFFFFFF // threads of them; one block more is refused at pack time,
    before any device work (fake device pointers)."""
    flags = _lib.FLAG_NATIVE_ARITH if dtype == 3 else 0
    limit = 0xFFFFFFFF // threads

    def pack(rows):
        ts = _tensors([(1, rows, blk_c)])
        need = L().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, ts, 1, dtype, 1, blk_c, flags)
        if need < 0:
            return need, None
        buf = np.zeros(need, np.uint8)
        return L().lrq_group_pack(_lib.FMT_FP8_BLOCK, ts, 1, dtype, 1, blk_c, flags, buf.ctypes.data, need), buf

    rc, buf = pack(limit)
    assert rc == 0, _lib.last_error()
    assert L().lrq_group_units(buf.ctypes.data) == limit
    rc, _ = pack(limit + 1)
    assert rc == _lib.ERR_ARG and "too large" in _lib.last_error()
