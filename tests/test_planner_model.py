"""The FP8 planner against a model of its rules (no GPU).

``lrq_group_table_bytes`` / ``lrq_group_pack`` choose a kernel for each tensor
from its dtype, block, shape, strides and pointer alignment, then count the
work-groups that kernel needs.  This module restates those rules in Python
(which kernel takes which input, and how many blocks a work-group covers) and
compares the library's work-group count with the model's on random inputs:
any disagreement in the kernel choice or the geometry shows up as a different
count, or as a table the library refuses.
"""

from __future__ import annotations

import ctypes

from hypothesis import given, settings, strategies as st

from lumenrl_amd import _lib

ES = {_lib.DTYPE_BF16: 2, _lib.DTYPE_F16: 2, _lib.DTYPE_F32: 4}
ROW_BLOCKS = 4  # wave instructions per lane of the row kernels


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def model_units(dt, batch, rows, cols, ld, bstride, blk_r, blk_c, in_off, codes_off):
    es = ES[dt]
    aligned_in = in_off % es == 0
    aligned_codes = codes_off % 8 == 0
    folds = batch == 1 or bstride == rows * ld
    vec = aligned_in and aligned_codes and cols % 8 == 0
    vec_row = aligned_in and aligned_codes and folds
    nblocks = batch * rows * cols // blk_c if blk_r == 1 else 0
    generic = batch * cdiv(rows, blk_r) * cdiv(cols, blk_c)
    if (blk_r, blk_c) == (128, 128) and vec:
        return generic  # one 512-thread work-group per tile
    if blk_r != 1 or cols % blk_c:
        return generic
    if (dt == _lib.DTYPE_F32 and blk_c in (8, 16, 32, 64, 128, 256, 512, 1024) and vec
            and codes_off % 4 == 0 and folds):
        per = 4 * ROW_BLOCKS * (256 // blk_c) if blk_c <= 256 else 4 * ROW_BLOCKS // (blk_c // 256)
        return cdiv(nblocks, per)
    if blk_c in (32, 64, 128, 256, 512, 1024, 2048) and vec and folds:
        per = 4 * ROW_BLOCKS * (512 // blk_c) if blk_c <= 512 else 4 * ROW_BLOCKS // (blk_c // 512)
        return cdiv(nblocks, per)
    if 8 <= blk_c <= 512 and vec_row:
        lanes = 1
        while lanes < cdiv(blk_c, 8):
            lanes *= 2
        return cdiv(nblocks, 4 * ROW_BLOCKS * (64 // lanes))
    if 512 < blk_c <= 65536 and vec_row:
        # the fewest 64-lane steps (a power of two) of 8-element chunk slots that
        # hold a block, as 4 or 8 slots per lane
        chunks = cdiv(blk_c, 8)
        steps = 2
        while steps * 64 < chunks:
            steps *= 2
        eight = steps > 16 or chunks == 512 or (dt != _lib.DTYPE_F32 and chunks > 768)
        if eight:
            return cdiv(nblocks, 4 if steps == 8 else 1)  # 4 one-wave blocks, or one block of 4-16 waves
        if steps <= 4:
            return cdiv(nblocks, 4 * (4 // steps))  # 4 waves of 4/steps blocks
        return cdiv(nblocks, 4 // (steps // 4))  # blocks of 2 or 4 waves
    return generic


def library_units(dt, batch, rows, cols, ld, bstride, blk_r, blk_c, in_off, codes_off):
    t = (_lib.LrqTensor * 1)()
    t[0].in_ = 0x100000000 + in_off
    t[0].codes = 0x200000000 + codes_off
    t[0].scales = 0x300000000
    t[0].batch, t[0].rows, t[0].cols, t[0].ld, t[0].batch_stride = batch, rows, cols, ld, bstride
    need = _lib.lib().lrq_group_table_bytes(_lib.FMT_FP8_BLOCK, t, 1, dt, blk_r, blk_c, 0)
    assert need > 0, _lib.last_error()
    host = (ctypes.c_uint8 * need)()
    assert _lib.lib().lrq_group_pack(_lib.FMT_FP8_BLOCK, t, 1, dt, blk_r, blk_c, 0, host, need) == 0
    return _lib.lib().lrq_group_units(host)


WIDTHS = [5, 8, 12, 16, 24, 32, 36, 40, 64, 96, 100, 128, 256, 500, 512, 640, 1000, 1024, 1536,
          2048, 2056, 3001, 4090, 4096, 4104, 6144, 6152, 8192, 8200, 9999, 16384, 16392, 18944,
          29568, 65536, 65544]


@settings(max_examples=400, deadline=None)
@given(dt=st.sampled_from([_lib.DTYPE_BF16, _lib.DTYPE_F16, _lib.DTYPE_F32]),
       blk=st.one_of(st.sampled_from([(128, 128), (64, 64), (2, 128), (3, 40)]),
                     st.sampled_from(WIDTHS).map(lambda b: (1, b))),
       mult=st.integers(1, 5), extra=st.integers(0, 7), rows=st.integers(1, 300),
       batch=st.integers(1, 3), pitch=st.integers(0, 9), ragged=st.booleans(),
       in_off=st.sampled_from([0, 2, 4, 6, 8, 1]), codes_off=st.sampled_from([0, 8, 4, 1]))
def test_planner_matches_the_model(dt, blk, mult, extra, rows, batch, pitch, ragged, in_off, codes_off):
    blk_r, blk_c = blk
    cols = blk_c * mult if blk_r == 1 or extra == 0 else blk_c * mult + extra
    ld = cols + pitch
    bstride = rows * ld + (5 if ragged and batch > 1 else 0)
    if blk_r == 1 and not (batch == 1 or bstride == rows * ld):
        return  # the row kernels fold batches; a ragged stack goes through its matrices
    args = (dt, batch, rows, cols, ld, bstride, blk_r, blk_c, in_off, codes_off)
    assert library_units(*args) == model_units(*args), args


def test_model_spot_checks():
    """A few hand-computed counts, so the model itself is pinned."""
    bf = _lib.DTYPE_BF16
    assert model_units(bf, 1, 4096, 4096, 4096, 4096 * 4096, 128, 128, 0, 0) == 1024
    assert model_units(bf, 1, 256, 4096, 4096, 256 * 4096, 1, 128, 0, 0) == 256 * 32 // 64
    assert model_units(bf, 1, 256, 3600, 3600, 256 * 3600, 1, 36, 2, 0) == cdiv(256 * 100, 128)
    assert model_units(bf, 1, 4, 4096, 4096, 4 * 4096, 1, 4096, 0, 0) == 1
    assert model_units(bf, 1, 4, 10, 10, 40, 1, 5, 0, 0) == 8
    f32 = _lib.DTYPE_F32
    assert model_units(f32, 1, 64, 3840, 3840, 64 * 3840, 1, 640, 0, 0) == 64 * 6 // 8
    assert model_units(bf, 1, 64, 3840, 3840, 64 * 3840, 1, 640, 0, 0) == 64 * 6 // 8
    assert model_units(bf, 1, 8, 6144, 6144, 8 * 6144, 1, 3072, 0, 0) == 8  # 2 waves per block
    assert model_units(f32, 1, 4, 8192, 8192, 4 * 8192, 1, 4096, 0, 0) == 2  # one wave per block
    assert model_units(bf, 1, 4, 8192, 8192, 4 * 8192, 1, 4096, 0, 0) == 2
    assert model_units(bf, 1, 4, 12000, 12000, 4 * 12000, 1, 6000, 0, 0) == 8  # 4 waves per block
    assert model_units(bf, 1, 4, 7000, 7000, 4 * 7000, 1, 7000, 0, 0) == 4
    assert model_units(bf, 1, 64, 18944, 18944, 64 * 18944, 1, 18944, 0, 0) == 64  # 8 waves per block
    assert model_units(bf, 1, 4, 65544, 65544, 4 * 65544, 1, 65544, 0, 0) == 4  # generic, one per block
    assert library_units(bf, 1, 4096, 4096, 4096, 4096 * 4096, 128, 128, 0, 0) == 1024
