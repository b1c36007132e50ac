"""Model of the pipelined GEMM's DMA lane map (csrc/fp8_gemm_pipe.h, pipe_tile).

One stage copies BT rows x 128 bytes of an operand (BT = BM activation rows or
BN weight rows: 64, 128, 192 or 256) with BT/32 buffer_load ... lds
instructions per wave (4 waves).  Lane l of wave w reads row
``w * BT/4 + l // 8 + 8 * (i % 2) + 16 * (i // 2)`` for instruction i, chunk
``(l % 8) ^ swizzle``.  The buffer range check sees only the lane offset:
  * vector-offset DMA: the lane offset holds the whole row, so a row at or past
    the operand's last row reads zero;
  * scalar-offset DMA: the lane offset holds ``w * BT/4 + l // 8 + 8 * (i % 2)``
    and the 16-row block step is in soffset, which the check does not cover.
The kernel uses the scalar-offset form only in full tiles.
"""

import numpy as np
import pytest


def lane_rows(bt):
    """(row read, row the range check sees) under both forms: arrays [wave, lane, instr]."""
    dma_a = bt // 32
    w = np.arange(4)[:, None, None]
    lane = np.arange(64)[None, :, None]
    i = np.arange(dma_a)[None, None, :]
    row0 = w * dma_a * 8 + lane // 8
    read = row0 + 8 * (i % 2) + 16 * (i // 2)
    return read, row0 + 8 * (i % 2)


def uses_scalar_offset(rows_valid, bt):
    return rows_valid == bt


@pytest.mark.parametrize("bt", [64, 128, 192, 256])
def test_every_tile_row_is_loaded_once_per_stage(bt):
    read, _ = lane_rows(bt)
    rows = np.sort(read.reshape(-1, read.shape[-1]), axis=None)
    # eight lanes (one 16-byte chunk each) per row
    assert np.array_equal(np.bincount(rows, minlength=bt), np.full(bt, 8))


@pytest.mark.parametrize("bt", [64, 128, 192, 256])
@pytest.mark.parametrize("rows_valid", [1, 4, 16, 17, 48, 63, 64, 100, 127, 128, 191, 192, 200,
                                        255, 256])
def test_no_read_past_the_operand(bt, rows_valid):
    if rows_valid > bt:
        pytest.skip("tile smaller than the valid rows")
    read, checked = lane_rows(bt)
    live = (checked if uses_scalar_offset(rows_valid, bt) else read) < rows_valid
    # every access that the range check lets through stays inside the operand
    assert (read[live] < rows_valid).all()
    # and every valid row is still loaded
    assert set(read[live].ravel()) == set(range(rows_valid))


def test_scalar_offset_form_would_overrun_a_partial_tile():
    # Why partial tiles take the vector-offset form: with one valid row the
    # scalar-offset form reads rows up to 48 past it.
    read, checked = lane_rows(256)
    live = checked < 1
    assert read[live].max() == 48
