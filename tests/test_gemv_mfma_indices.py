"""CPU check of the batched head GEMV's (k_gemv_mfma) memory indices: for
every shape its launcher accepts (molten_amd/csrc/gemv_mfma.hip, mh::gemv_mfma:
group 64, K % 512 == 0, K <= 2048, N % 16 == 0; Q4 and Q6), every global
address the kernel forms for codes, scales and biases -- including the stages
it prefetches past a wave's last tile -- and every LDS index of the scale /
bias table and the code staging buffer stays in bounds.  The kernel's
constants are read from its source, so a change there is checked here.

The index model restates the kernel's issue() / stage_sb() / compute()
arithmetic over all 256 x 8 waves and 64 lanes at once (numpy)."""
import os
import re

import numpy as np
import pytest

SRC = os.path.join(os.path.dirname(__file__), "..", "molten_amd", "csrc", "gemv_mfma.hip")


def _const(name):
    text = open(SRC).read()
    m = re.search(r"constexpr\s+(?:int|uint32_t)\s+%s\s*=\s*([0-9]+)u?\s*;" % name, text)
    assert m, name
    return int(m.group(1))


def _stride_words(bits):
    text = open(SRC).read()
    m = re.search(r"kStrideWords\s*=\s*BITS\s*==\s*6\s*\?\s*([0-9]+)\s*:\s*([0-9]+)", text)
    assert m
    return int(m.group(1)) if bits == 6 else int(m.group(2))


WAVES, GRID, ROWS, SG, DEPTH = (_const("kWaves"), _const("kGrid"), _const("kTileRows"), _const("kStageGroups"),
                                _const("kDepth"))
MAX_K = _const("kMaxK")


def check_shape(n, k, bits):
    g = k // 64
    row_bytes = k * bits // 8
    stage_bytes = SG * 64 * bits // 8          # SS::kRowBytes
    pieces = stage_bytes // 16                 # SS::kRowPieces
    loads = ROWS * pieces // 64                # SS::kLoads
    stride_w = _stride_words(bits)
    n_st = (g + SG - 1) // SG
    n_tiles = n // ROWS
    stride = GRID * WAVES
    wave = np.arange(stride, dtype=np.int64)[:, None]   # blockIdx.x * kWaves + wave
    lane = np.arange(64, dtype=np.int64)[None, :]
    first = wave
    my_tiles = np.where(first < n_tiles, (n_tiles - first + stride - 1) // stride, 0)
    n_stages = my_tiles * n_st
    last_st = np.where(n_stages > 0, n_stages - 1, 0)
    first_c = np.where(first < n_tiles, first, 0)
    srow, sgl = lane >> 2, 2 * (lane & 3)
    # LDS: the scale / bias table sbl[..][sg + e][srow] and the staging rows
    assert int((sgl + 1).max()) < SG and int(srow.max()) < ROWS
    for i in range(loads):
        pc = i * 64 + lane
        top = (pc // pieces) * stride_w + (pc % pieces) * 4 + 4
        assert int(top.max()) <= ROWS * stride_w
    codes_end = n * row_bytes
    sb_end = n * g
    # every stage a wave issues: st in [0, n_stages + kDepth - 1), clamped
    for st in range(int(n_stages.max()) + DEPTH):
        s_c = np.minimum(st, last_st)
        tile = np.where(n_stages > 0, first + (s_c // n_st) * stride, first_c)
        stage = s_c % n_st
        assert int(tile.max()) < max(n_tiles, 1)
        base = tile * ROWS * row_bytes + stage * stage_bytes
        for i in range(loads):
            pc = i * 64 + lane
            off = base + (pc // pieces) * row_bytes + (pc % pieces) * 16
            assert int(off.min()) >= 0 and int((off + 16).max()) <= codes_end
        sbi = (tile * ROWS + srow) * g + stage * SG + sgl
        assert int(sbi.min()) >= 0 and int((sbi + 2).max()) <= sb_end
        # the two bf16 of one 4-byte load stay in one row (groups sg, sg + 1)
        assert int(((stage * SG + sgl + 1) // g).max()) == 0 or g == 0


# every N up to 64 tiles, then N around whole rounds of the 2048 waves (one
# tile more or less than a round), then the heads' own sizes
ROUND = GRID * WAVES * ROWS
SMALL_N = list(range(16, 64 * 16 + 1, 16)) + [j * ROUND + d * 16 for j in (1, 2) for d in (-1, 0, 1)]


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("k", [kk for kk in range(512, MAX_K + 1, 512)])
def test_indices_small_and_round_n(bits, k):
    for n in SMALL_N:
        check_shape(n, k, bits)


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("n", [65536, 128000, 32768 * 3 + 48, 1 << 20])
def test_indices_large_n(bits, n):
    for k in range(512, MAX_K + 1, 512):
        check_shape(n, k, bits)


def test_model_catches_a_wrong_staging_width():
    """The model fails for 4-group stages, the form whose scale reads ran past
    the matrix (groups 2 (l % 4) .. + 1 cover exactly 8 groups of 16 rows)."""
    global SG
    saved = SG
    try:
        SG = 4
        with pytest.raises(AssertionError):
            check_shape(64, 512, 4)
    finally:
        SG = saved
