"""Host-side checks of the LDS-direct SGEMM layouts (silarray_amd/csrc/gemm.hip,
sgemm_dtl_k, tiles of 256 and 128): the index functions below restate
dtl_src / dtl_window / dtl_elem, and the tests check the properties the
kernel relies on -- every element of a TILE x 16 operand tile lands in exactly
one LDS slot inside the operand's part of a stage, every fragment read finds
the element it asks for, and the 64 lanes of a 16x16x4 fragment read touch 64
distinct LDS banks (4-byte banks).  No GPU."""

import pytest

BK = 16
PITCH = {256: 272, 128: 288}  # M/N-contiguous window pitch per tile width (floats)


def windows(tile):
    return tile // 16


def lane_chunks(kcontig, tile, w, lane):
    """The 4 (x, k) elements lane `lane` loads for window w, in LDS order."""
    if kcontig:
        rr = lane // 4
        kq = (lane % 4) ^ ((rr // 4) & 3)
        return [(16 * w + rr, 4 * kq + e) for e in range(4)]
    if tile == 256:
        return [(4 * lane + e, w) for e in range(4)]
    p = lane // 32
    c = (lane % 32) ^ (4 * p)
    return [(4 * c + e, 2 * w + p) for e in range(4)]


def window_base(kcontig, tile, w):
    return w * 256 if kcontig else w * PITCH[tile]


def elem(kcontig, tile, x, k):
    if kcontig:
        return (x // 16) * 256 + ((x % 16) * 4 + ((k // 4) ^ (((x % 16) // 4) & 3))) * 4 + k % 4
    if tile == 256:
        return k * PITCH[256] + x
    p = k % 2
    return (k // 2) * PITCH[128] + (32 * p + ((x // 4) ^ (4 * p))) * 4 + x % 4


def operand_floats(tile):
    return windows(tile) * PITCH[tile]


def placed(kcontig, tile):
    lds = {}
    for w in range(windows(tile)):
        for lane in range(64):
            for e, (x, k) in enumerate(lane_chunks(kcontig, tile, w, lane)):
                pos = window_base(kcontig, tile, w) + 4 * lane + e  # lane L writes floats 4L..4L+3
                assert 0 <= x < tile and 0 <= k < BK
                assert pos not in lds and 0 <= pos < operand_floats(tile)
                lds[pos] = (x, k)
    return lds


@pytest.mark.parametrize("tile", [256, 128])
@pytest.mark.parametrize("kcontig", [True, False])
def test_every_element_placed_once_and_found(kcontig, tile):
    lds = placed(kcontig, tile)
    assert len(lds) == tile * BK
    for x in range(tile):
        for k in range(BK):
            assert lds[elem(kcontig, tile, x, k)] == (x, k)


@pytest.mark.parametrize("tile", [256, 128])
@pytest.mark.parametrize("kcontig", [True, False])
def test_fragment_reads_are_bank_conflict_free(kcontig, tile):
    for row_block in range(tile // 16):
        for step in range(BK // 4):
            banks = {elem(kcontig, tile, 16 * row_block + lm, 4 * step + kl) % 64
                     for kl in range(4) for lm in range(16)}
            assert len(banks) == 64, (row_block, step)
