"""Host-side checks of the LDS-direct SGEMM layout (silarray_amd/csrc/gemm.hip,
sgemm_dtl_k): the index functions below restate dtl_src / dtl_window /
dtl_elem, and the tests check the properties the kernel relies on -- every
element of a 256 x 16 operand tile lands in exactly one LDS slot inside one
stage, every fragment read finds the element it asks for, and the 64 lanes of
a 16x16x4 fragment read touch 64 distinct LDS banks (4-byte banks).  No GPU."""

import pytest

PITCH, WINDOWS, TILE, BK = 272, 16, 256, 16
STAGE_HALF = WINDOWS * PITCH  # each operand's share of a stage (floats)


def lane_chunk(kcontig, w, lane):
    """(x, k) of the first float of the 16-byte chunk lane `lane` loads for
    window w, and the axis its 4 floats run along."""
    if kcontig:
        rr = lane // 4
        kq = (lane % 4) ^ ((rr // 4) & 3)
        return 16 * w + rr, 4 * kq, "k"
    return 4 * lane, w, "x"


def window_base(kcontig, w):
    return w * 256 if kcontig else w * PITCH


def elem(kcontig, x, k):
    if kcontig:
        return (x // 16) * 256 + ((x % 16) * 4 + ((k // 4) ^ (((x % 16) // 4) & 3))) * 4 + k % 4
    return k * PITCH + x


def placed(kcontig):
    lds = {}
    for w in range(WINDOWS):
        for lane in range(64):
            x, k, axis = lane_chunk(kcontig, w, lane)
            for e in range(4):
                pos = window_base(kcontig, w) + 4 * lane + e  # lane L writes floats 4L..4L+3
                xe, ke = (x, k + e) if axis == "k" else (x + e, k)
                assert 0 <= xe < TILE and 0 <= ke < BK
                assert pos not in lds and 0 <= pos < STAGE_HALF
                lds[pos] = (xe, ke)
    return lds


@pytest.mark.parametrize("kcontig", [True, False])
def test_every_element_placed_once_and_found(kcontig):
    lds = placed(kcontig)
    assert len(lds) == TILE * BK
    for x in range(TILE):
        for k in range(BK):
            assert lds[elem(kcontig, x, k)] == (x, k)


@pytest.mark.parametrize("kcontig", [True, False])
@pytest.mark.parametrize("row_block", [0, 5, 15])
def test_fragment_reads_are_bank_conflict_free(kcontig, row_block):
    for step in range(BK // 4):
        banks = {elem(kcontig, 16 * row_block + lm, 4 * step + kl) % 64
                 for kl in range(4) for lm in range(16)}
        assert len(banks) == 64
