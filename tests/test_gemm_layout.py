"""Host-side checks of the LDS-direct SGEMM layouts (silarray_amd/csrc/gemm.hip,
sgemm_dtl_k, operand extents 256, 128 and 64, K tiles of 16 and 32).

The index functions below restate dtl_src / dtl_window / dtl_elem / dtl_frag4,
and the tests check the properties the kernel relies on: every element of a
TILE x BK operand tile lands in exactly one LDS slot inside the operand's part
of a stage, every fragment read finds the elements it asks for, and no
fragment read has an LDS bank conflict.

LDS model, measured on MI355X (gfx950) with rocprofv3 SQ_LDS_BANK_CONFLICT on
kernels in which only two lanes read: ds_read_b32 serves one half-wave (lanes
0-31, then 32-63) per pass over 32 four-byte banks; ds_read_b128 serves 16
lanes per pass over 64 four-byte banks, the lanes of a pass being those with
equal lane bit 5 and equal parity of lane bits 2-4 (lane 0 shares its pass
with lanes 1-3, 12-15, 20-23 and 24-27).  Two lanes of one pass that touch one
bank at different addresses conflict.

Fragment reads of the 16x16x4 MFMA (lane l: row or column r = l % 16, k slot
g = l / 16).  Step j of a 16-deep k block uses k = 4g + j in slot g, for both
operands, so:
  - an operand contiguous in K is read with one ds_read_b128 per 16-row block
    and k block: lane l reads the four k values 4g .. 4g+3 of row r, one for
    each of the four steps;
  - an operand contiguous in M or N is read with one ds_read_b32 per 16-wide
    block and step: lane l reads element (r, 4g + j).
No GPU."""

import pytest

PITCH = {256: 260, 128: 264, 64: 272}  # M/N-contiguous window pitch per tile extent (floats)
SHAPES = [(256, 16), (256, 32), (128, 16), (128, 32), (64, 16), (64, 32)]  # (extent, BK)


def windows(tile, bk):
    return tile * bk // 256


def swz(r):
    return (r // 2) & 3


def lane_chunks(kcontig, tile, w, lane):
    """The 4 (x, k) elements lane `lane` loads for window w, in LDS order."""
    if kcontig:
        rr = lane // 4
        kq = (lane % 4) ^ swz(rr)
        rg, kh = w % (tile // 16), w // (tile // 16)
        return [(16 * rg + rr, 16 * kh + 4 * kq + e) for e in range(4)]
    if tile == 256:
        return [(4 * lane + e, w) for e in range(4)]
    if tile == 128:
        p, c = lane // 32, lane % 32
        return [(4 * c + e, 2 * w + p) for e in range(4)]
    p, c = lane // 16, lane % 16
    return [(4 * c + e, 4 * w + p) for e in range(4)]


def window_base(kcontig, tile, w):
    return w * 256 if kcontig else w * PITCH[tile]


def elem(kcontig, tile, x, k):
    if kcontig:
        r = x % 16
        return (((k // 16) * (tile // 16) + x // 16) * 256 +
                (4 * r + (((k % 16) // 4) ^ swz(r))) * 4 + k % 4)
    if tile == 256:
        return k * PITCH[256] + x
    if tile == 128:
        return (k // 2) * PITCH[128] + 128 * (k % 2) + x
    return (k // 4) * PITCH[64] + 64 * (k % 4) + x


def operand_floats(tile, bk):
    return windows(tile, bk) * PITCH[tile]


def placed(kcontig, tile, bk):
    lds = {}
    for w in range(windows(tile, bk)):
        for lane in range(64):
            for e, (x, k) in enumerate(lane_chunks(kcontig, tile, w, lane)):
                pos = window_base(kcontig, tile, w) + 4 * lane + e  # lane L writes floats 4L..4L+3
                assert 0 <= x < tile and 0 <= k < bk
                assert pos not in lds and 0 <= pos < operand_floats(tile, bk)
                lds[pos] = (x, k)
    return lds


def b32_conflict_free(addrs):
    """addrs[l] = float offset read by lane l with ds_read_b32."""
    for half in (range(0, 32), range(32, 64)):
        bank = {}
        for l in half:
            b = addrs[l] % 32
            if bank.setdefault(b, addrs[l]) != addrs[l]:
                return False
    return True


def b128_pass(l):
    return (l >> 5) & 1, bin((l >> 2) & 7).count("1") & 1


def b128_conflict_free(addrs):
    """addrs[l] = float offset (a multiple of 4) read by lane l with ds_read_b128."""
    passes = {}
    for l in range(64):
        passes.setdefault(b128_pass(l), []).append(l)
    assert sorted(len(v) for v in passes.values()) == [16] * 4
    for lanes in passes.values():
        bank = {}
        for l in lanes:
            for e in range(4):
                a = addrs[l] + e
                if bank.setdefault(a % 64, a) != a:
                    return False
    return True


@pytest.mark.parametrize("tile,bk", SHAPES)
@pytest.mark.parametrize("kcontig", [True, False])
def test_every_element_placed_once_and_found(kcontig, tile, bk):
    lds = placed(kcontig, tile, bk)
    assert len(lds) == tile * bk
    for x in range(tile):
        for k in range(bk):
            assert lds[elem(kcontig, tile, x, k)] == (x, k)


def test_lds_budget():
    # two stages of two operands, as dtl_cfg::kLdsBytes; LDS is 160 KiB per CU
    for tile, bk in SHAPES:
        assert 2 * 2 * operand_floats(tile, bk) * 4 <= 160 * 1024
        assert operand_floats(tile, bk) >= windows(tile, bk) * 256  # K-contiguous fits too
    assert 2 * 2 * operand_floats(256, 32) * 4 == 133120


@pytest.mark.parametrize("tile,bk", SHAPES)
def test_kcontig_b128_reads(tile, bk):
    """One ds_read_b128 per 16-row block and k block: 16-byte aligned, the four
    floats are k = 4g .. 4g+3 of row r in order, and no pass conflicts."""
    for rb in range(tile // 16):
        for kh in range(bk // 16):
            addrs = []
            for l in range(64):
                r, g = l % 16, l // 16
                a = elem(True, tile, 16 * rb + r, 16 * kh + 4 * g)
                assert a % 4 == 0
                for e in range(4):
                    assert elem(True, tile, 16 * rb + r, 16 * kh + 4 * g + e) == a + e
                addrs.append(a)
            assert b128_conflict_free(addrs), (rb, kh)


@pytest.mark.parametrize("tile,bk", SHAPES)
def test_mncontig_b32_reads(tile, bk):
    """One ds_read_b32 per 16-wide block and step, k = 16 kh + 4g + j: no
    half-wave touches a bank twice."""
    for cb in range(tile // 16):
        for kh in range(bk // 16):
            for j in range(4):
                addrs = [elem(False, tile, 16 * cb + l % 16, 16 * kh + 4 * (l // 16) + j)
                         for l in range(64)]
                assert b32_conflict_free(addrs), (cb, kh, j)


def test_bank_model_matches_the_measurements():
    """The probe patterns measured on the GPU, through the model above: conflict
    (True) or not, as observed."""
    lin32 = list(range(64))
    assert b32_conflict_free(lin32)
    assert b32_conflict_free([l % 32 + 64 * (l // 32) for l in range(64)])
    assert not b32_conflict_free([(l % 32) * 2 for l in range(64)])
    # the previous K-contiguous fragment pattern (b32, chunk swizzle (r/4)&3): 2-way
    assert not b32_conflict_free([16 * (l % 16) + 4 * (((l % 16) // 4) & 3) + l // 16
                                  for l in range(64)])
    assert b128_conflict_free([4 * l for l in range(64)])
    assert not b128_conflict_free([4 * (l % 8) + 256 * (l // 8) for l in range(64)])
    assert b128_conflict_free([4 * (l % 16) + 256 * (l // 16) for l in range(64)])
    r = [l % 16 for l in range(64)]
    g = [l // 16 for l in range(64)]
    assert not b128_conflict_free([4 * (4 * r[l] + (g[l] ^ ((r[l] // 4) & 3))) for l in range(64)])
    assert b128_conflict_free([4 * (4 * r[l] + (g[l] ^ ((r[l] // 2) & 3))) for l in range(64)])


@pytest.mark.parametrize("kg,lds_bytes,per_cu", [(2, 69632, 2), (4, 139264, 1)])
def test_k_groups_lds_budget_and_exchange(kg, lds_bytes, per_cu):
    """The 64 x 64 tile with K split between two or four groups of 4 waves of
    32 x 32 (BK 32, two stages each): the groups' stages fit in LDS (69,632
    and 139,264 B per workgroup, the sizes the compiler reports; two and one
    workgroups per CU), and the accumulator exchange slot ((i * TN + j) * NW
    + w) * 64 + l (float4 units) is a bijection of (i, j, wave, lane) onto
    the first TM * TN * NW * 64 float4 of the first stage array, which holds
    kg * kStage floats."""
    ns, nw, tm, tn = 2, 4, 2, 2
    stage = 2 * operand_floats(64, 32)  # A and B windows of one stage, floats
    assert kg * ns * stage * 4 == lds_bytes
    assert per_cu * lds_bytes <= 160 * 1024 < (per_cu + 1) * lds_bytes
    slots = {((i * tn + j) * nw + w) * 64 + l
             for i in range(tm) for j in range(tn) for w in range(nw) for l in range(64)}
    assert slots == set(range(tm * tn * nw * 64))
    assert 4 * len(slots) <= kg * stage
