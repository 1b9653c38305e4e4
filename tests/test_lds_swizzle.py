"""Model check of the LDS swizzles in csrc/vt_hip_gemm.hip (host only).

The formulas below restate a_off / b_swz and the fragment and staging
address patterns of the MFMA kernels; the test checks that every access group
hits distinct 4-byte banks both when the LDS serves 256 bytes per cycle (16
lanes of a 16-byte access, 32 lanes of an 8-byte access) and 128 bytes per
cycle (half those groups), and that every swizzle is a permutation.
"""
import pytest


def a_off(row, c):
    return row * 64 + ((c ^ (((row >> 1) ^ (row >> 3)) & 3)) << 4)


def b_swz(chunks, row):
    if chunks >= 16:
        return ((row & 7) << 1) | ((row >> 2) & 1)
    if chunks == 8:
        return row & 7
    return (row >> 1) & 3


def worst_conflict(accesses, width, lanes_per_cycle):
    worst = 0
    for g in range(0, len(accesses), lanes_per_cycle):
        banks = {}
        for addr, nbytes in accesses[g:g + lanes_per_cycle]:
            for b in range(nbytes // 4):
                bank = (addr % width) // 4 + b
                banks[bank] = banks.get(bank, 0) + 1
        worst = max(worst, max(banks.values()) - 1)
    return worst


def check(accesses, nbytes):
    per256 = 256 // nbytes
    assert worst_conflict(accesses, 256, per256) == 0
    assert worst_conflict(accesses, 128, per256 // 2) == 0


@pytest.mark.parametrize("bn", [128, 256])
def test_b_fragment_reads_conflict_free(bn):
    chunks = bn // 16
    for wn in (0, 1):
        for ni in range(bn // 2 // 32):
            for ks in (0, 1):
                acc = []
                for lane in range(64):
                    g, j = lane >> 4, lane & 15
                    nc = (wn * bn // 2 + ni * 32) // 16 + (g & 1)
                    r0 = ks * 32 + (g >> 1) * 16 + (j >> 1)
                    acc.append((r0 * bn + ((nc ^ b_swz(chunks, r0)) << 4) + (j & 1) * 8, 8))
                check(acc, 8)


def test_a_fragment_reads_conflict_free():
    for wm in (0, 1):
        for mi in range(4):
            for ks in (0, 1):
                check([(a_off(wm * 128 + mi * 32 + (l & 31), ks * 2 + (l >> 5)), 16)
                       for l in range(64)], 16)


@pytest.mark.parametrize("chunks", [8, 16])
def test_slice_writes_conflict_free_and_bijective(chunks):
    for w in range(4):
        check([(a_off((w * 64 + l) >> 2, (w * 64 + l) & 3), 16) for l in range(64)], 16)
        check([(((w * 64 + l) // chunks) * chunks * 16
                + ((((w * 64 + l) % chunks) ^ b_swz(chunks, (w * 64 + l) // chunks)) << 4), 16)
               for l in range(64)], 16)
    for row in range(256):
        assert sorted(c ^ b_swz(chunks, row) for c in range(chunks)) == list(range(chunks))
        assert sorted((a_off(row, c) - row * 64) >> 4 for c in range(4)) == [0, 1, 2, 3]


def test_dma_lane_mapping_inverts_the_swizzle():
    """Direct-to-LDS: lane L of a wave writes byte 16*L of its 1 KB block, so it
    must fetch the logical chunk whose swizzled position is L's slot."""
    for block in range(16):
        for lane in range(64):
            arow = block * 16 + (lane >> 2)
            c = (lane & 3) ^ (((arow >> 1) ^ (arow >> 3)) & 3)
            assert a_off(arow, c) == block * 1024 + lane * 16
            brow = block * 4 + (lane >> 4)
            bc = (lane & 15) ^ b_swz(16, brow)
            assert brow * 256 + ((bc ^ b_swz(16, brow)) << 4) == block * 1024 + lane * 16
