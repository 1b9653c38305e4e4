"""Model check of the LDS layouts in csrc/vt_hip_gemm.hip (host only).

Bank model of gfx950's LDS, measured on an MI355X with SQ_LDS_BANK_CONFLICT
(two active lanes, the second reading the first one's bank 256 or 512 bytes
further on): 64 banks of 4 bytes; a 16-byte read serves four groups of 16
lanes, lane L in group parity((L >> 2) & 7) + 2 * (L >> 5); an 8-byte read
(ds_read_b64, ds_read_b64_tr_b8) serves lanes 0-31, then 32-63. An access is
conflict-free when each group touches distinct banks.

The address formulas below restate the kernels' (a_off, b_swz,
skinny_a_stride and the fragment / staging offsets). Each test checks
one kernel access pattern, so a swizzle change that reintroduces a conflict
fails here. The first tests pin the model itself: the plain linear pattern
must pass it, and the A swizzle used before this model was measured must fail it.
"""
import pytest

from veritac_amd.specializations.hip_gemm.backend import skinny_a_stride


def group_b128(lane):
    return bin((lane >> 2) & 7).count("1") % 2 + 2 * (lane >> 5)


def group_b64(lane):
    return lane >> 5


def conflicts(addrs, nbytes):
    """Extra bank cycles of one wave-wide access (0 = conflict-free)."""
    group = group_b128 if nbytes == 16 else group_b64
    worst = 0
    for g in set(group(l) for l in range(64)):
        banks = {}
        for lane, addr in enumerate(addrs):
            if group(lane) != g:
                continue
            for w in range(nbytes // 4):
                b = (addr // 4 + w) % 64
                banks[b] = banks.get(b, 0) + 1
        worst = max(worst, max(banks.values()) - 1)
    return worst


def a_swz(row):
    return (row >> 2) & 3


def a_off(row, c):
    return row * 64 + ((c ^ a_swz(row)) << 4)


def b_swz(chunks, row):
    if chunks >= 16:
        return ((row & 7) << 1) | ((row >> 2) & 1)
    if chunks == 8:
        return row & 7
    return (row >> 1) & 3


def test_model_linear_is_conflict_free_and_old_a_swizzle_is_not():
    assert conflicts([16 * l for l in range(64)], 16) == 0
    assert conflicts([8 * l for l in range(64)], 8) == 0
    assert conflicts([32 * l for l in range(64)], 16) == 1

    def old(row, c):
        return row * 64 + ((c ^ (((row >> 1) ^ (row >> 3)) & 3)) << 4)
    assert conflicts([old(l & 31, l >> 5) for l in range(64)], 16) == 1


@pytest.mark.parametrize("wtm", [32, 64, 128])
def test_a_fragment_reads_conflict_free(wtm):
    """32x32x32 A operand: lane l reads row l % 32, k chunk ks*2 + l / 32."""
    for wm in (0, 1):
        for mi in range(wtm // 32):
            for ks in (0, 1):
                addrs = [a_off(wm * wtm + mi * 32 + (l & 31), ks * 2 + (l >> 5)) for l in range(64)]
                assert conflicts(addrs, 16) == 0


@pytest.mark.parametrize("bn", [64, 128, 256])
def test_b_fragment_reads_conflict_free(bn):
    """ds_read_b64_tr_b8: 16-lane group g reads rows (g>>1)*16 + j/2, chunk nc + (g&1)."""
    chunks = bn // 16
    for wn in (0, 1):
        for ni in range(bn // 2 // 32):
            for ks in (0, 1):
                for half in (0, 8):
                    addrs = []
                    for lane in range(64):
                        g, j = lane >> 4, lane & 15
                        nc = (wn * bn // 2 + ni * 32) // 16 + (g & 1)
                        r0 = ks * 32 + (g >> 1) * 16 + (j >> 1)
                        addrs.append((r0 + half) * bn + ((nc ^ b_swz(chunks, r0 + half)) << 4) + (j & 1) * 8)
                    assert conflicts(addrs, 8) == 0


@pytest.mark.parametrize("bn", [64, 128, 256])
def test_vgpr_staged_writes_conflict_free(bn):
    """gemm_mfma_kernel: thread t stores A row t/4 chunk t%4 and B row t/chunks."""
    chunks = bn // 16
    for w in range(4):
        tids = [w * 64 + l for l in range(64)]
        assert conflicts([a_off(t >> 2, t & 3) for t in tids], 16) == 0
        assert conflicts([(t // chunks) * bn + (((t % chunks) ^ b_swz(chunks, t // chunks)) << 4)
                          for t in tids], 16) == 0


def test_dma_lane_mapping_inverts_the_swizzle():
    """Direct-to-LDS: lane L of a wave writes byte 16*L of its 1 KB block, so it
    must fetch the logical chunk whose swizzled position is L's slot."""
    for block in range(16):
        for lane in range(64):
            arow = block * 16 + (lane >> 2)
            c = (lane & 3) ^ a_swz(arow)
            assert a_off(arow, c) == block * 1024 + lane * 16
            brow = block * 4 + (lane >> 4)
            bc = (lane & 15) ^ b_swz(16, brow)
            assert brow * 256 + ((bc ^ b_swz(16, brow)) << 4) == block * 1024 + lane * 16


@pytest.mark.parametrize("k_chunk", [128, 256, 384, 1024, 1152, 4096])
def test_skinny_a_reads_conflict_free(k_chunk):
    """16x16x64 A operand from the [16][stride] slice: lane l reads row l % 16,
    chunk l / 16 of the wave's 64-byte k block."""
    stride = skinny_a_stride(k_chunk)
    assert stride % 16 == 0 and k_chunk <= stride < k_chunk + 64
    for kb in range(4):
        for s in range(0, k_chunk, 64):
            addrs = [(l & 15) * stride + s + kb * 64 + (l >> 4) * 16 for l in range(64)]
            if s + kb * 64 + 64 <= k_chunk:
                assert conflicts(addrs, 16) == 0


def test_swizzles_are_permutations():
    for row in range(256):
        assert sorted(c ^ a_swz(row) for c in range(4)) == [0, 1, 2, 3]
        for chunks in (4, 8, 16):
            assert sorted(c ^ b_swz(chunks, row) for c in range(chunks)) == list(range(chunks))


def skinny_b_swz(row):
    return (row & 7) | (((row >> 4) & 1) << 3)


def test_skinny_b_stage_conflict_free():
    """skinny_kernel<256,...>: thread t stores row t/16 chunk t%16 of a 64-row
    stage; wave (kb, nblk) reads rows kb*64 + g*16 + j/2 (+8) of chunk nblk."""
    for w in range(16):
        tids = [w * 64 + l for l in range(64)]
        assert conflicts([(t // 16) * 256 + (((t % 16) ^ skinny_b_swz(t // 16)) << 4) for t in tids], 16) == 0
    for kb in range(1):
        for nblk in range(16):
            for half in (0, 8):
                addrs = []
                for lane in range(64):
                    g, j = lane >> 4, lane & 15
                    r0 = kb * 64 + g * 16 + (j >> 1) + half
                    addrs.append(r0 * 256 + ((nblk ^ skinny_b_swz(r0)) << 4) + (j & 1) * 8)
                assert conflicts(addrs, 8) == 0
    for row in range(64):
        assert sorted(c ^ skinny_b_swz(row) for c in range(16)) == list(range(16))


def strip_off(row, chunk):
    return row * 512 + ((chunk ^ (((row >> 2) & 3) << 2)) << 4)


def conflicts_b32(addrs):
    """Extra bank cycles of a wave-wide 4-byte access, all 64 lanes served
    together (the epilogue profile reads SQ_LDS_BANK_CONFLICT = 0 for it)."""
    banks = {}
    for addr in addrs:
        banks[(addr // 4) % 64] = banks.get((addr // 4) % 64, 0) + 1
    return max(banks.values()) - 1


def strip_write_addr(lane, ni, e):
    """store_tile16_lds: element e of lane l of 16x16 block ni (row 4*(l/16)+e,
    column l%16) goes to strip row 4*(l/16)+e, 4-byte word ni*16 + l%16."""
    c, g = lane & 15, lane >> 4
    return strip_off(4 * g + e, ni * 4 + (c >> 2)) + (c & 3) * 4


def strip_read_addr(lane, j):
    """Read j: lane l takes 16 bytes of strip row 2*j + l/32, chunk l%32."""
    return strip_off(2 * j + (lane >> 5), lane & 31)


def test_epilogue_strip_is_a_permutation():
    offs = sorted(strip_off(r, c) for r in range(16) for c in range(32))
    assert offs == [16 * i for i in range(512)]


def test_epilogue_strip_conflict_free():
    for ni in range(8):
        for e in range(4):
            assert conflicts_b32([strip_write_addr(l, ni, e) for l in range(64)]) == 0
    for j in range(8):
        assert conflicts([strip_read_addr(l, j) for l in range(64)], 16) == 0
    # unswizzled, every write of one instruction hits 4 lanes per bank
    assert conflicts_b32([(4 * (l >> 4) + e) * 512 + ni * 64 + (l & 15) * 4
                          for l in range(64) for ni, e in [(0, 0)]]) == 3


def simulate_epilogue(acc, write=strip_write_addr, read=strip_read_addr):
    """acc[ni][lane][e] (one 16-row strip of a wave's 16 x 128 block) -> the
    16 x 128 int32 rows the stores write: read j of lane l goes to row
    2*j + l/32, columns 4*(l%32) .. +3."""
    import numpy as np
    lds = np.zeros(8192 // 4, np.int64)
    for ni in range(8):
        for lane in range(64):
            for e in range(4):
                lds[write(lane, ni, e) // 4] = acc[ni][lane][e]
    out = np.zeros((16, 128), np.int64)
    for j in range(8):
        for lane in range(64):
            a = read(lane, j) // 4
            out[2 * j + (lane >> 5), 4 * (lane & 31):4 * (lane & 31) + 4] = lds[a:a + 4]
    return out


def test_epilogue_round_trip_matches_accumulator_layout():
    """Values placed by the v_mfma_i32_16x16x64_i8 accumulator layout (element
    e of lane l of block ni is row 4*(l/16)+e, column 16*ni + l%16) come back as
    the row-major strip; planted index mistakes do not."""
    import numpy as np
    want = np.arange(16 * 128, dtype=np.int64).reshape(16, 128) * 7 - 5000
    acc = [[[want[4 * (l >> 4) + e, 16 * ni + (l & 15)] for e in range(4)] for l in range(64)]
           for ni in range(8)]
    assert np.array_equal(simulate_epilogue(acc), want)
    swapped = lambda lane, ni, e: strip_off(4 * e + (lane >> 4), ni * 4 + ((lane & 15) >> 2)) + (lane & 3) * 4
    assert not np.array_equal(simulate_epilogue(acc, write=swapped), want)
    unswizzled_read = lambda lane, j: (2 * j + (lane >> 5)) * 512 + (lane & 31) * 16
    assert not np.array_equal(simulate_epilogue(acc, read=unswizzled_read), want)


def test_strip_lane_bases_equal_strip_off():
    """The epilogue addresses the strip as per-lane bases plus immediate
    offsets (strip_lanes in vt_hip_gemm.hip): writes wb[ni % 4] + 512 e +
    64 (ni & 4), reads rb[j / 2] + 1024 j. Both equal strip_off's layout."""
    for lane in range(64):
        g = lane >> 4
        wb = [2048 * g + (((k ^ g) & 3) << 6) + (lane & 15) * 4 for k in range(4)]
        rb = [512 * (lane >> 5) + (((lane & 31) ^ (m << 2)) << 4) for m in range(4)]
        for ni in range(8):
            for e in range(4):
                assert wb[ni & 3] + 512 * e + 64 * (ni & 4) == strip_write_addr(lane, ni, e)
                assert 512 * e + 64 * (ni & 4) < 65536
        for j in range(8):
            assert rb[j >> 1] + 1024 * j == strip_read_addr(lane, j)


# gemm_dma16_kernel (16x16x64, slices filled by direct-to-LDS loads): A slice
# [256][64 B] (a16_swz), B slice [64][BN B] row-major (b16_swz for the 256-wide
# tile, b8_swz for the 256x128 form), and the 256x128 form's 64-column
# epilogue strip (strip64_off).
def a16_swz(row):
    return ((row >> 3) & 1) << 1


def a16_off(row, c):
    return row * 64 + ((c ^ a16_swz(row)) << 4)


def b16_swz(row):
    return (row & 7) | (((row >> 4) & 1) << 3)


def b8_swz(row):
    return ((row >> 1) & 3) | (((row >> 4) & 1) << 2)


DMA16_B = {256: b16_swz, 128: b8_swz}


def test_dma16_a_fragment_reads_conflict_free():
    """Lane l reads row wm*128 + mi*16 + l%16, chunk l/16."""
    for wm in (0, 1):
        for mi in range(8):
            assert conflicts([a16_off(wm * 128 + mi * 16 + (l & 15), l >> 4) for l in range(64)], 16) == 0


@pytest.mark.parametrize("bn", [256, 128])
def test_dma16_b_fragment_reads_conflict_free(bn):
    """ds_read_b64_tr_b8 of block ni (columns cb*16 ..): lane l reads 8 bytes
    of row 16*(l/16) + (l%16)/2 (+ 8 for the high half), chunk cb, byte 8*(l&1)."""
    swz = DMA16_B[bn]
    for cb in range(bn // 16):
        for half in (0, 8):
            addrs = []
            for l in range(64):
                row = 16 * (l >> 4) + ((l & 15) >> 1) + half
                addrs.append(row * bn + ((cb ^ swz(row)) << 4) + (l & 1) * 8)
            assert conflicts(addrs, 8) == 0, (cb, half)
    if bn == 128:
        # the 256-wide swizzle's low three bits alone conflict on 128-byte rows
        plain = lambda row: row & 7
        addrs = [(16 * (l >> 4) + ((l & 15) >> 1)) * 128 + ((0 ^ plain(16 * (l >> 4) + ((l & 15) >> 1))) << 4)
                 + (l & 1) * 8 for l in range(64)]
        assert conflicts(addrs, 8) > 0


@pytest.mark.parametrize("bn", [256, 128])
def test_dma16_lane_mapping_inverts_the_swizzles(bn):
    """Lane L of a 1 KB DMA block writes byte 16 L; the global chunk it fetches
    must be the one the swizzle stores there (A: 16 rows of 64 B per block;
    B: 1024 / bn rows of bn bytes)."""
    swz = DMA16_B[bn]
    per = 1024 // bn
    slots = bn // 16
    for block in range(16):
        for lane in range(64):
            arow = block * 16 + (lane >> 2)
            assert a16_off(arow, (lane & 3) ^ a16_swz(arow)) == block * 1024 + lane * 16
        if block * per >= 64:
            continue
        for lane in range(64):
            brow = block * per + lane // slots
            bc = (lane % slots) ^ swz(brow)
            assert brow * bn + ((bc ^ swz(brow)) << 4) == block * 1024 + lane * 16
            assert 0 <= bc < slots


def strip64_off(row, chunk):
    return row * 256 + ((chunk ^ (((row >> 2) & 3) << 2)) << 4)


def strip64_write_addr(lane, ni, e):
    """Element e of block ni: strip row 4*(l/16)+e, 4-byte word 16*ni + l%16."""
    g, c = lane >> 4, lane & 15
    return strip64_off(4 * g + e, ni * 4 + (c >> 2)) + (c & 3) * 4


def strip64_read_addr(lane, j):
    """Read j: lane l takes 16 bytes of strip row 4*j + l/16, chunk l%16."""
    return strip64_off(4 * j + (lane >> 4), lane & 15)


def test_strip64_is_a_permutation_and_conflict_free():
    assert sorted(strip64_off(r, c) for r in range(16) for c in range(16)) == list(range(0, 4096, 16))
    for ni in range(4):
        for e in range(4):
            assert conflicts_b32([strip64_write_addr(l, ni, e) for l in range(64)]) == 0
    for j in range(4):
        assert conflicts([strip64_read_addr(l, j) for l in range(64)], 16) == 0
    # unswizzled, each write instruction puts 4 lanes on every bank it uses
    assert conflicts_b32([(4 * (l >> 4)) * 256 + (l & 15) * 4 for l in range(64)]) == 3


def test_strip64_round_trip_and_lane_bases():
    """The accumulator layout comes back as the row-major 16 x 64 strip (read j
    of lane l is row 4*j + l/16, columns 4*(l%16) ..); the per-lane bases of
    the kernel (strip64_wb + 256 e, strip64_rb + 1024 j) equal the layout."""
    import numpy as np
    want = np.arange(16 * 64, dtype=np.int64).reshape(16, 64) * 11 - 3000
    lds = np.zeros(1024, np.int64)
    for ni in range(4):
        for l in range(64):
            for e in range(4):
                lds[strip64_write_addr(l, ni, e) // 4] = want[4 * (l >> 4) + e, 16 * ni + (l & 15)]
    out = np.zeros((16, 64), np.int64)
    for j in range(4):
        for l in range(64):
            a = strip64_read_addr(l, j) // 4
            out[4 * j + (l >> 4), 4 * (l & 15):4 * (l & 15) + 4] = lds[a:a + 4]
    assert np.array_equal(out, want)
    for l in range(64):
        g = l >> 4
        for ni in range(4):
            for e in range(4):
                assert 1024 * g + 64 * (ni ^ g) + 4 * (l & 15) + 256 * e == strip64_write_addr(l, ni, e)
        for j in range(4):
            assert 256 * g + (((l & 15) ^ (4 * j)) << 4) + 1024 * j == strip64_read_addr(l, j)
