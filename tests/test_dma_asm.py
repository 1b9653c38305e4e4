"""The direct-to-LDS loads of gemm_dma_kernel are inline assembly the
compiler does not see into: each writes M0 and issues
global_load_lds_dwordx4, and the kernel's own s_waitcnt / s_barrier
sequences (not the compiler's wait insertion) order them against the LDS
reads. That is sound only while the compiler itself neither uses M0 in the
kernel nor inserts vmcnt waits into the k loop. This compiles the kernel
file for gfx950 to assembly, as the build does, and checks both, so a
compiler update that breaks either assumption fails here instead of on the
GPU. (The compiler's own LDS-DMA builtin is not used: it cannot tell which
LDS stage a DMA writes, so it waits for every outstanding DMA before the
fragment reads, which halves the kernel's speed.)"""
import os
import re
import shutil
import subprocess

import pytest

from veritac_amd import build as vb

def _k32(has_d, packed, edge=0):
    """gemm_dma_kernel<4, HAS_D, PACKED_B, EDGE>"""
    return "_ZN12_GLOBAL__N_115gemm_dma_kernelILi4ELb%dELb%dELb%dEEEvNS_8GemmArgsE" % (
        has_d, packed, edge)


# (mangled name, fragment reads of one 32-deep k step): 4 A blocks plus the
# lo/hi halves of 4 row-major B blocks, or 4 whole packed B blocks. The edge
# kinds move last tiles back and mask their stores.
KERNELS = {"no_d": (_k32(0, 0), 12), "with_d": (_k32(1, 0), 12),
           "packed_b": (_k32(0, 1), 8), "packed_b_with_d": (_k32(1, 1), 8),
           "edge": (_k32(0, 0, 1), 12), "edge_with_d": (_k32(1, 0, 1), 12),
           "packed_b_edge": (_k32(0, 1, 1), 8), "packed_b_edge_with_d": (_k32(1, 1, 1), 8)}


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    try:
        hipcc = vb.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "vt_hip_gemm.s")
    flags = [f for f in vb.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [hipcc] + flags + ["-I", vb.INCLUDE, "-S", "--cuda-device-only"] + vb.SOURCES + ["-o", out]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return open(out).read()


def kernel_body(asm, name):
    start = asm.index(name + ":")
    return asm[start:asm.index("s_endpgm", start)].split("\n")


@pytest.mark.parametrize("kind", sorted(KERNELS))
def test_m0_is_only_written_by_the_dma_sequences(asm, kind):
    body = [l.strip() for l in kernel_body(asm, KERNELS[kind][0])]
    dmas = 0
    for i, line in enumerate(body):
        if re.search(r"\bm0\b", line):
            # s_mov_b32 m0, sX ; s_nop 0 ; global_load_lds_dwordx4 vY, s[..]
            assert line.startswith("s_mov_b32 m0, s"), line
            assert body[i + 1].startswith("s_nop 0"), body[i + 1]
            assert body[i + 2].startswith("global_load_lds_dwordx4"), body[i + 2]
            dmas += 1
    # prologue (3 slices) and the k loop (one slice), 8 DMAs each per wave
    assert dmas == 32
    assert sum(l.startswith("global_load_lds_dwordx4") for l in body) == dmas


@pytest.mark.parametrize("kind", sorted(KERNELS))
def test_k_loop_waits_are_the_kernels_own(asm, kind):
    name, nunit = KERNELS[kind]
    body = [l.strip() for l in kernel_body(asm, name)]
    first_mfma = next(i for i, l in enumerate(body) if l.startswith("v_mfma"))
    last_mfma = max(i for i, l in enumerate(body) if l.startswith("v_mfma"))
    # the k loop runs from its first MFMA to the slice barrier after its last
    end = next(i for i in range(last_mfma, len(body)) if body[i].startswith("s_barrier"))
    loop = body[first_mfma:end + 1]
    # the slice barrier: only slice g+3's 8 DMAs may be in flight, and only
    # the next step's early fragment reads
    assert loop[-2:] == ["s_waitcnt vmcnt(8) lgkmcnt(%d)" % nunit, "s_barrier"]
    assert not [l for l in loop if re.match(r"s_waitcnt .*vmcnt\(0\)", l)]


# gemm_dma16_kernel<HAS_D, PACKED_B>: the same DMA discipline, plus MFMAs
# issued as inline asm (v_mfma_i32_16x16x64_i8 accumulating in place in
# AGPRs), whose hazards the compiler does not check. The kernel fences them
# itself: s_nop 7 pairs between the accumulators' zeroing (v_accvgpr_write)
# and the next MFMA, and three s_nop 7 between the last MFMA of a tile and
# the epilogue's reads of the AGPRs.
def _k16(has_d, packed, edge=0, bn=256):
    return "_ZN12_GLOBAL__N_117gemm_dma16_kernelILb%dELb%dELb%dELi%dEEEvNS_8GemmArgsE" % (
        has_d, packed, edge, bn)


# gemm_dma16_kernel<HAS_D, PACKED_B, EDGE, BN>
KERNELS16 = {"no_d": _k16(0, 0), "with_d": _k16(1, 0), "packed_b": _k16(0, 1),
             "packed_b_with_d": _k16(1, 1), "edge": _k16(0, 0, 1), "edge_with_d": _k16(1, 0, 1),
             "packed_b_edge": _k16(0, 1, 1), "packed_b_edge_with_d": _k16(1, 1, 1),
             "bn128": _k16(0, 0, 0, 128), "bn128_with_d": _k16(1, 0, 0, 128),
             "bn128_edge": _k16(0, 0, 1, 128), "bn128_edge_with_d": _k16(1, 0, 1, 128),
             "bn128_packed": _k16(0, 1, 0, 128), "bn128_packed_with_d": _k16(1, 1, 0, 128),
             "bn128_packed_edge": _k16(0, 1, 1, 128), "bn128_packed_edge_with_d": _k16(1, 1, 1, 128)}
# kinds whose tile's last k iteration is peeled to store early strips: no D,
# and all tiles whole (the edge kinds mask their stores after the loop)
EARLY16 = {"no_d", "packed_b"}
# the 256x128 form: 4 A and 2 B DMAs per wave per slice, 8 x 4 MFMAs per step
BN128 = {k for k in KERNELS16 if k.startswith("bn128")}


def dmas_per_slice(kind):
    return 6 if kind in BN128 else 8


def mfmas_per_step(kind):
    return 32 if kind in BN128 else 64


def instructions(asm, name):
    return [l.strip() for l in kernel_body(asm, name)
            if l.strip() and not l.strip().startswith((";", "."))]


@pytest.mark.parametrize("kind", sorted(KERNELS16))
def test_dma16_m0_is_only_written_by_the_dma_sequences(asm, kind):
    body = instructions(asm, KERNELS16[kind])
    dmas = 0
    for i, line in enumerate(body):
        if re.search(r"\bm0\b", line):
            assert line.startswith("s_mov_b32 m0, s"), line
            assert body[i + 1].startswith("s_nop 0"), body[i + 1]
            assert body[i + 2].startswith("global_load_lds_dwordx4"), body[i + 2]
            dmas += 1
    # prologue (3 slices) and the k loop unrolled over the 4 stages, 8 DMAs
    # per wave per slice (6 in the 256x128 form); with early strips the
    # tile's last iteration is a second, peeled copy of the loop body
    assert dmas == (3 + 4 + (4 if kind in EARLY16 else 0)) * dmas_per_slice(kind)
    assert sum(l.startswith("global_load_lds_dwordx4") for l in body) == dmas


@pytest.mark.parametrize("kind", sorted(KERNELS16))
def test_dma16_slice_barriers_and_no_full_waits_in_the_k_loop(asm, kind):
    body = instructions(asm, KERNELS16[kind])
    mfma = [i for i, l in enumerate(body) if l.startswith("v_mfma")]
    # 4 unrolled steps of 8 x 8 MFMAs accumulating in place (and without D
    # the peeled last iteration's 4)
    loop_mfma = [i for i in mfma if re.match(r"v_mfma_i32_16x16x64_i8 (a\[\d+:\d+\]), v.*, \1$", body[i])]
    steps = 8 if kind in EARLY16 else 4
    assert len(loop_mfma) == len(mfma) == steps * mfmas_per_step(kind)
    loop = body[loop_mfma[0]:loop_mfma[-1] + 1]
    assert not [l for l in loop if re.match(r"s_waitcnt .*vmcnt\(0\)", l)]
    # every slice barrier waits for all but the slice's own DMAs; the tile's
    # last step also leaves the 6 early strips' 8 stores each
    own = "s_waitcnt vmcnt(%d)" % dmas_per_slice(kind)
    waits = [body[i - 1] for i in range(loop_mfma[0], loop_mfma[-1] + 8) if body[i] == "s_barrier"]
    want = [own] * 7 + ["s_waitcnt vmcnt(56)"] if kind in EARLY16 else [own] * 4
    assert sorted(waits) == sorted(want), waits


def _agprs(text):
    """AGPR numbers named in an operand list (a7, a[4:7])."""
    regs = set()
    for lo, hi, one in re.findall(r"\ba\[(\d+):(\d+)\]|\ba(\d+)\b", text):
        regs.update(range(int(lo), int(hi) + 1) if lo else {int(one)})
    return regs


def _mfma_regs(line):
    """(accumulator written, accumulator read as srcC) of an MFMA line."""
    ops = line.split(None, 1)[1].split(", ")
    return _agprs(ops[0]), _agprs(ops[-1])


def _agpr_reads(line):
    if line.startswith("v_accvgpr_read"):
        return _agprs(line.split(", ", 1)[1])
    if line.startswith(("global_store", "buffer_store", "ds_write")):
        return _agprs(line.split(None, 1)[1])
    return set()


def fence_violations(body, far=8):
    """Accumulator writes (v_accvgpr_write) with fewer than two s_nop 7 and
    fewer than `far` MFMAs before the next MFMA that reads the register, and
    AGPR reads with fewer than three s_nop 7 and fewer than `far` MFMAs since
    the MFMA that wrote it (in layout order)."""
    bad = []
    mfma = [(i,) + _mfma_regs(l) for i, l in enumerate(body) if l.startswith("v_mfma")]
    nops = [0]
    for line in body:
        nops.append(nops[-1] + (line == "s_nop 7"))
    for i, line in enumerate(body):
        if line.startswith("v_accvgpr_write"):
            reg = _agprs(line.split(",")[0])
            later = [m for m in mfma if m[0] > i]
            hit = next((k for k, m in enumerate(later) if m[2] & reg), None)
            if hit is not None and hit < far and nops[later[hit][0]] - nops[i] < 2:
                bad.append((i, line))
        reads = _agpr_reads(line)
        if reads:
            earlier = [m for m in mfma if m[0] < i]
            hit = next((k for k, m in enumerate(reversed(earlier)) if m[1] & reads), None)
            if hit is not None and hit < far and nops[i] - nops[earlier[-1 - hit][0]] < 3:
                bad.append((i, line))
    return bad


@pytest.mark.parametrize("kind", sorted(KERNELS16))
def test_dma16_mfma_hazards_are_fenced(asm, kind):
    assert fence_violations(instructions(asm, KERNELS16[kind])) == []


def test_fence_check_catches_missing_nops():
    mf = "v_mfma_i32_16x16x64_i8 a[0:3], v[0:3], v[4:7], a[0:3]"
    ok = ["v_accvgpr_write_b32 a0, 0", "s_nop 7", "s_nop 7", mf,
          "s_nop 7", "s_nop 7", "s_nop 7", "global_store_dword v[0:1], a0, off nt"]
    assert fence_violations(ok) == []
    assert fence_violations(ok[:2] + ok[3:]) == [(0, ok[0])]                 # one nop short
    assert fence_violations(ok[:5] + ok[6:]) == [(6, ok[7])]                 # store too early
    assert fence_violations(ok[:4] + ["v_accvgpr_read_b32 v0, a0"]) != []
    # distance in MFMAs on other accumulators counts as a fence
    other = "v_mfma_i32_16x16x64_i8 a[4:7], v[0:3], v[4:7], a[4:7]"
    assert fence_violations(["v_accvgpr_write_b32 a0, v1"] + [other] * 8 + [mf]) == []
    assert fence_violations(["v_accvgpr_write_b32 a0, v1"] + [other] * 3 + [mf]) != []
    assert fence_violations([mf] + [other] * 8 + ["v_accvgpr_read_b32 v0, a2"]) == []
    assert fence_violations([mf] + [other] * 2 + ["v_accvgpr_read_b32 v0, a2"]) != []
