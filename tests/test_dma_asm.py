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

# (mangled name, fragment reads of one 32-deep k step): 4 A blocks plus the
# lo/hi halves of 4 row-major B blocks, or 4 whole packed B blocks
KERNELS = {"no_d": ("_ZN12_GLOBAL__N_115gemm_dma_kernelILi4ELb0ELb0EEEvNS_8GemmArgsE", 12),
           "with_d": ("_ZN12_GLOBAL__N_115gemm_dma_kernelILi4ELb1ELb0EEEvNS_8GemmArgsE", 12),
           "packed_b": ("_ZN12_GLOBAL__N_115gemm_dma_kernelILi4ELb0ELb1EEEvNS_8GemmArgsE", 8),
           "packed_b_with_d": ("_ZN12_GLOBAL__N_115gemm_dma_kernelILi4ELb1ELb1EEEvNS_8GemmArgsE", 8)}


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
