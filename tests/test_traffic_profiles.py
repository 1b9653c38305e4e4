"""bench.py's HBM traffic figures agree with the committed rocprofv3 summaries.

bench.py reports `roofline.traffic` from FETCH_SIZE / WRITE_SIZE runs kept
under profiles/ (FETCH_SIZE scaled by the copy calibration's 2.00, WRITE_SIZE
by 1.00). These tests read the per-dispatch KiB figures out of those summaries
and check bench.py's constants against them, so refreshing a profile without
the constants (or the reverse) fails here instead of leaving a stale figure in
the bench line. CPU only; nothing here touches a GPU.
"""
import os
import re

import pytest

import bench

PROFILES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles")


def read(name):
    with open(os.path.join(PROFILES, name)) as fh:
        return fh.read()


def kib(text):
    return int(text.replace(",", ""))


def kernel_rows(name):
    """{kernel: (FETCH_SIZE KiB, WRITE_SIZE KiB)} from a summary's counter table
    (| kernel | FETCH_SIZE KiB | scaled | WRITE_SIZE KiB | reading |)."""
    rows = {}
    for line in read(name).splitlines():
        m = re.match(r"\|\s*(\w+)\s*\|\s*([\d,]+)\s*\|[^|]*\|\s*([\d,]+)\s*\|", line)
        if m:
            rows[m.group(1)] = (kib(m.group(2)), kib(m.group(3)))
    return rows


def test_copy_calibration_factors():
    text = read("copy_calibration_1GiB.md")
    assert re.search(r"\|\s*FETCH_SIZE\s*\|.*\*\*2\.00\*\*", text)
    assert re.search(r"\|\s*WRITE_SIZE\s*\|.*\*\*1\.00\*\*", text)


def test_gemm_traffic_matches_its_profile():
    # the headline kernel (K = 8192: gemm_dma16_kernel)
    text = read("gemm_dma16_256x256_8192cube.md")
    fetch = kib(re.search(r"\|\s*FETCH_SIZE\s*\|\s*([\d,]+) KiB", text).group(1))
    write = kib(re.search(r"\|\s*WRITE_SIZE\s*\|\s*([\d,]+) KiB", text).group(1))
    assert bench.TRAFFIC_GEMM_8192["read"] == pytest.approx(2.0 * fetch * 1024, rel=1e-3)
    assert bench.TRAFFIC_GEMM_8192["written"] == pytest.approx(write * 1024, rel=1e-3)


# (packed B, M) -> (summary, kernels of one step)
DECODE = {
    (False, 16): ("skinny_decode_m16_k4096_n14336.md", ("skinny_kernel",)),
    (True, 16): ("skinny_packed_m16_k4096_n14336.md", ("packed_skinny_kernel",)),
    (False, 1): ("decode_m1_k4096_n14336.md", ("skinny_kernel",)),
    (True, 1): ("decode_m1_k4096_n14336.md", ("packed_skinny_kernel",)),
}


@pytest.mark.parametrize("key", sorted(DECODE))
def test_decode_traffic_matches_its_profile(key):
    name, kernels = DECODE[key]
    rows = kernel_rows(name)
    fetch = sum(rows[k][0] for k in kernels)
    write = sum(rows[k][1] for k in kernels)
    want = bench.TRAFFIC_DECODE[key]
    # the constants are the summaries' figures rounded to 10 KB
    assert want["read"] == pytest.approx(2.0 * fetch * 1024, rel=2e-3, abs=1e4)
    assert want["written"] == pytest.approx(write * 1024, rel=2e-3, abs=1e4)


def test_every_decode_figure_has_traffic():
    assert set(bench.TRAFFIC_DECODE) == set(DECODE)


def test_planted_stale_constant_fails():
    """A constant off by 1 % (as after a kernel change) is caught."""
    rows = kernel_rows("skinny_packed_m16_k4096_n14336.md")
    measured = 2.0 * rows["packed_skinny_kernel"][0] * 1024
    assert measured * 1.01 != pytest.approx(measured, rel=2e-3, abs=1e4)
