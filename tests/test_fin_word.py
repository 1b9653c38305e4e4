"""The finishing word of K-split decode sums finished inside the kernel.

skinny_kernel (FIN) finishes two output elements of a K-split launch (rows 2i
and 2i + 1 of one column) through one 64-bit word. A slice's partial over
k_chunk rows of int8 products lies in [-16256 k_chunk, 16384 k_chunk]; biased
by 16256 k_chunk it is a non-negative field value below 32640 k_chunk. Every
slice adds (1 << 2F) | hi << F | lo with one atomic add, F being the bit
length of 32640 k_chunk k_split, and the slice whose add returns k_split - 1
earlier arrivals (bits 2F-63) holds both exact sums: each field plus its own
biased partial, less k_split biases. It writes C = D + sum (mod 2^32) for
both rows and stores 0 back into the word.

This CPU model checks that arithmetic: for every arrival order that matters
the last arrival, and only it, sees the count k_split - 1; both sums are
exact at the extremes of the partial range and for partials of real int8
data; the fields never carry into each other or into the count; the word
returns to zero; and the host's choice of F (skinny_fin_bits in the HIP
source, mirrored by backend.skinny_finishes) refuses every split whose count
would not fit. Planted mistakes (a field one bit narrower, the count at bit F,
no bias) must fail.
"""
import itertools

import numpy as np

from veritac_amd.specializations.hip_gemm import backend as hg

BIAS = 16256              # kFinBiasPerRow in vt_hip_gemm.hip
SPAN = 16256 + 16384      # kFinSpanPerRow
MASK64 = (1 << 64) - 1


def fin_bits(ks, chunk):
    """skinny_fin_bits: the field width, or 0 when the count does not fit."""
    bits = (ks * chunk * SPAN).bit_length()
    return bits if 2 * bits + (ks - 1).bit_length() <= 64 else 0


def finish(p0, p1, chunk, order, bits=None, count_shift=None, bias=BIAS):
    """Replay the slices' atomic adds in `order`; return ((sum0, sum1) seen
    by the slice that found itself last, final word, number of such slices)."""
    ks = len(p0)
    F = fin_bits(ks, chunk) if bits is None else bits
    cs = 2 * F if count_shift is None else count_shift
    b = bias * chunk
    field = (1 << F) - 1
    word, out, lasts = 0, None, 0
    for i in order:
        lo, hi = int(p0[i]) + b, int(p1[i]) + b
        old = word
        word = (word + ((1 << cs) | (hi << F) | lo)) & MASK64
        if (old >> cs) == ks - 1:
            lasts += 1
            out = ((old & field) + lo - ks * b, ((old >> F) & field) + hi - ks * b)
            word = 0                       # the last slice's reset
    return out, word, lasts


def exact(p):
    return int(np.sum(np.asarray(p, dtype=np.int64)))


def test_every_order_of_four_slices():
    """The decode shape's split (K = 4096: four slices of 1024 rows)."""
    rng = np.random.default_rng(3)
    chunk = 1024
    assert fin_bits(4, chunk) == 27
    for _ in range(40):
        p0 = rng.integers(-BIAS * chunk, 16384 * chunk + 1, 4)
        p1 = rng.integers(-BIAS * chunk, 16384 * chunk + 1, 4)
        for order in itertools.permutations(range(4)):
            assert finish(p0, p1, chunk, order) == ((exact(p0), exact(p1)), 0, 1)


def largest_split(chunk):
    ks = 2
    while fin_bits(ks + 1, chunk):
        ks += 1
    return ks


def test_extreme_partials_up_to_the_largest_split():
    """Every partial at the top or bottom of its range (the fields at their
    largest), up to the largest split the count allows for the chunk."""
    rng = np.random.default_rng(4)
    for chunk in (128, 256, 1024, 8192):
        top = largest_split(chunk)
        assert fin_bits(top + 1, chunk) == 0
        for ks in sorted({2, 3, 4, 16, top}):
            if not fin_bits(ks, chunk):
                continue
            for lo, hi in ((16384, 16384), (-BIAS, -BIAS), (16384, -BIAS), (-BIAS, 16384)):
                p0, p1 = np.full(ks, lo * chunk), np.full(ks, hi * chunk)
                order = rng.permutation(ks)
                assert finish(p0, p1, chunk, order) == ((exact(p0), exact(p1)), 0, 1), (chunk, ks)


def test_partials_of_int8_data():
    """Two rows of int8 A against int8 B, K cut into k_chunk slices (the last
    slice short, as past K the kernel adds zero rows): the finished sums are
    the full dot products."""
    rng = np.random.default_rng(5)
    for K, chunk in ((4096, 1024), (8256, 256), (1000, 128), (4096, 2048)):
        ks = -(-K // chunk)
        assert fin_bits(ks, chunk)
        for fill in (None, -128, 127):
            A = (rng.integers(-128, 128, (2, K)) if fill is None else
                 np.full((2, K), fill)).astype(np.int64)
            B = (rng.integers(-128, 128, K) if fill is None else np.full(K, -128)).astype(np.int64)
            parts = [[int(A[r, s * chunk:(s + 1) * chunk] @ B[s * chunk:(s + 1) * chunk])
                      for s in range(ks)] for r in range(2)]
            order = rng.permutation(ks)
            out, word, lasts = finish(parts[0], parts[1], chunk, order)
            assert (out, word, lasts) == ((int(A[0] @ B), int(A[1] @ B)), 0, 1), (K, chunk, fill)


def test_host_rule_mirrors_the_model():
    """backend.skinny_finishes takes a split exactly when the model's field
    width is nonzero (and the rows and split qualify)."""
    for m, n, k, ks in ((1, 14336, 4096, 0), (16, 14336, 4096, 0), (4, 1040, 8256, 64),
                        (2, 4096, 65536, 0), (8, 1024, 131072, 2), (17, 14336, 4096, 0)):
        plan = hg.make_plan(m, n, k, variant="skinny", k_split=ks)
        split, chunk = hg.skinny_split(plan)
        want = split > 1 and m <= hg.SKINNY_FIN_MAX_M and fin_bits(split, chunk) > 0
        assert hg.skinny_finishes(plan) == want, (m, n, k, ks)


def test_planted_mistakes_fail():
    """A field one bit narrower than the host's choice carries into its
    neighbour at the extremes; the count at bit F (inside the high field)
    miscounts; without the bias a negative partial borrows from the field
    above."""
    chunk, ks = 1024, 4
    F = fin_bits(ks, chunk)
    top = np.full(ks, 16384 * chunk)
    bottom = np.full(ks, -BIAS * chunk)
    good = ((exact(top), exact(top)), 0, 1)
    assert finish(top, top, chunk, range(ks)) == good
    assert finish(top, top, chunk, range(ks), bits=F - 1) != good
    assert finish(top, top, chunk, range(ks), count_shift=F) != good
    assert finish(bottom, top, chunk, range(ks), bias=0) != ((exact(bottom), exact(top)), 0, 1)
