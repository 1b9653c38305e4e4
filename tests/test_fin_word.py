"""The finishing word of a K-split decode sum finished inside the kernel.

skinny_kernel (FIN) finishes each output element of a K-split launch through
one 64-bit word: every slice adds (1 << 48) | partial (the int32 partial as an
unsigned 32-bit value) with one atomic add, and the slice whose add returns
k_split - 1 earlier arrivals writes C = D + (low 32 bits of the returned word
+ its partial) mod 2^32 and swaps the word back to 0. This CPU model checks
the arithmetic of that word for every arrival order that matters: the last
arrival, and only it, sees the count k_split - 1; its sum is the int32 sum of
all partials wrapped as vt_gemm_i8 promises; the carries out of the low 32
bits never reach the count (bits 32-47 hold fewer than 2^16 of them); and the
word returns to zero. A planted mistake (the count kept at bit 32, where the
carries land) must fail.
"""
import itertools

import numpy as np

COUNT_SHIFT = 48          # kFinCountShift in vt_hip_gemm.hip
MASK64 = (1 << 64) - 1


def finish(partials, order, shift=COUNT_SHIFT):
    """Replay the slices' atomic adds in `order`; return (C, final word,
    number of slices that saw themselves last)."""
    ks = len(partials)
    word, out, lasts = 0, None, 0
    for i in order:
        p = int(partials[i]) & 0xFFFFFFFF
        old = word
        word = (word + ((1 << shift) | p)) & MASK64
        if (old >> shift) == ks - 1:
            lasts += 1
            out = ((old & 0xFFFFFFFF) + p) & 0xFFFFFFFF
            word = 0                       # the last slice's swap
    if out is not None and out >= 1 << 31:
        out -= 1 << 32
    return out, word, lasts


def wrapped_sum(partials):
    s = int(np.sum(np.asarray(partials, dtype=np.int64))) & 0xFFFFFFFF
    return s - (1 << 32) if s >= 1 << 31 else s


def test_every_order_of_four_slices():
    rng = np.random.default_rng(3)
    for _ in range(50):
        parts = rng.integers(-2**31, 2**31, 4, dtype=np.int64)
        for order in itertools.permutations(range(4)):
            out, word, lasts = finish(parts, order)
            assert (out, word, lasts) == (wrapped_sum(parts), 0, 1)


def test_extreme_partials_and_many_slices():
    """Partials at the int32 extremes carry out of the low word on nearly
    every add; 64 and 4096 slices (the explicit k_split limit) still count
    exactly."""
    rng = np.random.default_rng(4)
    for ks in (2, 3, 64, 4096):
        for fill in (-2**31, 2**31 - 1, None):
            parts = (np.full(ks, fill, np.int64) if fill is not None
                     else rng.integers(-2**31, 2**31, ks, dtype=np.int64))
            order = rng.permutation(ks)
            assert finish(parts, order) == (wrapped_sum(parts), 0, 1), (ks, fill)


def test_count_beside_the_carries_is_a_planted_mistake():
    """With the count at bit 32 a carry from the low word is taken for an
    arrival: some slice other than the last decides it is last."""
    parts = np.full(4, -1, np.int64)        # 0xFFFFFFFF: every add after the first carries
    out, _, lasts = finish(parts, range(4), shift=32)
    assert lasts != 1 or out != wrapped_sum(parts)
