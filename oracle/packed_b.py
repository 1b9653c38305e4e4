"""CPU restatement of the packed-B weight layout (TEST INFRASTRUCTURE ONLY).

The packed layout is this build's own format for the decode-shaped GEMM
(include/vt_hip_gemm.h, "Packed-B decode path"); the reference keeps weights
row-major and has no counterpart. What the format must preserve is the
reference's GEMM, C[r,c] = sum_t A[r*k+t] * B[t*n+c]
(VeriTac/Gemmini/Semantics.lean:76-77, specializations/gemmini_gemm/
backend.py:569-580), so every function here is pinned by that product, not
by restating the byte formula:

  pack_b / unpack_b   unpack_b(pack_b(B)) == B for every shape, and every
                      byte of the padding rows is zero;
  gemm_from_packed    reads the packed bytes under the operand convention of
                      v_mfma_i32_16x16x64_i8 (B operand: lane l holds column
                      l % 16, k = 16*(l//16) .. +15 of a 64-deep block) and
                      must equal the closed-form int64 A @ B. A transposed
                      tile, a swapped lane mapping or a wrong block order
                      fails it (tests/test_packed_host.py plants each).

Only tests/ may import this module.
"""
from __future__ import annotations

import numpy as np

TILE = 1024          # bytes of one packed tile: 64 rows x 16 columns
KBLK, NBLK = 64, 16  # rows and columns one tile covers


def packed_size(k, n):
    """Bytes of one packed B: n * (k rounded up to a multiple of 64)."""
    if n % NBLK:
        raise ValueError("n must be a multiple of 16")
    return n * (-(-k // KBLK) * KBLK)


def pack_b(B):
    """Row-major int8 B [k, n] -> packed bytes (int8, flat).

    Tile (nb, kb) sits at (nb * kbt + kb) * 1024; inside it lane l's 16 bytes
    are column nb*16 + l%16 over rows kb*64 + 16*(l//16) .. +15.
    """
    B = np.asarray(B, dtype=np.int8)
    k, n = B.shape
    kbt = -(-k // KBLK)
    pad = np.zeros((kbt * KBLK, n), np.int8)
    pad[:k] = B
    # [kbt, 4 (k group), 16 (i), nbt, 16 (column in block)]
    t = pad.reshape(kbt, 4, 16, n // NBLK, NBLK)
    # -> [nbt, kbt, 4 (k group), 16 (column), 16 (i)]: lane = kgroup*16 + column
    t = t.transpose(3, 0, 1, 4, 2)
    return np.ascontiguousarray(t).reshape(-1)


def unpack_b(Bp, k, n):
    """Packed bytes -> row-major int8 B [k, n] (inverse of pack_b)."""
    kbt = -(-k // KBLK)
    t = np.asarray(Bp, dtype=np.int8).reshape(n // NBLK, kbt, 4, NBLK, 16)
    full = t.transpose(1, 2, 4, 0, 3).reshape(kbt * KBLK, n)
    return np.ascontiguousarray(full[:k])


def gemm_from_packed(A, Bp, k, n):
    """C = A @ B computed from packed B the way the MFMA consumes it.

    For every 16-column block and 64-row block, lane l of the B operand is
    the 16 bytes at tile offset l*16: column l % 16 of the block, rows
    16*(l//16) .. +15. The A operand of the same lane group covers the same
    16 rows of k. int64 accumulation, cast to int32 (wrapping).
    """
    A = np.asarray(A, dtype=np.int64)
    m = A.shape[0]
    kbt = -(-k // KBLK)
    Apad = np.zeros((m, kbt * KBLK), np.int64)
    Apad[:, :k] = A
    tiles = np.asarray(Bp, dtype=np.int8).reshape(n // NBLK, kbt, 64, 16).astype(np.int64)
    C = np.zeros((m, n), np.int64)
    for nb in range(n // NBLK):
        for kb in range(kbt):
            for lane in range(64):
                col = nb * NBLK + lane % 16
                k0 = kb * KBLK + 16 * (lane // 16)
                C[:, col] += Apad[:, k0:k0 + 16] @ tiles[nb, kb, lane]
    return C.astype(np.int32)
