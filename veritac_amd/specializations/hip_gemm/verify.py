"""Exact device-side check of a GEMM result: C == D + A.B (mod 2^32).

The reference certifies its GEMM outputs by comparing every element with a
scalar matmul (examples/gemmini_gemm_demo.py:63-70,
benchmarks/gemmini/blind_search/2026-09-17/check_local_execution.py:47-52).
At the MI355X sizes (8192^3 is 5.5e11 multiply-adds) that comparison is the
work being measured, so this module checks the result on the GPU by
projection instead (Freivalds' method), in float64 arithmetic in which every
value involved is an integer below 2^53 and hence exact:

  * T projection vectors x with entries drawn uniformly from {0, 1}:
    C.x must equal D.x + A.(B.x) modulo 2^32. For any wrong result the
    residue of one wrong row differs from zero for at least one of the two
    values of the entry that meets a wrong element, so one vector misses
    with probability at most 1/2 and T vectors with at most 2^-T;
  * the all-ones projections on both sides (row and column checksums),
    which catch any single wrong element deterministically.

The comparison is modulo 2^32 because the contract is the wrapped int32 sum
(VeriTac/Gemmini/Word.lean:11, :31): outside the legality bound the GPU
result is the true product reduced to int32, and the check accepts exactly
that. It costs two float64 GEMMs with T columns plus a few reductions.
"""
from __future__ import annotations

WRAP = float(2 ** 32)
EXACT_LIMIT = 2 ** 53


class VerifyError(ValueError):
    """The shapes are inconsistent or exceed the float64 exactness bound."""


def _shapes(A, B, C, D):
    if A.dim() not in (2, 3) or B.dim() not in (2, 3) or C.dim() != A.dim():
        raise VerifyError("A, C must both be 2-D or both 3-D; B 2-D or 3-D")
    m, k = A.shape[-2:]
    n = B.shape[-1]
    if B.shape[-2] != k or tuple(C.shape[-2:]) != (m, n):
        raise VerifyError("shapes A%s B%s C%s do not compose" %
                          (tuple(A.shape), tuple(B.shape), tuple(C.shape)))
    if A.dim() == 3 and (C.shape[0] != A.shape[0] or (B.dim() == 3 and B.shape[0] != A.shape[0])):
        raise VerifyError("batch sizes differ")
    if A.dim() == 2 and B.dim() == 3:
        raise VerifyError("batched B needs batched A")
    if D is not None and tuple(D.shape) != tuple(C.shape):
        raise VerifyError("D has shape %s, C %s" % (tuple(D.shape), tuple(C.shape)))
    return m, n, k


def exactness_bound(m, n, k):
    """Largest magnitude any float64 intermediate of the check reaches."""
    ab = 128 * 128 * k * max(n, m)         # A.(B.x) and the checksums
    cd = 2 ** 31 * max(n, m) * 2            # C.x and D.x
    return ab + cd


def exact_check(A, B, C, D=None, *, vectors=16, seed=0):
    """Check C == D + A.B (mod 2^32) on the tensors' device; returns a dict.

    A int8 [.., m, k], B int8 [.., k, n] (2-D B is shared by all batches),
    C and the optional D int32 [.., m, n]. Raises VerifyError when the shapes
    do not compose or an intermediate could exceed 2^53.
    """
    import torch
    m, n, k = _shapes(A, B, C, D)
    bound = exactness_bound(m, n, k)
    if bound >= EXACT_LIMIT:
        raise VerifyError("m=%d n=%d k=%d: check intermediates reach %.3g >= 2^53" %
                          (m, n, k, bound))
    g = torch.Generator(device=A.device)
    g.manual_seed(seed)
    X = torch.randint(0, 2, (n, vectors), device=A.device, generator=g).double()
    Af, Bf, Cf = A.double(), B.double(), C.double()
    Df = None if D is None else D.double()

    def same_mod(lhs, rhs):
        return bool(torch.all(torch.remainder(lhs - rhs, WRAP) == 0))

    rhs = Af @ (Bf @ X)
    if Df is not None:
        rhs = rhs + Df @ X
    proj = same_mod(Cf @ X, rhs)
    col_rhs = Af.sum(-2, keepdim=True) @ Bf
    row_rhs = Af @ Bf.sum(-1, keepdim=True)
    if Df is not None:
        col_rhs = col_rhs + Df.sum(-2, keepdim=True)
        row_rhs = row_rhs + Df.sum(-1, keepdim=True)
    cols = same_mod(Cf.sum(-2, keepdim=True), col_rhs)
    rows = same_mod(Cf.sum(-1, keepdim=True), row_rhs)
    return {
        "method": "freivalds projections and checksums in float64, modulo 2^32",
        "vectors": vectors,
        "seed": seed,
        "projections_equal": proj,
        "checksums_equal": cols and rows,
        "passed": proj and cols and rows,
        "miss_probability_bound": 2.0 ** -vectors,
    }
