"""Deterministic int8 GEMM inputs: the reference's generators and the five
benchmark configurations.

deterministic_inputs mirrors specializations/gemmini_gemm/backend.py:583-602
(same name, arguments, modes and value stream), vectorised with numpy.
lcg8_bytes / spike_inputs mirror the Spike harness patterns of
specializations/gemmini_gemm/runtime/run_raw_spike.py:133-151.
config_inputs builds the five workloads of the benchmark configurations
(seeded numpy generators, int8 row-major, int32 D).
"""
from __future__ import annotations

import numpy as np

ELEM_MIN, ELEM_MAX = -128, 127
_LCG_A, _LCG_C = 1103515245, 12345


def _lcg_states(seed, count):
    """States x_1..x_count of x <- 1103515245 x + 12345 (mod 2^32), x_0 = seed.

    Computed in blocks with the affine-map jump x_{i+s} = A_s x_i + C_s so a
    multi-million-element stream costs a few numpy passes.
    """
    out = np.empty(count, dtype=np.uint64)
    if count == 0:
        return out
    block = min(count, 4096)
    # first block sequentially
    x = seed & 0xFFFFFFFF
    for i in range(block):
        x = (_LCG_A * x + _LCG_C) & 0xFFFFFFFF
        out[i] = x
    # jump coefficients for a stride of `block`
    a_s, c_s = 1, 0
    for _ in range(block):
        a_s, c_s = (_LCG_A * a_s) & 0xFFFFFFFF, (_LCG_A * c_s + _LCG_C) & 0xFFFFFFFF
    mask = np.uint64(0xFFFFFFFF)
    done = block
    while done < count:
        n = min(block, count - done)
        prev = out[done - block:done - block + n]
        out[done:done + n] = (prev * np.uint64(a_s) + np.uint64(c_s)) & mask
        done += n
    return out


def deterministic_inputs(m, n, k, seed, mode="lcg"):
    """int8 arrays A [m,k] and B [k,n] (backend.py:583-602 as numpy).

    lcg: value ((x >> 16) % 256) - 128 over one stream, A first then B;
    max / minmax / min / zero: constant fills.
    """
    if mode == "lcg":
        states = _lcg_states(seed, m * k + k * n)
        vals = (((states >> np.uint64(16)) % np.uint64(256)).astype(np.int16) - 128).astype(np.int8)
        return vals[:m * k].reshape(m, k), vals[m * k:].reshape(k, n)
    fills = {"max": (ELEM_MAX, ELEM_MAX), "minmax": (ELEM_MIN, ELEM_MAX),
             "min": (ELEM_MIN, ELEM_MIN), "zero": (0, 0)}
    if mode not in fills:
        raise ValueError(mode)
    a, b = fills[mode]
    return np.full((m, k), a, dtype=np.int8), np.full((k, n), b, dtype=np.int8)


def lcg8_bytes(count, seed=0x12345678):
    """Bytes (x >> 16) & 0xFF of the Spike harness stream (run_raw_spike.py:133-138)."""
    return ((_lcg_states(seed, count) >> np.uint64(16)) & np.uint64(0xFF)).astype(np.uint8)


def spike_inputs(mode, m, n, k):
    """A [m,k], B [k,n] int8 for the Spike modes zeros / extrema / lcg.

    run_raw_spike.py:141-151: extrema alternates 0x80,0x7F in A and 0x7F,0x80
    in B over the flat buffers; lcg is one lcg8 stream, A then B; bytes are
    read as two's-complement int8 (run_raw_spike.py:154-155).
    """
    sa, sb = m * k, k * n
    if mode == "zeros":
        a = np.zeros(sa, np.uint8)
        b = np.zeros(sb, np.uint8)
    elif mode == "extrema":
        a = np.where(np.arange(sa) % 2 == 0, 0x80, 0x7F).astype(np.uint8)
        b = np.where(np.arange(sb) % 2 == 0, 0x7F, 0x80).astype(np.uint8)
    elif mode == "lcg":
        s = lcg8_bytes(sa + sb)
        a, b = s[:sa], s[sa:]
    else:
        raise ValueError("unknown mode %r" % (mode,))
    return a.view(np.int8).reshape(m, k), b.view(np.int8).reshape(k, n)


# ---------------------------------------------------------------------------
# The benchmark configurations
# ---------------------------------------------------------------------------

CONFIGS = {
    1: "int8 GEMM M=N=K=64, A,B ~ U{-128..127}, zero initial C",
    2: "int8 GEMM M=N=K=256, D ~ U{-2^20..2^20} int32, out = D + A.B",
    3: "batched B-reuse: 64 x A[512x1024] sharing B[1024x1024] -> C[64x512x1024]",
    4: "decode: M in {1,16}, K=4096, N=14336, A ~ U{-127..127}, "
       "B = clip(rint(N(0,32)), -128, 127)",
    5: "M=N=K=8192, half of A and B fixed at -128 or 127, the rest U{-128..127}",
}


def _uniform_i8(rng, shape, lo=-128, hi=127):
    return rng.integers(lo, hi + 1, size=shape, dtype=np.int8)


def _adversarial_i8(rng, shape):
    """Bernoulli(1/2) mask of entries fixed at -128 or 127 (fair coin), else uniform."""
    x = _uniform_i8(rng, shape)
    mask = rng.integers(0, 2, size=shape, dtype=np.uint8).astype(bool)
    ext = np.where(rng.integers(0, 2, size=shape, dtype=np.uint8).astype(bool),
                   np.int8(127), np.int8(-128))
    x[mask] = ext[mask]
    return x


def config_shape(config, m=None):
    """(batch, M, N, K, has_d, b_shared) of a configuration."""
    if config == 1:
        return 1, 64, 64, 64, False, False
    if config == 2:
        return 1, 256, 256, 256, True, False
    if config == 3:
        return 64, 512, 1024, 1024, False, True
    if config == 4:
        return 1, (16 if m is None else m), 14336, 4096, False, False
    if config == 5:
        return 1, 8192, 8192, 8192, False, False
    raise ValueError("unknown config %r" % (config,))


def config_inputs(config, seed=0, m=None):
    """Seeded inputs of a configuration: dict(A, B, D) of numpy arrays.

    A is [batch, M, K] for config 3 (B shared) and [M, K] otherwise;
    D is None unless the configuration has an initial partial sum.
    """
    rng = np.random.default_rng(seed)
    batch, M, N, K, has_d, _ = config_shape(config, m)
    if config in (1, 2):
        A = _uniform_i8(rng, (M, K))
        B = _uniform_i8(rng, (K, N))
        D = rng.integers(-(1 << 20), (1 << 20) + 1, size=(M, N), dtype=np.int32) if has_d else None
    elif config == 3:
        A = _uniform_i8(rng, (batch, M, K))
        B = _uniform_i8(rng, (K, N))
        D = None
    elif config == 4:
        A = _uniform_i8(rng, (M, K), -127, 127)
        B = np.clip(np.rint(rng.normal(0.0, 32.0, size=(K, N))), -128, 127).astype(np.int8)
        D = None
    else:
        A = _adversarial_i8(rng, (M, K))
        B = _adversarial_i8(rng, (K, N))
        D = None
    return {"A": A, "B": B, "D": D}
