"""Seeded random sweep of the C ABI against the oracle (needs a gfx950 GPU).

Each case draws a variant (automatic, each vector variant, the any-shape
variants, packed B), a shape fitting it (M, N, K from 1 to about 1100, with
the variant's divisibility rules, often landing on tile edges; half of the
256 x 256 draws in whole tiles with K % 256 == 0, and half of the 256 x 128
draws in whole 256 x 128 tiles with K % 256 == 0), a batch count,
shared or separate B, D or not, C in place of D or not, and adversarial
inputs (int8 extremes mixed with uniform bytes). Every output element is
compared with the oracle; a case that the plan validation refuses is
redrawn. The draws are fixed by the seed, so a failure names a reproducible
case.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg

pytestmark = pytest.mark.gpu

N_CASES = 256
EDGES = (1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 256, 257, 384, 512, 640, 1024)


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def draw_dim(rng, multiple, hi):
    if rng.random() < 0.5:
        v = int(rng.choice(EDGES))
    else:
        v = int(rng.integers(1, hi + 1))
    if multiple > 1:
        v = max(multiple, (v + multiple - 1) // multiple * multiple)
    return min(v, hi // multiple * multiple if multiple > 1 else hi)


def draw_case(rng):
    while True:
        variant = str(rng.choice(["auto", "auto", "mfma_256x256", "mfma_256x128", "mfma_128x128",
                                  "skinny", "generic", "padded", hg.PACKED_VARIANT]))
        any_shape = variant in ("auto", "generic", "padded")
        m = draw_dim(rng, 1, 64 if variant in ("skinny", hg.PACKED_VARIANT) else 1100)
        n = draw_dim(rng, 1 if any_shape else 16, 1100)
        k = draw_dim(rng, 64 if variant == hg.PACKED_VARIANT else (1 if any_shape else 16), 1100)
        if variant == "mfma_256x256" and rng.random() < 0.5:
            # whole 256 x 256 tiles with K % 256 == 0: the 16x16x64 kernel
            m, n, k = (max(256, (v + 255) // 256 * 256) for v in (m, n, k))
        if variant == "mfma_256x128" and rng.random() < 0.5:
            # whole 256 x 128 tiles with K % 256 == 0: its persistent form
            m, k = (max(256, (v + 255) // 256 * 256) for v in (m, k))
            n = max(128, (n + 127) // 128 * 128)
        batch = int(rng.choice([1, 1, 2, 3]))
        shared = bool(rng.random() < 0.5) and batch > 1
        has_d = bool(rng.random() < 0.5)
        in_place = has_d and bool(rng.random() < 0.5)
        d_max = int(rng.choice([1000, 1 << 20, (1 << 31) - 1 - 16384 * k])) if has_d else 0
        try:
            plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=has_d,
                                d_max_abs=d_max, variant=variant)
        except Exception:
            continue
        if hg.validate_plan(plan)[0]:
            return plan, in_place


def adversarial(rng, shape):
    x = rng.integers(-128, 128, shape, dtype=np.int8)
    pick = rng.random(shape)
    x[pick < 0.2] = -128
    x[(pick >= 0.2) & (pick < 0.3)] = 127
    return x


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_case(dev, case):
    rng = np.random.default_rng(20261202 + case)
    plan, in_place = draw_case(rng)
    m, n, k, batch = plan["m"], plan["n"], plan["k"], plan["batch"]
    print("case", case, plan["variant"], m, n, k, "batch", batch, "shared", plan["b_shared"],
          "D", plan["has_d"], "in place", in_place, flush=True)
    A = adversarial(rng, (batch, m, k) if batch > 1 else (m, k))
    B = adversarial(rng, (k, n) if (batch == 1 or plan["b_shared"]) else (batch, k, n))
    D = None
    if plan["has_d"]:
        lim = plan["d_max_abs"]
        D = rng.integers(-lim, lim + 1, (batch, m, n) if batch > 1 else (m, n), dtype=np.int64)
        D = D.astype(np.int32)
    At = torch.from_numpy(A).to(dev)
    Bt = torch.from_numpy(B).to(dev)
    Bop = hg.pack_b(Bt) if plan["variant"] == hg.PACKED_VARIANT else Bt
    if D is None:
        C = hg.run(plan, At, Bop).cpu().numpy()
    else:
        Dt = torch.from_numpy(D).to(dev)
        C = hg.run(plan, At, Bop, Dt, out=Dt if in_place else None).cpu().numpy()
    if batch == 1:
        want = go.gemm_i8(A, B, D)
    else:
        want = np.stack([go.gemm_i8(A[b], B if plan["b_shared"] else B[b],
                                    None if D is None else D[b]) for b in range(batch)])
    assert C.shape == want.shape
    bad = np.argwhere(C != want)
    assert bad.size == 0, "first mismatch at %s: got %d want %d" % (
        tuple(bad[0]), C[tuple(bad[0])], want[tuple(bad[0])])
