"""emit_c programs run on the GPU (needs a gfx950 GPU).

Each emitted program generates its inputs, poisons C with INT32_MIN, runs
the plan's GEMM through libvt_hip_gemm.so and compares every output with its
own scalar loop, whose inputs and expected outputs the CPU tests pin to the
oracle (tests/test_emit_program.py). It must print VERITAC_HIP_GEMM_PASS and
exit 0, as the reference's emitted program must print VERITAC_GEMMINI_PASS
(specializations/gemmini_gemm/backend.py:772-790).
"""
import subprocess

import pytest

torch = pytest.importorskip("torch")

from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import program as pg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"


CASES = [
    ("config1_auto", lambda: hg.make_plan(64, 64, 64), {}),
    ("config2_d_auto", lambda: hg.make_plan(256, 256, 256, has_d=True, d_max_abs=1 << 20), {}),
    ("mfma_256x256", lambda: hg.make_plan(512, 256, 192, variant="mfma_256x256"), {}),
    ("mfma_256x128_d", lambda: hg.make_plan(300, 208, 160, has_d=True, d_max_abs=99,
                                           variant="mfma_256x128"), {}),
    ("mfma_128x128_batched_shared", lambda: hg.make_plan(48, 80, 96, batch=3, b_shared=True,
                                                         variant="mfma_128x128"), {}),
    ("mfma_128x128_batched", lambda: hg.make_plan(40, 48, 64, batch=2, has_d=True, d_max_abs=7,
                                                  variant="mfma_128x128"), {}),
    ("skinny_split3", lambda: hg.make_plan(16, 512, 1024, variant="skinny", k_split=3), {}),
    ("skinny_m1_d", lambda: hg.make_plan(1, 1024, 4096, has_d=True, d_max_abs=1 << 10,
                                         variant="skinny"), {}),
    ("generic_odd", lambda: hg.make_plan(33, 70, 45, variant="generic"), {}),
    ("padded_odd_d", lambda: hg.make_plan(100, 129, 77, has_d=True, d_max_abs=5,
                                          variant="padded"), {}),
    ("packed_d_batched", lambda: hg.make_plan(16, 256, 320, variant=hg.PACKED_VARIANT,
                                              has_d=True, d_max_abs=1000, batch=2), {}),
    ("packed_256_rows", lambda: hg.make_plan(272, 512, 256, variant=hg.PACKED_VARIANT), {}),
    ("extremes_max", lambda: hg.make_plan(64, 64, 8192, variant="mfma_128x128"),
     dict(input_mode="max")),
    ("extremes_minmax", lambda: hg.make_plan(256, 256, 8192, variant="mfma_256x256"),
     dict(input_mode="minmax")),
    ("extremes_min_skinny", lambda: hg.make_plan(16, 256, 8192, variant="skinny"),
     dict(input_mode="min")),
    ("zero_d", lambda: hg.make_plan(64, 64, 64, has_d=True, d_max_abs=1 << 20, variant="generic"),
     dict(input_mode="zero")),
]


@pytest.mark.parametrize("name,make,kw", CASES, ids=[c[0] for c in CASES])
def test_emitted_program_passes_on_the_gpu(gpu, tmp_path, name, make, kw):
    plan = make()
    info = hg.emit_c(plan, str(tmp_path / (name + ".c")), **kw)
    exe = pg.build_program(info["path"])
    print("emitted program", name, plan["variant"], info["sha256"][:16], flush=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(out.stdout, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = out.stdout.strip().splitlines()
    assert lines[-1] == pg.PASS_MARKER
    n = plan["batch"] * plan["m"] * plan["n"]
    assert "all %d scalar output comparisons matched" % n in out.stdout
