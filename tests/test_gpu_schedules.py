"""Generated Gemmini schedules replayed on the GPU (vt_replay_i8 through
replay.run_commands) against the oracle interpreter and the scalar GEMM:
the reference's unseen shapes under both schedules
(tests/test_gemmini_general.py:13-19), its partial-last-batch case
(:47-57: 48x16x32, batch_rows 2, mvin_B == 4, five input modes, seed 917),
reordered tiles, and larger shapes and batch sizes (needs a gfx950 GPU)."""
import copy

import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from oracle import gemmini_replay as gr
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import replay as rp
from veritac_amd.specializations.hip_gemm import schedules as sc

pytestmark = pytest.mark.gpu

MODES = ("zero", "max", "min", "minmax", "lcg")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def replay_matches(dev, plan, cmds, seed, modes=MODES):
    m, n, k = plan["m"], plan["n"], plan["k"]
    print("replay", m, n, k, plan["schedule"], len(cmds), "commands", flush=True)
    for mode in modes:
        A, B = go.deterministic_inputs(m, n, k, seed, mode)
        C, stats = rp.run_commands(cmds, plan, A, B, device=dev)
        want, want_stats = gr.run_commands(cmds, plan, A, B)
        assert C == want == go.scalar_matmul(A, B, m, n, k), (m, n, k, mode)
        assert stats == want_stats


@pytest.mark.parametrize("shape", [(32, 16, 32), (16, 32, 48), (48, 32, 64), (64, 64, 64)])
@pytest.mark.parametrize("schedule", ["baseline", "reuse_b"])
def test_unseen_shapes_both_schedules(dev, shape, schedule):
    plan = sc.make_plan(*shape, schedule)
    cmds = sc.gen_commands(plan)
    assert sc.check_program(plan, cmds)[:2] == (True, "accepted")
    replay_matches(dev, plan, cmds, seed=7)


def test_batched_reuse_partial_last_batch(dev):
    plan = sc.make_plan(48, 16, 32, "baseline")
    plan["accumulator_rows"] = 32
    cmds = sc.gen_batched_reuse_b(plan, 2)
    assert sc.modeled_counts(cmds)["mvin_B"] == 4
    replay_matches(dev, plan, cmds, seed=917)


@pytest.mark.parametrize("shape,batch", [((128, 48, 64), 3), ((80, 32, 96), 2), ((96, 64, 32), 4)])
def test_batched_reuse_larger_shapes(dev, shape, batch):
    plan = sc.make_plan(*shape, "reuse_b")
    cmds = sc.gen_batched_reuse_b(plan, batch)
    assert sc.check_program(plan, cmds)[:2] == (True, "accepted")
    replay_matches(dev, plan, cmds, seed=11, modes=("minmax", "lcg"))


def test_reordered_output_tiles(dev):
    plan = sc.make_plan(32, 16, 32, "baseline")
    cmds = sc.gen_commands(plan)
    rev = cmds[:4] + cmds[13:22] + cmds[4:13] + cmds[-1:]
    assert sc.check_program(plan, rev)[:2] == (True, "accepted")
    replay_matches(dev, plan, rev, seed=917)


def test_refused_overwrite_runs_like_the_interpreter_and_is_not_the_gemm(dev):
    """The replay executes what the interpreter executes; only the program
    check refuses a stream whose k > 0 step overwrites its partial sum."""
    plan = sc.make_plan(32, 16, 32, "baseline")
    cmds = copy.deepcopy(sc.gen_commands(plan))
    next(c for c in cmds if c["kind"] == "preload" and c["out_addr"] & sc.ACCUMULATE_BIT)[
        "out_addr"] &= ~sc.ACCUMULATE_BIT
    assert not sc.check_program(plan, cmds)[0]
    A, B = go.deterministic_inputs(32, 16, 32, 917, "max")
    C, _ = rp.run_commands(cmds, plan, A, B, device=dev)
    assert C == gr.run_commands(cmds, plan, A, B)[0]
    assert C != go.scalar_matmul(A, B, 32, 16, 32)
