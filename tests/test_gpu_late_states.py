"""HIP engine vs CPU oracle on late states of the benchmark workloads, at
their full sizes and launch shapes.

The other full-size comparisons start from resets.  Here the engine alone
runs a workload for hundreds of env steps, until the cars have spread to
the walls and corners and the contact search walks its longest candidate
lists (about 470 items per wave and tick in the headline workload, against
64 in its first steps); then the oracle takes over the engine's state and
both run three more steps, compared bit for bit over every field of the
persistent state and every output buffer (the transition observations on the
rows of the simulations that finish in the step: the others keep rows from
steps the oracle did not run):
  * the headline workload, 1v1 at 65,536 simulations with frameskip 8, after
    300 steps, in the production launch shape (64 simulations per window
    workgroup, dealt to the workgroups by the contact work of the step
    before);
  * the clustered 3v3 workload at 16,384 simulations (every car within
    500 uu of the ball, at the floor, the walls or the ceiling), compared for
    its first three steps and again after 100 steps;
  * clustered 2v2 scenes at 32,768 simulations with frameskip 8, whose
    launches are dealt, after 150 steps.
"""
import numpy as np
import pytest

from carl_amd import workloads
from gpu_harness import Pair, dev

pytestmark = pytest.mark.gpu


def _assert_clean(report, context):
    if report:
        pytest.fail(f"{context}:\n  " + "\n  ".join(report))


def _engine_steps(pair: Pair, rng: np.random.Generator, steps: int):
    for _ in range(steps):
        pair.gpu.step_continuous(dev(workloads.random_continuous_actions(rng, pair.n_sim, pair.n_cars)))
    pair.gpu.synchronize()


def _compared_steps(pair: Pair, rng: np.random.Generator, steps: int, context: str, synced: bool):
    for step in range(steps):
        pair.step_continuous(workloads.random_continuous_actions(rng, pair.n_sim, pair.n_cars))
        _assert_clean(pair.state_mismatches(), f"{context}: state after compared step {step}")
        outputs = pair.fresh_output_mismatches() if synced else pair.output_mismatches()
        _assert_clean(outputs, f"{context}: outputs after compared step {step}")


@pytest.mark.timeout(900)
def test_headline_workload_after_300_steps(gpu):
    rng = np.random.default_rng(300)
    n = 65536
    p = Pair(n, 1, 1, seed=1, frameskip=8)
    assert p.gpu.tick_window_launch == 64      # the production launch shape,
    assert p.gpu.tick_balanced_launch          # its simulations dealt to the workgroups by cost
    odd = np.arange(1, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(odd), 2), simulation_indices=odd.astype(np.int64))
    _engine_steps(p, rng, 300)
    p.sync_oracle_from_engine()
    _compared_steps(p, rng, 3, "1v1 65,536 after 300 steps", synced=True)
    p.close()


@pytest.mark.timeout(900)
def test_clustered_3v3_at_walls_and_ceiling(gpu):
    rng = np.random.default_rng(16384)
    n = 16384
    p = Pair(n, 3, 3, seed=2, frameskip=8)
    p.apply_reset_state(workloads.clustered_reset_state(rng, n, 6))
    _compared_steps(p, rng, 3, "clustered 3v3 16,384 from the reset", synced=False)
    _engine_steps(p, rng, 100)
    p.sync_oracle_from_engine()
    _compared_steps(p, rng, 3, "clustered 3v3 16,384 after 103 steps", synced=True)
    p.close()


@pytest.mark.timeout(900)
def test_clustered_2v2_dealt_after_150_steps(gpu):
    """2v2 at 32,768 simulations with frameskip 8 runs dealt launches (32
    simulations per window workgroup in units of 8); from clustered scenes
    at the arena's surfaces, 150 steps on the engine, then three compared
    steps."""
    rng = np.random.default_rng(32768)
    n = 32768
    p = Pair(n, 2, 2, seed=3, frameskip=8)
    assert p.gpu.tick_window_launch == 32 and p.gpu.tick_balanced_launch
    p.apply_reset_state(workloads.clustered_reset_state(rng, n, 4))
    _engine_steps(p, rng, 150)
    p.sync_oracle_from_engine()
    _compared_steps(p, rng, 3, "clustered 2v2 32,768 after 150 steps", synced=True)
    p.close()
