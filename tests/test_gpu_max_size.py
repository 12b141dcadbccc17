"""The largest environments the engine accepts, at the top of their index
range.

The engine addresses its state through 32-bit buffer offsets and refuses
larger sizes at creation (tests/test_abi.py checks the refusal).  Here
environments at that limit run, and the simulations at the very end of the
index range, whose offsets come closest to 2^31 bytes, are compared with a
small environment started from the same states, while the CPU oracle checks
the small environment: every output row of those simulations must be
bit-identical.

Simulations share nothing, so a simulation's results do not depend on its
index, except through two index-seeded draws: the kickoff chosen when an
episode ends, and the respawn spot of a demolished car (used only when it
respawns, seconds later).  A simulation whose episode ends in a step is
compared up to that step's transition outputs and left out afterwards.

Cases: 1v1 at the limit (its last window workgroup half full, so the launch
is not dealt), 1v1 and 2v2 at the largest sizes whose workgroups are all
full (dealt launches), and 4v4 at the limit (the any-count kernel instance).
All start from clustered scenes at the arena's surfaces, so the tested rows
run car-car, car-ball and wall contacts.
"""
import numpy as np
import pytest
import torch

import carl_amd
from abi import enum_values
from carl_amd import workloads
from gpu_harness import Pair, dev

pytestmark = pytest.mark.gpu

K = 64          # simulations compared at the top of the index range
STEPS = 6
FRAMESKIP = 8


def _max_cars() -> int:
    """The documented car limit: the car block, 4 * CARL_CAR_FIELDS bytes per
    car in whole tiles of 64 cars, stays below 2^31 bytes."""
    return ((2 ** 31 - 1) // (4 * enum_values("CARL_")["CARL_CAR_FIELDS"])) & ~63


def _cases():
    m = _max_cars()
    return [
        pytest.param(m // 2, 1, False, id="1v1-limit"),
        pytest.param(m // 2 // 64 * 64, 1, True, id="1v1-full-workgroups"),
        pytest.param(m // 4 // 32 * 32, 2, True, id="2v2-full-workgroups"),
        pytest.param(m // 8, 4, False, id="4v4-limit"),
    ]


def _rows(env, name, lo, hi):
    """Rows lo..hi-1 of an output buffer, as (rows, bytes) uint8 arrays."""
    t = torch.from_dlpack(getattr(env, "get_" + name)())
    t = t.reshape(env.n_sim, -1)[lo:hi]
    return t.cpu().numpy().copy().view(np.uint8).reshape(hi - lo, -1)


PER_STEP = ("obs", "state", "score_difference", "episode_ticks", "overtime")
TRANSITION = ("rewards", "dones", "transition_state", "transition_score_difference",
              "transition_episode_ticks", "transition_overtime")


@pytest.mark.parametrize("n_sim,team,dealt", _cases())
def test_top_of_the_index_range_matches_a_small_environment(gpu, n_sim, team, dealt):
    nc = 2 * team
    assert n_sim * nc <= _max_cars()
    print(f"\n{team}v{team} at {n_sim} simulations ({n_sim * nc} cars)", flush=True)
    rng = np.random.default_rng(1000 + n_sim % 997)
    big = carl_amd.Env(n_sim, team, team, 7, FRAMESKIP, True, False, False)
    small = Pair(K, team, team, seed=7, frameskip=FRAMESKIP)
    try:
        assert big.tick_balanced_launch == dealt
        top = np.arange(n_sim - K, n_sim, dtype=np.int64)
        scene = workloads.clustered_reset_state(rng, K, nc)
        small.apply_reset_state(scene)
        big.apply_reset_state(**{k: dev(v) for k, v in scene.items()}, simulation_indices=dev(top))
        actions = torch.zeros((n_sim, nc, 7), dtype=torch.float32, device=gpu)
        live = np.ones(K, dtype=bool)
        for step in range(STEPS):
            a = workloads.random_continuous_actions(rng, K, nc)
            small.step_continuous(a)
            actions[n_sim - K:] = dev(a)
            big.step_continuous(actions)
            big.synchronize()
            report = small.output_mismatches(TRANSITION + PER_STEP)
            assert not report, f"small environment vs oracle, step {step}:\n  " + "\n  ".join(report)
            # a simulation that finished in this step has had its kickoff drawn
            # from its index: its transition outputs are compared, its new
            # episode's rows are not
            done = _rows(small.gpu, "dones", 0, K)[:, 0] != 0
            for names, rows in ((TRANSITION, live), (PER_STEP, live & ~done)):
                for name in names:
                    b = _rows(big, name, n_sim - K, n_sim)
                    s = _rows(small.gpu, name, 0, K)
                    bad = np.nonzero(rows & (b != s).any(axis=1))[0]
                    assert len(bad) == 0, (f"{name} differs at step {step} on simulation {n_sim - K + bad[0]} "
                                           f"({len(bad)} of {int(rows.sum())} compared rows)")
            live &= ~done
        assert live.sum() >= K // 2, "too few simulations stayed in their episode to compare"
    finally:
        small.close()
        del big
