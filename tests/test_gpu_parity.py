"""HIP engine vs CPU oracle: bit-exact parity on identical inputs.

Both sides follow the same evaluation-order contract (own sin/cos/atan2, no
FMA contraction, comparison min/max), so every output buffer and every field
of the persistent state must agree bit for bit after any sequence of calls.
The workloads restate the benchmark configurations at oracle-sized scale:
kickoffs, random states (1v1), clustered 3v3, 2v2 with per-step resets, and a
per-tick resynchronised run that isolates single-tick error.
"""
import ctypes

import numpy as np
import pytest
import torch

from carl_amd import workloads
from gpu_harness import Pair, dense_geometry_reset_state, dev, gpu_state, pad_reset_state

pytestmark = pytest.mark.gpu

CONTINUOUS = 1


def _assert_clean(report, context):
    if report:
        pytest.fail(f"{context}:\n  " + "\n  ".join(report))


def _lib():
    from carl_amd import build

    return ctypes.CDLL(str(build.engine_path()))


def test_scan_known_answer_and_random(gpu):
    """Wave64 DPP exclusive scan: {3,1,4,2} -> {0,3,4,8} (tests/direct_controls.cu:15-33)."""
    lib = _lib()
    lib.carl_exclusive_scan_i32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    rng = np.random.default_rng(3)
    cases = [np.array([3, 1, 4, 2], np.int32)] + [rng.integers(0, 50, n).astype(np.int32)
                                                  for n in (1, 63, 64, 65, 2047, 2048, 2049, 100_000, 3_000_000)]
    for x in cases:
        src = dev(x)
        out = torch.full_like(src, -1)
        assert lib.carl_exclusive_scan_i32(src.data_ptr(), out.data_ptr(), len(x), None) == 0
        torch.cuda.synchronize()
        expect = np.concatenate([[0], np.cumsum(x)[:-1]]).astype(np.int32)
        np.testing.assert_array_equal(out.cpu().numpy(), expect, err_msg=f"n={len(x)}")


@pytest.mark.parametrize("teams", [(1, 1), (2, 2), (3, 3), (1, 0), (2, 1)])
def test_reset_state_and_outputs_match(gpu, teams):
    p = Pair(33, *teams, seed=11, previous_controls=True)
    _assert_clean(p.state_mismatches(), f"state after reset {teams}")
    _assert_clean(p.output_mismatches(), f"outputs after reset {teams}")
    p.close()


def test_kickoff_trajectory_1v1(gpu):
    rng = np.random.default_rng(1)
    p = Pair(64, 1, 1, seed=5, frameskip=8)
    for step in range(40):
        p.step_continuous(workloads.random_continuous_actions(rng, 64, 2))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


def test_queued_steps_with_temporary_actions(gpu):
    """Steps queued without synchronising, each from a temporary actions tensor
    the caller drops at once: the engine must read every step's own actions."""
    rng = np.random.default_rng(12)
    n = 96
    p = Pair(n, 1, 1, seed=4, frameskip=8)
    for _ in range(12):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 2))
    _assert_clean(p.state_mismatches(), "state after 12 queued steps")
    _assert_clean(p.output_mismatches(), "outputs after 12 queued steps")
    p.close()


def test_random_state_trajectory_1v1(gpu):
    rng = np.random.default_rng(2)
    n = 256
    p = Pair(n, 1, 1, seed=9, frameskip=8, normalize=True)
    odd = np.arange(1, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(odd), 2), simulation_indices=odd.astype(np.int64))
    _assert_clean(p.state_mismatches(), "state after random reset")
    for step in range(24):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 2))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


def test_clustered_3v3_contacts(gpu):
    """Cars within 500 uu of the ball: dense car-car SAT, bumps, demos and ball hits."""
    rng = np.random.default_rng(4)
    n = 48
    p = Pair(n, 3, 3, seed=3, frameskip=8)
    p.apply_reset_state(workloads.random_reset_state(rng, n, 6, cluster_radius=500.0))
    _assert_clean(p.state_mismatches(), "state after clustered reset")
    for step in range(16):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 6))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


@pytest.mark.parametrize("n_blue,frameskip", [(1, 8), (2, 1), (3, 4), (4, 2)])
def test_short_episodes_timeouts_overtime_and_resets(gpu, n_blue, frameskip):
    """Episodes of a few steps: regulation timeouts, ties that enter overtime,
    overtime expiry and no-touch timeouts end simulations on most steps, so
    the packing's reset decisions, the match state after the resets and the
    transition rows of finished simulations all run against the oracle.  In
    3v3 and 4v4 the state rows take more than one LDS chunk and only a few
    finished rows fit beside the first, so the packing's further rounds for
    both run too (96 simulations: one full packing workgroup and one partial)."""
    rng = np.random.default_rng(18 + n_blue)
    n, nc = 96, 2 * n_blue
    p = Pair(n, n_blue, n_blue, seed=12, frameskip=frameskip)
    p.set_param("max_ticks", 3 * frameskip + 1)
    p.set_param("overtime_timeout_ticks", 2 * frameskip)
    p.set_param("no_touch_timeout_ticks", 7 * frameskip)
    half = np.arange(0, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(half), nc), simulation_indices=half.astype(np.int64))
    for step in range(18):
        p.step_continuous(workloads.random_continuous_actions(rng, n, nc))
        _assert_clean(p.state_mismatches(), f"{n_blue}v{n_blue} state after step {step}")
        _assert_clean(p.output_mismatches(), f"{n_blue}v{n_blue} outputs after step {step}")
    p.close()


@pytest.mark.parametrize("n_blue,n_orange", [(1, 1), (2, 2), (4, 4)])
def test_boost_pad_pickups(gpu, n_blue, n_orange):
    """Cars parked on boost pads, some sharing one (the last car in order
    takes it), with empty to full boost: pickups and cooldowns against the
    oracle, up to the largest team size."""
    rng = np.random.default_rng(16 + n_blue)
    n, nc = 64, n_blue + n_orange
    p = Pair(n, n_blue, n_orange, seed=6, frameskip=2)
    p.apply_reset_state(pad_reset_state(rng, n, nc))
    _assert_clean(p.state_mismatches(), f"{n_blue}v{n_orange} state after pad reset")
    for step in range(10):
        p.step_continuous(workloads.random_continuous_actions(rng, n, nc))
        _assert_clean(p.state_mismatches(), f"{n_blue}v{n_orange} state after step {step}")
        _assert_clean(p.output_mismatches(), f"{n_blue}v{n_orange} outputs after step {step}")
    p.close()


@pytest.mark.parametrize("n_blue,n_orange,window,frameskip", [
    (1, 0, 128, 2),   # one car per simulation: one range of all 34 pads
    (1, 1, 64, 2),    # two ranges of 17 (launches too short to be dealt)
    (1, 1, 32, 2),    # four ranges of 8 or 9
    (2, 2, 32, 8),    # dealt 2v2 launches: four ranges of 8 or 9
    (3, 3, 21, 2),    # six ranges of 5 or 6
])
def test_boost_pad_ranges_by_workgroup_size(gpu, n_blue, n_orange, window, frameskip):
    """The window kernel splits each simulation's pads into as many ranges as
    its workgroup has threads per simulation; cars parked on pads, for every
    split the workgroup sizes give: pickups and cooldowns against the
    oracle."""
    rng = np.random.default_rng(window + 7 * n_blue + n_orange)
    n, nc = 128, n_blue + n_orange
    p = Pair(n, n_blue, n_orange, seed=6, frameskip=frameskip)
    p.gpu.tick_window = window
    assert p.gpu.tick_window_launch == window
    p.apply_reset_state(pad_reset_state(rng, n, nc))
    for step in range(8):
        p.step_continuous(workloads.random_continuous_actions(rng, n, nc))
        _assert_clean(p.state_mismatches(), f"{n_blue}v{n_orange} window {window}: state after step {step}")
        _assert_clean(p.output_mismatches(), f"{n_blue}v{n_orange} window {window}: outputs after step {step}")
    p.close()


def test_dense_geometry_1v1_and_3v3(gpu):
    """Cars and balls in corners, goal mouths, on posts, walls and the ceiling:
    long cell runs, many SAT hits and large ball contact lists."""
    rng = np.random.default_rng(14)
    for n_blue, n, steps in ((1, 128, 20), (3, 32, 12)):
        nc = 2 * n_blue
        p = Pair(n, n_blue, n_blue, seed=8, frameskip=4)
        p.apply_reset_state(dense_geometry_reset_state(rng, n, nc))
        _assert_clean(p.state_mismatches(), f"{n_blue}v{n_blue} state after dense reset")
        for step in range(steps):
            p.step_continuous(workloads.random_continuous_actions(rng, n, nc))
            _assert_clean(p.state_mismatches(), f"{n_blue}v{n_blue} state after step {step}")
            _assert_clean(p.output_mismatches(), f"{n_blue}v{n_blue} outputs after step {step}")
        p.close()


def test_balls_at_and_beyond_the_candidate_grid_edge(gpu):
    """Balls inside the arena's broadphase box but outside the walls, and
    beyond the box (where the sequential gather serves them), next to balls
    on the floor, the walls and in the goals."""
    rng = np.random.default_rng(15)
    n = 64
    p = Pair(n, 1, 1, seed=9, frameskip=2)
    state = workloads.random_reset_state(rng, n, 2)
    spots = np.array([[0.0, 0.0, 93.2], [4004.0, 100.0, 500.0], [4150.0, 0.0, 300.0], [4300.0, -200.0, 300.0],
                      [0.0, 5300.0, 100.0], [0.0, 6100.0, 200.0], [100.0, 0.0, 2100.0], [-50.0, 30.0, 2250.0],
                      [-4212.5, 0.0, 400.0], [0.0, -6031.0, 150.0]])
    state["ball_position"] = np.ascontiguousarray(
        spots[np.arange(n) % len(spots)] + rng.uniform(-2.0, 2.0, (n, 3)), dtype=np.float32)
    p.apply_reset_state(state)
    for step in range(20):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 2))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


def test_2v2_masked_resets_every_step(gpu):
    """tick_skip 1 with 25% of arenas reset from random states each step (masked path)."""
    rng = np.random.default_rng(6)
    n = 64
    p = Pair(n, 2, 2, seed=13, frameskip=1)
    for step in range(40):
        p.step_discrete(workloads.random_discrete_actions(rng, n, 4))
        mask = rng.uniform(0, 1, n) < 0.25
        p.apply_reset_state(workloads.random_reset_state(rng, n, 4), reset_mask=mask)
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


def test_per_tick_from_identical_state(gpu):
    """Resynchronise the oracle from the engine before every tick; one tick must agree."""
    rng = np.random.default_rng(8)
    n = 128
    p = Pair(n, 2, 2, seed=21, frameskip=1)
    p.apply_reset_state(workloads.random_reset_state(rng, n, 4, cluster_radius=900.0))
    for tick in range(60):
        a = workloads.random_continuous_actions(rng, n, 4)
        p.sync_oracle_from_engine()
        p.gpu.tick(dev(a), CONTINUOUS, 1)
        p.cpu.tick(a, CONTINUOUS, 1)
        _assert_clean(p.state_mismatches(), f"state after tick {tick}")
    p.close()


def test_thousand_ticks_stay_bit_exact_1v1(gpu):
    """1,000 ticks (125 steps of 8) without resynchronisation: every state
    field and every output stays bit-equal to the oracle after every step.
    The trajectories are chaotic - a one-ulp change to one car's starting
    velocity ends tens of uu away after these 1,000 ticks
    (test_oracle_invariants.py::test_one_ulp_grows_past_the_long_run_tolerance)
    - so a tolerance of 1e-3 uu over 1,000 ticks could only be met bit for
    bit, and a single differing rounding in the engine would show here."""
    rng = np.random.default_rng(10)
    n = 32
    p = Pair(n, 1, 1, seed=17, frameskip=8)
    p.apply_reset_state(workloads.random_reset_state(rng, n, 2))
    for step in range(125):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 2))
        report = p.state_mismatches() + p.output_mismatches()
        assert not report, f"after step {step}:\n  " + "\n  ".join(report)
    p.close()
