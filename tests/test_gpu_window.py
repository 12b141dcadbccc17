"""The tick-window kernel changes no result.

With CARL_PARAM_TICK_WINDOW > 0 a step's ticks run in one launch per
partition, a workgroup taking every phase of every tick for its own
simulations; with 0 they run as four phase kernels per tick.  These tests run
both on identical inputs and require every field of the persistent state and
every packed output to agree bit for bit, over team sizes, workgroup sizes,
partition counts and frameskips, at sizes the oracle cannot reach.
"""
import numpy as np
import pytest
import torch

import carl_amd
from carl_amd import workloads
from gpu_harness import dense_geometry_reset_state, describe_mismatch, dev, gpu_state, pad_reset_state
from abi import CAR_NAMES, SIM_NAMES

pytestmark = pytest.mark.gpu


def _run_both(n, n_blue, n_orange, frameskip, steps, make_state, seed, window=64, streams=4, reset_every=0,
              balanced=False):
    rng = np.random.default_rng(seed)
    nc = n_blue + n_orange
    fused = carl_amd.Env(n, n_blue, n_orange, 5, frameskip, True, False, True)
    phased = carl_amd.Env(n, n_blue, n_orange, 5, frameskip, True, False, True)
    fused.tick_window = window
    fused.tick_streams = streams
    fused.tick_balance = int(balanced)
    phased.tick_window = 0
    phased.tick_streams = streams
    assert (fused.tick_window, phased.tick_window) == (window, 0)
    assert fused.tick_balanced_launch == balanced
    state = {k: dev(v) for k, v in make_state(rng, n, nc).items()}
    for env in (fused, phased):
        env.apply_reset_state(**state)
    for step in range(steps):
        if reset_every and step % reset_every == 0:
            mask = dev(rng.uniform(size=n) < 0.25)
            fresh = {k: dev(v) for k, v in make_state(rng, n, nc).items()}
            for env in (fused, phased):
                env.apply_reset_state(**fresh, reset_mask=mask)
        actions = dev(workloads.random_continuous_actions(rng, n, nc))
        fused.step_continuous(actions)
        phased.step_continuous(actions)
        a, b = gpu_state(fused), gpu_state(phased)
        report = describe_mismatch(CAR_NAMES, a[0], b[0]) + describe_mismatch(SIM_NAMES, a[1], b[1])
        for name in ("get_obs", "get_state", "get_rewards", "get_dones"):
            x = torch.from_dlpack(getattr(fused, name)()).cpu().numpy()
            y = torch.from_dlpack(getattr(phased, name)()).cpu().numpy()
            if x.tobytes() != y.tobytes():
                report.append(f"{name} differs")
        if report:
            pytest.fail(f"window {window} vs phase kernels after step {step}:\n  " + "\n  ".join(report))


def test_window_random_states_1v1(gpu):
    _run_both(8192, 1, 1, 8, 30, workloads.random_reset_state, seed=41)


@pytest.mark.parametrize("window,streams", [(16, 4), (128, 1), (37, 3)])
def test_window_block_sizes_and_partitions(gpu, window, streams):
    _run_both(3001, 1, 1, 8, 12, workloads.random_reset_state, seed=42, window=window, streams=streams)


def test_window_dense_geometry_3v3_and_2v2(gpu):
    _run_both(1024, 3, 3, 4, 20, dense_geometry_reset_state, seed=43)
    _run_both(2048, 2, 2, 4, 20, dense_geometry_reset_state, seed=44, window=32)


def test_window_per_tick_steps_with_masked_resets(gpu):
    _run_both(4096, 2, 2, 1, 40, workloads.random_reset_state, seed=45, reset_every=1)


@pytest.mark.parametrize("make_state,reset_every", [(workloads.random_reset_state, 0),
                                                     (workloads.clustered_reset_state, 3)])
def test_balanced_deal_1v1(gpu, make_state, reset_every):
    """Balanced 1v1 launches take their simulations in units of sixteen, dealt
    by the contact work of the launch before: the deal moves simulations
    between workgroups from step to step, never a result.  Clustered states
    put most cars against the walls, so the deal reorders heavily."""
    _run_both(8192, 1, 1, 8, 30, make_state, seed=48, streams=1, reset_every=reset_every, balanced=True)


def test_balanced_deal_2v2(gpu):
    """The same for 2v2: units of eight simulations, workgroups of 32, four and
    eight ticks per step."""
    _run_both(4096, 2, 2, 8, 20, workloads.clustered_reset_state, seed=49, streams=1, reset_every=4, balanced=True)
    _run_both(4096, 2, 2, 4, 30, workloads.random_reset_state, seed=50, streams=1, reset_every=1, balanced=True)


def test_balanced_deal_bare_ticks(gpu):
    """Bare tick launches (no packing) are dealt as steps are: a dealt and an
    undealt environment ticked 8 at a time stay bit-equal, and a launch of 2
    ticks in between (not dealt) leaves the deal's lists intact for the next
    dealt launch."""
    n = 8192
    rng = np.random.default_rng(51)
    envs = [carl_amd.Env(n, 1, 1, 5, 8, True, False, False) for _ in range(2)]
    state = {k: dev(v) for k, v in workloads.clustered_reset_state(rng, n, 2).items()}
    for env, balance in zip(envs, (1, 0)):
        env.tick_window, env.tick_streams, env.tick_balance = 64, 1, balance
        env.apply_reset_state(**state)
    assert envs[0].tick_balanced_launch and not envs[1].tick_balanced_launch
    for k in range(12):
        ticks = 2 if k == 5 else 8
        actions = dev(workloads.random_continuous_actions(rng, n, 2))
        for env in envs:
            env.tick(actions.reshape(-1), 1, ticks)
        a, b = gpu_state(envs[0]), gpu_state(envs[1])
        report = describe_mismatch(CAR_NAMES, a[0], b[0]) + describe_mismatch(SIM_NAMES, a[1], b[1])
        if report:
            pytest.fail(f"dealt vs undealt after bare launch {k}:\n  " + "\n  ".join(report))


def test_balanced_launch_conditions(gpu):
    """The deal runs only for 1v1 and 2v2 in one partition with full
    workgroups (64 and 32 simulations)."""
    env = carl_amd.Env(4096, 1, 1, 1, 8, True, False, False)
    env.tick_window, env.tick_streams = 64, 1
    assert env.tick_balance == 1 and env.tick_balanced_launch
    for attr, value in (("tick_streams", 2), ("tick_window", 32), ("tick_balance", 0)):
        setattr(env, attr, value)
        assert not env.tick_balanced_launch, attr
        env.tick_window, env.tick_streams, env.tick_balance = 64, 1, 1
        assert env.tick_balanced_launch
    # a partial workgroup, a partial 2v2 workgroup, 3v3, one car
    for n, blue, orange in ((4032 + 8, 1, 1), (2048 + 16, 2, 2), (2048, 3, 3), (2048, 1, 0)):
        other = carl_amd.Env(n, blue, orange, 1, 8, True, False, False)
        other.tick_window, other.tick_streams = 64, 1
        assert not other.tick_balanced_launch, (n, blue, orange)
    two = carl_amd.Env(2048, 2, 2, 1, 8, True, False, False)
    two.tick_window, two.tick_streams = 64, 1            # capped at 128 cars: workgroups of 32
    assert two.tick_window_launch == 32 and two.tick_balanced_launch
    for frameskip in (1, 3):                             # too few ticks per launch
        few = carl_amd.Env(2048, 1, 1, 1, frameskip, True, False, False)
        few.tick_window, few.tick_streams = 64, 1
        assert not few.tick_balanced_launch, frameskip
    with pytest.raises(ValueError):
        env.tick_balance = 2


def test_window_single_car(gpu):
    _run_both(1000, 1, 0, 8, 15, workloads.random_reset_state, seed=46)


@pytest.mark.parametrize("n_blue,n_orange,window", [(1, 1, 64), (2, 2, 37), (4, 3, 18), (4, 4, 64)])
def test_window_boost_pad_split_and_large_teams(gpu, n_blue, n_orange, window):
    """Cars parked on pads (some sharing one): the window kernel splits each
    simulation's pads over several threads, the phase kernels take them in one
    thread; both must give the same boosts and cooldowns."""
    _run_both(900, n_blue, n_orange, 2, 12, pad_reset_state, seed=47 + n_blue + n_orange, window=window)


def test_tick_timing_counts_every_launch(gpu):
    """The HIP-event timing records one positive duration per tick-kernel launch of partition 0 and per packing launch."""
    n, frameskip, steps = 2048, 4, 3
    env = carl_amd.Env(n, 1, 1, 3, frameskip, True, False, False)
    actions = dev(workloads.random_continuous_actions(np.random.default_rng(5), n, 2))
    phase = {name: steps * frameskip for name in ("contactKernel", "carArenaKernel", "ballKernel", "finishKernel")}
    phase["stepEnvKernel"] = steps
    window = {"tickWindowKernel": steps, "stepEnvKernel": steps}
    for window_sims, streams, expect in ((64, 1, window), (64, 3, window), (0, 1, phase)):
        env.tick_window = window_sims
        env.tick_streams = streams
        env.enable_tick_timing(True, packing=True)
        for _ in range(steps):
            env.step_continuous(actions)
        timing = env.tick_timing()
        env.enable_tick_timing(False)
        assert {k: v[1] for k, v in timing.items()} == expect, (window_sims, streams, timing)
        assert all(v[0] > 0.0 for v in timing.values()), timing
    # each selection alone
    env.tick_window = 64
    env.tick_streams = 1
    for ticks, packing, expect in ((True, False, {"tickWindowKernel": steps}), (False, True, {"stepEnvKernel": steps})):
        env.enable_tick_timing(True, ticks=ticks, packing=packing)
        for _ in range(steps):
            env.step_continuous(actions)
        timing = env.tick_timing()
        env.enable_tick_timing(False)
        assert {k: v[1] for k, v in timing.items()} == expect, (ticks, packing, timing)
