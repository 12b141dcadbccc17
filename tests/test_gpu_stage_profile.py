"""The stage profile (CARL_TIME_STAGES) of the tick.

The window kernel's profiled twin reads the wall clock at every phase
barrier.  Its clock must agree with the HIP events around the same launches:
the span from the first workgroup start to the last workgroup end is 95% to
101% of the launch time (the launch also holds the dispatch before the first
clock read and the end after the last).  The critical path, the phases of
the workgroup that finished each launch last plus its start delay, sums to
the span within 1% (the clock reads between its phases).  The per-stage
device shares sum to no more than the span.  The figures hold whether the
grid fits the device at once, fills it exactly, or runs in several rounds.
The profiled kernel computes the same state as the plain one, and the
phase-kernel path reports each phase kernel's event time.
"""
import numpy as np
import pytest

import carl_amd
from carl_amd import workloads
from carl_amd.profiler import stage_profile
from gpu_harness import dev, gpu_state

pytestmark = pytest.mark.gpu

STAGES = ["contact", "car-arena", "ball", "finish", "boost-pads"]
# The clock span runs from the first workgroup's first clock read to the last
# workgroup's last one; the launch time adds the dispatch before the first
# wave and the drain after the last (a few us, 95% of an 80 us tick was seen
# to dip to 94.9%).
SPAN_LOW, SPAN_HIGH = 0.90, 1.01


def _env(n, n_blue, n_orange, frameskip, seed, window=64, streams=1):
    env = carl_amd.Env(n, n_blue, n_orange, 5, frameskip, True, False, True)
    env.tick_window = window
    env.tick_streams = streams
    rng = np.random.default_rng(seed)
    env.apply_reset_state(**{k: dev(v) for k, v in workloads.random_reset_state(rng, n, n_blue + n_orange).items()})
    return env, rng


def _steps(env, rng, n, nc, steps):
    for _ in range(steps):
        env.step_continuous(dev(workloads.random_continuous_actions(rng, n, nc)))


@pytest.mark.parametrize("n,n_blue,n_orange,frameskip", [
    (65536, 1, 1, 8),     # one workgroup per resident slot
    (262144, 1, 1, 8),    # four rounds of workgroups
    (2048, 1, 1, 8),      # a grid smaller than the device
    (16384, 3, 3, 4),
])
def test_window_stage_sums_match_the_launch_time(gpu, n, n_blue, n_orange, frameskip):
    env, rng = _env(n, n_blue, n_orange, frameskip, seed=90 + n_blue)
    _steps(env, rng, n, n_blue + n_orange, 3)
    env.enable_tick_timing(True, ticks=False, stages=True)
    steps = 12
    _steps(env, rng, n, n_blue + n_orange, steps)
    table, fig = stage_profile(env, n)
    env.enable_tick_timing(False)
    print(f"\n{n} sims {n_blue}v{n_orange} frameskip {frameskip}\n{table}", flush=True)
    assert fig["ticks"] == steps * frameskip
    assert list(fig["stages"]) == STAGES
    assert list(fig["last_workgroup"]) == STAGES + ["start delay"]
    assert all(fig["stages"][s] > 0.0 and fig["last_workgroup"][s] > 0.0 for s in STAGES), fig
    span, launch = fig["span_us"], fig["launch_us"]
    assert SPAN_LOW <= span / launch <= SPAN_HIGH, (span / launch, fig)
    assert sum(fig["last_workgroup"].values()) == pytest.approx(span, rel=0.01)
    assert sum(fig["stages"].values()) <= span * 1.001
    # the reading cleared the period
    env.enable_tick_timing(True, ticks=False, stages=True)
    again = env.stage_timing()
    assert (again["ticks"], again["launch_us"], again["span_us"]) == (0, 0.0, 0.0)
    assert not any(again["stages"].values()) and not any(again["last_workgroup"].values())
    env.enable_tick_timing(False)


def test_profiled_window_kernel_changes_no_result(gpu):
    n, nc, frameskip = 4096, 4, 8
    plain, rng_a = _env(n, 2, 2, frameskip, seed=95)
    profiled, rng_b = _env(n, 2, 2, frameskip, seed=95)
    profiled.enable_tick_timing(True, ticks=False, stages=True)
    for step in range(10):
        actions = dev(workloads.random_continuous_actions(rng_a, n, nc))
        plain.step_continuous(actions)
        profiled.step_continuous(actions)
        a, b = gpu_state(plain), gpu_state(profiled)
        assert a[0].tobytes() == b[0].tobytes() and a[1].tobytes() == b[1].tobytes(), step
    assert profiled.stage_timing()["ticks"] == 10 * frameskip


def test_phase_kernel_stages_are_the_kernel_times(gpu):
    """With the phase kernels each stage is one kernel's event time; the pads
    run in the finish kernel; tick timing enabled alongside sees the same
    launches."""
    n, frameskip, steps = 8192, 4, 5
    env, rng = _env(n, 1, 1, frameskip, seed=96, window=0)
    env.enable_tick_timing(True, ticks=True, stages=True)
    _steps(env, rng, n, 2, steps)
    prof = env.stage_timing()
    stages, last, ticks = prof["stages"], prof["last_workgroup"], prof["ticks"]
    kernels = env.tick_timing()
    env.enable_tick_timing(False)
    ticks_run = steps * frameskip
    assert ticks == ticks_run and stages["boost-pads"] == 0.0
    names = ["contactKernel", "carArenaKernel", "ballKernel", "finishKernel"]
    assert sorted(kernels) == sorted(names)
    for stage, name in zip(STAGES, names):
        ms, launches = kernels[name]
        assert launches == ticks_run
        assert stages[stage] == last[stage] == pytest.approx(ms * 1e3 / ticks_run, rel=1e-9)
    assert prof["launch_us"] == prof["span_us"] == pytest.approx(sum(stages.values()), rel=1e-9)
    assert last["start delay"] == 0.0


def test_stage_profile_errors(gpu):
    n = 1024
    env, rng = _env(n, 1, 1, 2, seed=97)
    with pytest.raises(ValueError, match="not enabled"):
        env.stage_timing()
    env.enable_tick_timing(True, stages=True)
    _steps(env, rng, n, 2, 1)
    env.tick_window = 0
    _steps(env, rng, n, 2, 1)
    with pytest.raises(ValueError, match="launch shape changed"):
        env.stage_timing()
    # the failed read cleared the period; a period of one shape reads
    _steps(env, rng, n, 2, 2)
    assert env.stage_timing()["ticks"] == 4
    env.tick_window = 64
    env.tick_streams = 2
    _steps(env, rng, n, 2, 1)
    env.tick_streams = 1
    _steps(env, rng, n, 2, 1)
    with pytest.raises(ValueError, match="launch shape changed"):
        env.stage_timing()
    env.enable_tick_timing(False)


def test_event_pool_folds_beyond_its_size(gpu):
    """More timed launches than the event pool holds (1024): every launch is
    still counted, with a positive duration."""
    n, frameskip, steps = 256, 1, 700
    env, rng = _env(n, 1, 1, frameskip, seed=98, window=0)
    actions = dev(workloads.random_continuous_actions(rng, n, 2))
    env.enable_tick_timing(True, ticks=True, packing=True)
    for _ in range(steps):
        env.step_continuous(actions)
    timing = env.tick_timing()
    env.enable_tick_timing(False)
    assert {k: v[1] for k, v in timing.items()} == {
        "contactKernel": steps, "carArenaKernel": steps, "ballKernel": steps, "finishKernel": steps,
        "stepEnvKernel": steps}
    assert all(v[0] > 0.0 for v in timing.values())
