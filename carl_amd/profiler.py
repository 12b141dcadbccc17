"""Stage profile of the tick, printed as the reference's ScopedCudaProfiler
prints its PROFILE stages (include/Cuda/Profiler.cuh:119-162): one row of
us/tick per stage, the aggregate, and simulation ticks per second with a K/M
suffix.

The figures come from `Env.stage_timing()` after
`Env.enable_tick_timing(True, stages=True)` (`carl_env_stage_timing` in
include/carl_amd.h).  The reference's stages are whole kernel launches, so
one column holds all of a stage's time.  Here the phases of a tick run
inside one window launch, so the table has two columns: `us/tick`, each
phase's share of the device (workgroup time over the workgroups resident at
once), and `last wg`, the critical path (the phases of the workgroup that
finished each launch last, and the delay of its start).  The first column
sums to less than the launch by the launch's imbalance; the second sums to
the launch's span.
"""
from __future__ import annotations


def _rate(ticks_per_s: float) -> str:
    """The reference's rate text: one decimal, M above 1e6, K above 1e3."""
    for scale, unit in ((1e6, "M"), (1e3, "K")):
        if ticks_per_s >= scale:
            return f"{ticks_per_s / scale:.1f}{unit}"
    return f"{ticks_per_s:.1f}"


def format_stage_table(profile: dict, n_sim: int) -> str:
    """The table for one profile period (a dict as `Env.stage_timing()`
    returns it); n_sim is the simulations per tick (the reference's
    simScale), and `sim ticks/s` is n_sim over the launch time."""
    stages, last = profile["stages"], profile["last_workgroup"]
    rule = "-" * 36
    lines = [f"{'stage':<14s} {'us/tick':>10s} {'last wg':>10s}", rule]
    lines += [f"{name:<14s} {us:10.3f} {last[name]:10.3f}" for name, us in stages.items()]
    lines.append(f"{'start delay':<14s} {'':>10s} {last['start delay']:10.3f}")
    lines.append(rule)
    lines.append(f"{'aggregate':<14s} {sum(stages.values()):10.3f} {sum(last.values()):10.3f}")
    lines.append(f"{'span':<14s} {profile['span_us']:10.3f}")
    lines.append(f"{'launch':<14s} {profile['launch_us']:10.3f}")
    launch = profile["launch_us"]
    lines.append(f"{'sim ticks/s':<14s} {_rate(n_sim * 1e6 / launch if launch > 0 else 0.0):>10s}")
    return "\n".join(lines)


def stage_profile(env, n_sim: int) -> tuple[str, dict]:
    """Reads and clears the environment's stage profile; returns the table and
    the figures (`Env.stage_timing()`'s dict plus `sim_ticks_per_s`)."""
    profile = env.stage_timing()
    launch = profile["launch_us"]
    profile["sim_ticks_per_s"] = n_sim * 1e6 / launch if launch > 0 else 0.0
    return format_stage_table(profile, n_sim), profile
