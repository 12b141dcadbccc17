"""CARL step-engine benchmark on one MI355X.

Workload (headline): 1v1, fp32, n_sim = 65536, tick_skip = 8; even arenas
start from kickoff, odd arenas from seeded random states; seeded random
continuous actions (a pool of 64 action batches cycled per step); every env
step runs the full native sequence - 8 physics ticks, rewards/dones,
transition state/obs, done resets, obs/state packing - plus the default score
reward (score delta x team sign).  Inputs are resident in HBM before timing.

Prints one JSON line:
  value          sim-ticks/s = n_sim * tick_skip * steps / seconds
  roofline       the dominant tick kernel (largest share of the timed
                 steps): its algorithmic bytes per launch (kernel_bytes x
                 n_sim) / its average launch time, from HIP events the engine
                 records around every tick kernel on its own stream during
                 the timed steps, against 8 TB/s
  tick_pipeline  the whole tick (four kernels) against the 1,488 B per 1v1
                 sim-tick floor: persistent state read + written + actions
  packing        the step's packing kernel (packing_bytes x n_sim per
                 launch) against 8 TB/s, timed the same way over up to 200
                 further steps after the timed region
  cpu_baseline   the CPU model of the same physics (oracle/liboracle.so), one
                 1v1 arena per thread on this host's cores, direct controls
                 held 8 ticks (bounded sample)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "sim-ticks/sec (n_sim×ticks) 1v1 n_sim=65536 on 1 GPU; % HBM roofline"
HBM_PEAK_GBS = 8000.0
BYTES_PER_CAR = 232      # persistent per-car state carried across ticks
BYTES_PER_SIM = 252      # persistent per-simulation state
ACTION_BYTES = 28        # one car's action per tick


def tick_bytes(n_cars: int) -> int:
    """Algorithmic HBM bytes of one simulation tick (state read + write + actions)."""
    return 2 * (n_cars * BYTES_PER_CAR + BYTES_PER_SIM) + n_cars * ACTION_BYTES


def kernel_bytes(kernel: str, n_cars: int, ticks: int) -> int:
    """Algorithmic HBM bytes per simulation of one launch of a tick kernel, on
    the common path (no demolition, no car-car contact, ball awake): the state
    words the kernel must read and write once each.
      tickWindow every tick of the step (`ticks`) in one launch: the tick
                 floor (persistent state read + written, actions) per tick
      contact    per car: pose/velocity/demo flag 17 words read, 21-word
                 workspace written; per sim: ball position (3 words)
      carArena   per car: workspace 21 + actions 7 + car state 54 words read,
                 car state 69 words written
      ball       per pair: both cars' demo flag, centre and rotation (16
                 words); per sim: episode clock read + written (2 words),
                 ball state 28 words read, 30 written; per car: demo flag,
                 centre and last-hit tick (5 words)
      finish     per car: 18 words read, 17 written; per sim: 34 pad
                 cooldowns read, ball velocity/spin/impulse 9 read + 9 written
    """
    if kernel == "tickWindowKernel":
        return tick_bytes(n_cars) * ticks
    pairs = n_cars * (n_cars - 1) // 2
    words = {
        "contactKernel": n_cars * (17 + 21) + 3,
        "carArenaKernel": n_cars * (21 + 7 + 54 + 69),
        "ballKernel": pairs * 16 + 2 + 28 + 30 + n_cars * 5,
        "finishKernel": n_cars * (18 + 17) + 34 + 18,
    }[kernel]
    return 4 * words


PACK_KERNEL = "stepEnvKernel"


def packing_bytes(n_cars: int, obs_dim: int, state_dim: int) -> int:
    """Algorithmic HBM bytes per simulation of one launch of the step's packing
    kernel: every output written once, the state words its rows read once,
    and the actions read and kept once (the transition observations of the
    finished simulations depend on the data and are left out).
      writes  observations n_cars*obs_dim, state and transition state
              2*state_dim words; rewards, score differences and episode ticks
              (current and transition) 4 B each, dones and overtime flags
              1 B each (23 B); the kept actions 28 B per car
      reads   per car 26 state words (pose, velocity, spin, boost and flag
              words of the rows); per simulation 49 (ball 9, pad cooldowns
              34, score, clock and touch words 6); the actions 28 B per car
    """
    writes = 4 * (n_cars * obs_dim + 2 * state_dim) + 23 + ACTION_BYTES * n_cars
    reads = 4 * (26 * n_cars + 49) + ACTION_BYTES * n_cars
    return writes + reads


# committed rocprofv3 FETCH_SIZE / WRITE_SIZE summaries of the headline
# workload: the 20-step bench and the 1,000-step default
TRAFFIC_FILES = (ROOT / "profiles" / "hbm_traffic_1v1_n65536_ts8.md",
                 ROOT / "profiles" / "hbm_traffic_1v1_n65536_ts8_steps1000.md")


def measured_traffic(kernel: str, n_sim: int, n_cars: int, tick_skip: int, parts: int, window: int,
                     steps: int, warmup: int, tag: str = "traffic"):
    """(HBM bytes per dispatch of `kernel`, summary file name) from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summaries of the headline
    workload (copy-calibrated), for the same window of steps (`steps` timed
    after `warmup`; tag "traffic-after" for the steps after them, at most
    200, over which the packing kernel is timed); (None, None) for any other
    workload, launch shape or window, or when no summary holds it."""
    if (n_sim, n_cars, tick_skip, parts, window) != (65536, 2, 8, 1, 64):
        return None, None
    for path in TRAFFIC_FILES:
        if not path.is_file():
            continue
        for line in path.read_text().splitlines():
            f = line.split()
            if len(f) == 5 and f[0] == tag and f[1] == kernel and (int(f[2]), int(f[3])) == (steps, warmup):
                return int(f[4]), path.name
    return None, None


def _read_csv(path: Path) -> list[dict]:
    import csv

    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def summarize_rocprof(trace_dir: str | None, fetch_dir: str | None, write_dir: str | None,
                      copy_fetch_dir: str | None, copy_write_dir: str | None, copy_mib: int,
                      steps: int, warmup: int) -> None:
    """Markdown summary of rocprofv3 output of one bench run: per kernel, the
    average dispatch duration over all dispatches, over the timed env steps
    (warmup .. warmup+steps-1) and over the `steps` steps after them (over
    which the bench times the packing kernel), and the copy-calibrated
    FETCH_SIZE / WRITE_SIZE bytes per dispatch over the same windows.  Every
    env step ends with one packing-kernel dispatch, so a window is the range
    of dispatch ids between two of those: a kernel counts in the window its
    dispatches fall into (set-up dispatches fall into none)."""
    def short(name: str) -> str:
        # "(anonymous namespace)::tickWindowKernel(carl::Dev, ...)" -> "tickWindowKernel"
        head = name.replace("(anonymous namespace)::", "")
        return head.split("(")[0].split("<")[0].split()[-1] if "(" in head else head

    def kernel_series(rows, value):
        # kernel -> [(dispatch id, value)] in dispatch order
        out: dict[str, list] = {}
        for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
            out.setdefault(short(r["Kernel_Name"]), []).append((int(r["Dispatch_Id"]), value(r)))
        return out

    def step_windows(series):
        # dispatch-id ranges (lo, hi] of the timed steps and of the steps after
        ends = [i for i, _ in series.get(PACK_KERNEL, [])]

        def end(step):
            return -1 if step < 0 or not ends else ends[min(step, len(ends) - 1)]
        return {"timed": (end(warmup - 1), end(warmup + steps - 1)),
                "after": (end(warmup + steps - 1), end(warmup + 2 * steps - 1))}

    def pick(xs, window):
        lo, hi = window
        return [v for i, v in xs if lo < i <= hi]

    def mean(xs):
        return sum(xs) / len(xs) if xs else float("nan")

    if trace_dir:
        rows = _read_csv(next(Path(trace_dir).rglob("*kernel_trace.csv")))
        dur = kernel_series(rows, lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        windows = step_windows(dur)
        print("| kernel | dispatches | avg us (all) | avg us (timed steps) | avg us (steps after) |")
        print("|---|---|---|---|---|")
        for k, xs in sorted(dur.items(), key=lambda kv: -sum(v for _, v in kv[1])):
            w = {n: mean(pick(xs, win)) for n, win in windows.items()}
            print(f"| {k} | {len(xs)} | {mean([v for _, v in xs]):.1f} | {w['timed']:.1f} | {w['after']:.1f} |")
        print()

    def counter(dir_, name):
        rows = [r for r in _read_csv(next(Path(dir_).rglob("*counter_collection.csv"))) if r["Counter_Name"] == name]
        return kernel_series(rows, lambda r: float(r["Counter_Value"]))

    if fetch_dir and write_dir and copy_fetch_dir and copy_write_dir:
        copy_bytes = copy_mib * (1 << 20)
        cf = max(mean([x for _, x in v]) for v in counter(copy_fetch_dir, "FETCH_SIZE").values())
        cw = max(mean([x for _, x in v]) for v in counter(copy_write_dir, "WRITE_SIZE").values())
        f_scale, w_scale = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
        print(f"Calibration: a {copy_mib} MiB device copy reads FETCH_SIZE {cf:.1f} KiB and WRITE_SIZE {cw:.1f} KiB: "
              f"FETCH_SIZE x {f_scale:.3f}, WRITE_SIZE x {w_scale:.3f} to bytes.")
        print()
        fetch, write = counter(fetch_dir, "FETCH_SIZE"), counter(write_dir, "WRITE_SIZE")
        fwin, wwin = step_windows(fetch), step_windows(write)
        print("| kernel | window | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes (scaled) |")
        print("|---|---|---|---|---|---|")
        lines = []
        for k in sorted(fetch, key=lambda k: -sum(v for _, v in fetch[k])):
            for n in fwin:
                fk, wk = pick(fetch[k], fwin[n]), pick(write.get(k, []), wwin[n])
                if not fk or not wk:
                    continue
                total = mean(fk) * 1024 * f_scale + mean(wk) * 1024 * w_scale
                print(f"| {k} | {n} | {len(fk)} | {mean(fk):.1f} | {mean(wk):.1f} | {total / 1e6:.1f} MB |")
                if k in ("tickWindowKernel", PACK_KERNEL):
                    tag = "traffic" if n == "timed" else "traffic-after"
                    lines.append(f"{tag} {k} {steps} {warmup} {int(total)}")
        print()
        print("Machine-readable (read by bench.py for `roofline.traffic` and `packing.traffic`):")
        print()
        for line in lines:
            print(line)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(ticks_per_thread: int, seed: int) -> dict:
    import ctypes

    lib_path = ROOT / "oracle" / "liboracle.so"
    lib = ctypes.CDLL(str(lib_path))
    lib.oracle_cpu_throughput.restype = ctypes.c_double
    lib.oracle_cpu_throughput.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    cores = len(os.sched_getaffinity(0))
    obj = str(ROOT / "carl_amd" / "assets" / "arena.obj").encode()
    rate = lib.oracle_cpu_throughput(obj, cores, ticks_per_thread, seed)
    return {
        "value": rate,
        "unit": "sim-ticks/s",
        "cores": cores,
        "per_core": rate / cores,
        "cpu_model": cpu_model(),
        "logical_cpus": os.cpu_count(),
        "kind": "port",
        "sample": (f"1v1 arena per thread x {cores} threads, {ticks_per_thread} ticks each, seeded direct "
                   f"controls held 8 ticks, done-resets every tick (CPU model of the same physics)"),
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--n-sim", type=int, default=65536)
    ap.add_argument("--blue", type=int, default=1)
    ap.add_argument("--orange", type=int, default=1)
    ap.add_argument("--tick-skip", type=int, default=8)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-ticks", type=int, default=1_200_000,
                    help="CPU-baseline ticks per host thread (0 skips it)")
    ap.add_argument("--tick-streams", type=int, default=0,
                    help="partitions of the simulations ticked on separate streams (0: engine default)")
    ap.add_argument("--tick-window", type=int, default=-1,
                    help="simulations per workgroup of the tick-window kernel, 0 for phase kernels "
                         "(-1: engine default)")
    ap.add_argument("--tick-balance", type=int, default=-1, choices=(-1, 0, 1),
                    help="1v1 window launches dealt to the workgroups by the last launch's contact work "
                         "(1), or workgroups of consecutive simulations (0); -1: engine default")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (HBM counter calibration) and exit")
    ap.add_argument("--summarize-rocprof", nargs=5, metavar=("TRACE", "FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="print a markdown summary of rocprofv3 output directories of one bench run "
                         "(use - for an absent one; --steps/--warmup name its window, --copy-mib the copy size)")
    ap.add_argument("--copy-mib", type=int, default=512)
    ap.add_argument("--clustered", action="store_true",
                    help="start every simulation from a clustered scene (every car within 500 uu of the ball, "
                         "at the floor, a wall or the ceiling) instead of half kickoffs, half random states")
    ap.add_argument("--reset-fraction", type=float, default=0.0,
                    help="after every step, reset this fraction of the simulations (a seeded Bernoulli mask) "
                         "from random states through apply_reset_state(reset_mask=...); the masks and states "
                         "come from pools made before timing")
    ap.add_argument("--stage-profile", action="store_true",
                    help="after the timed region, run further steps with the stage profile, print its table "
                         "on stderr and add it to the JSON line")
    args = ap.parse_args()

    if args.summarize_rocprof:
        dirs = [None if d == "-" else d for d in args.summarize_rocprof]
        summarize_rocprof(*dirs, args.copy_mib, args.steps, args.warmup)
        return

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(a multi-GPU run shards the simulations by range, one process per GPU, with no exchange "
              "inside a step)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 4 * n, "launches": 5}), flush=True)
        return

    import carl_amd
    from carl_amd import workloads
    from carl_amd.profiler import stage_profile

    dev = torch.device("cuda:0")
    n_sim, n_cars = args.n_sim, args.blue + args.orange
    rng = np.random.default_rng(args.seed)
    env = carl_amd.Env(n_sim, args.blue, args.orange, args.seed, args.tick_skip, True, False, False)
    stream = torch.cuda.ExternalStream(env.stream, device=dev)
    if args.tick_streams:
        env.tick_streams = args.tick_streams
    if args.tick_window >= 0:
        env.tick_window = args.tick_window
    if args.tick_balance >= 0:
        env.tick_balance = args.tick_balance

    if args.clustered:
        reset = workloads.clustered_reset_state(rng, n_sim, n_cars)
        env.apply_reset_state(**{k: torch.from_numpy(v).to(dev) for k, v in reset.items()})
    else:
        odd = np.arange(1, n_sim, 2)
        reset = workloads.random_reset_state(rng, len(odd), n_cars)
        env.apply_reset_state(**{k: torch.from_numpy(v).to(dev) for k, v in reset.items()},
                              simulation_indices=torch.from_numpy(odd.astype(np.int64)).to(dev))
    pool = [torch.from_numpy(workloads.random_continuous_actions(rng, n_sim, n_cars)).to(dev) for _ in range(64)]
    resets, masks = [], []
    if args.reset_fraction > 0.0:
        for _ in range(4):
            resets.append({k: torch.from_numpy(v).to(dev)
                           for k, v in workloads.random_reset_state(rng, n_sim, n_cars).items()})
        masks = [torch.from_numpy(rng.uniform(0, 1, n_sim) < args.reset_fraction).to(dev) for _ in range(64)]
    team_sign = torch.tensor([1.0] * args.blue + [-1.0] * args.orange, device=dev)
    torch.cuda.synchronize()

    def env_step(i: int) -> torch.Tensor:
        env.step_continuous(pool[i % len(pool)])
        with torch.cuda.stream(stream):
            score = torch.from_dlpack(env.get_rewards())
            reward = (score[:, None] * team_sign).reshape(-1)  # default score reward
        if resets:
            env.apply_reset_state(**resets[i % len(resets)], reset_mask=masks[i % len(masks)])
        return reward

    for i in range(args.warmup):
        env_step(i)
    torch.cuda.synchronize()
    env.enable_tick_timing(True)      # HIP events around every tick kernel launch
    t0 = time.perf_counter()
    for i in range(args.steps):
        reward = env_step(i)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    timing = env.tick_timing()        # {kernel: (total ms, launches)} over the timed steps
    env.enable_tick_timing(False)
    # the packing kernel is timed over further steps, outside the timed region
    env.enable_tick_timing(True, ticks=False, packing=True)
    for i in range(args.steps, args.steps + min(args.steps, 200)):
        reward = env_step(i)
    timing.update(env.tick_timing())
    env.enable_tick_timing(False)
    stages = None
    if args.stage_profile:
        env.enable_tick_timing(True, ticks=False, stages=True)
        for i in range(args.steps, args.steps + min(args.steps, 200)):
            reward = env_step(i)
        table, stages = stage_profile(env, n_sim // min(env.tick_streams, n_sim))
        env.enable_tick_timing(False)
        print(table, file=sys.stderr, flush=True)
    del reward

    sim_ticks = n_sim * args.tick_skip * args.steps
    value = sim_ticks / seconds

    # dominant kernel: the tick kernel with the largest share of the timed
    # region, timed on the engine stream by the engine's own events
    pack_timing = timing.pop(PACK_KERNEL, None)
    kernel = max(timing, key=lambda k: timing[k][0])
    kernel_ms, launches = timing[kernel]
    launch_ms = kernel_ms / launches
    # each launch covers one partition of the simulations; the engine times
    # partition 0, which holds n_sim // tick_streams of them
    parts = min(env.tick_streams, n_sim)
    launch_sims = n_sim // parts
    launch_bytes = kernel_bytes(kernel, n_cars, args.tick_skip) * launch_sims
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    tick_ms = sum(ms for ms, _ in timing.values())
    traffic, traffic_source = measured_traffic(kernel, n_sim, n_cars, args.tick_skip, parts,
                                               env.tick_window_launch, args.steps, args.warmup)

    result = {
        "metric": METRIC,
        "value": value,
        "unit": "sim-ticks/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "env_steps_per_s": n_sim * args.steps / seconds,
        "config": {
            "workload": (f"{args.blue}v{args.orange} n_sim={n_sim} tick_skip={args.tick_skip}: "
                         + ("clustered scenes at the floor, walls and ceiling" if args.clustered
                            else "kickoff + seeded random states")
                         + ", seeded random continuous actions, obs/state packing, done resets, default score reward"
                         + (f", {args.reset_fraction:.0%} of the simulations reset from random states after "
                            "every step (masked apply_reset_state)" if args.reset_fraction > 0.0 else "")),
            "n_sim": n_sim,
            "n_cars": n_cars,
            "tick_skip": args.tick_skip,
            "parallelism": "single GPU",
            "tick_streams": parts,
            "tick_window": env.tick_window_launch,
            "balanced_deal": env.tick_balanced_launch,
            "timed_steps": f"env steps {args.warmup + 1}..{args.warmup + args.steps} after the initial reset",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": traffic_source,
            "launch_ms": launch_ms,
            "launches": launches,
            "bytes_per_launch": launch_bytes,
            "sims_per_launch": launch_sims,
        },
        "tick_kernels_ms_per_launch": {k: ms / n for k, (ms, n) in timing.items()},
        "tick_pipeline": {
            "share_of_timed_region": tick_ms / (seconds * 1e3),
            "bytes_per_sim_tick": tick_bytes(n_cars),
            "achieved_GBs": tick_bytes(n_cars) * sim_ticks / (tick_ms * 1e-3) / 1e9,
        },
    }
    if pack_timing:
        pack_ms = pack_timing[0] / pack_timing[1]
        state_dim = torch.from_dlpack(env.get_state()).shape[1]
        pack_bytes = packing_bytes(n_cars, env.obs_dim, state_dim) * n_sim
        pack_gbs = pack_bytes / (pack_ms * 1e-3) / 1e9
        result["packing"] = {
            "bound": "hbm",
            "kernel": PACK_KERNEL,
            "achieved": pack_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": pack_gbs / HBM_PEAK_GBS,
            "launch_ms": pack_ms,
            "launches": pack_timing[1],
            "bytes_per_launch": pack_bytes,
            "traffic": measured_traffic(PACK_KERNEL, n_sim, n_cars, args.tick_skip, parts,
                                        env.tick_window_launch, args.steps, args.warmup, tag="traffic-after")[0],
        }
    if stages is not None:
        result["stage_profile"] = stages
    if args.cpu_ticks > 0:
        result["cpu_baseline"] = cpu_baseline(args.cpu_ticks, args.seed)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
