"""Engine-vs-oracle harness for the GPU parity tests.

A `Pair` drives the HIP engine (carl_amd._carl.Env) and the CPU oracle with
identical calls and inputs, and compares every output buffer and the full
persistent state (include/carl_amd.h layout) field by field.
"""
from __future__ import annotations

import numpy as np
import torch

import carl_amd
from abi import CAR_NAMES, SIM_NAMES
from oracle_py import OracleEnv

OUTPUTS = ("obs", "transition_obs", "state", "transition_state", "rewards", "dones", "score_difference",
           "episode_ticks", "transition_score_difference", "transition_episode_ticks", "overtime",
           "transition_overtime", "actions", "continuous_actions")


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def gpu_outputs(env) -> dict[str, np.ndarray]:
    env.synchronize()
    out = {}
    for name in OUTPUTS:
        t = torch.from_dlpack(getattr(env, "get_" + name)())
        out[name] = t.cpu().numpy().copy()
    return out


def gpu_state(env):
    car, sim, tick = env.export_state()
    n_cars = env.n_cars
    car = np.frombuffer(car, dtype=np.uint32).reshape(len(CAR_NAMES), -1)
    sim = np.frombuffer(sim, dtype=np.uint32).reshape(len(SIM_NAMES), -1)
    assert car.shape[1] == env.n_sim * n_cars
    return car, sim, tick


def describe_mismatch(names, a, b, limit=8) -> list[str]:
    """Per-field report of where two state blocks (planes x items) differ."""
    lines = []
    for f in range(a.shape[0]):
        bad = np.nonzero(a[f] != b[f])[0]
        if len(bad) == 0:
            continue
        fa = a[f].view(np.float32)
        fb = b[f].view(np.float32)
        diff = np.abs(fa[bad].astype(np.float64) - fb[bad].astype(np.float64))
        lines.append(f"{names[f]}: {len(bad)}/{a.shape[1]} differ, first item {bad[0]} "
                     f"(engine {fa[bad[0]]!r} / {a[f][bad[0]]:#x}, oracle {fb[bad[0]]!r} / {b[f][bad[0]]:#x}), "
                     f"max |d| {diff.max():.3g}")
        if len(lines) >= limit:
            break
    return lines


class Pair:
    def __init__(self, n_sim, n_blue, n_orange, seed=7, frameskip=1, invert_orange=True, normalize=False,
                 previous_controls=False, obj_path=None):
        """obj_path: the oracle's arena mesh (the engine reads CARL_ARENA_OBJ,
        which the caller sets to the same file)."""
        self.gpu = carl_amd.Env(n_sim, n_blue, n_orange, seed, frameskip, invert_orange, normalize,
                                previous_controls)
        kw = {} if obj_path is None else {"obj_path": obj_path}
        self.cpu = OracleEnv(n_sim, n_blue, n_orange, seed, frameskip, invert_orange, normalize, previous_controls,
                             **kw)
        self.n_sim, self.n_cars = n_sim, n_blue + n_orange

    def close(self):
        self.cpu.close()
        del self.gpu

    # -- mirrored calls
    def step_continuous(self, actions: np.ndarray):
        self.gpu.step_continuous(dev(actions))
        self.cpu.step(np.ascontiguousarray(actions, dtype=np.float32))

    def step_discrete(self, actions: np.ndarray):
        self.gpu.step(dev(actions.astype(np.int32)))
        self.cpu.step(np.ascontiguousarray(actions, dtype=np.int32))

    def tick(self, actions: np.ndarray, kind: int, n_ticks: int = 1):
        """Bare physics ticks (no packing) on the same actions for both sides;
        kind 2 takes a structured array of direct controls."""
        words = np.ascontiguousarray(actions).view(np.int32 if kind != 1 else np.float32)
        self.gpu.tick(dev(words.reshape(-1)), kind, n_ticks)
        self.cpu.tick(np.ascontiguousarray(actions), kind, n_ticks)

    def apply_reset_state(self, values: dict, **kw):
        gv = {k: dev(v) for k, v in values.items()}
        gk = {k: (dev(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
        self.gpu.apply_reset_state(**gv, **gk)
        self.cpu.apply_reset_state(**values, **kw)

    def set_param(self, name: str, value: int):
        setattr(self.gpu, name, value)
        ids = {"max_ticks": 0, "overtime_timeout_ticks": 1, "no_touch_timeout_ticks": 2, "frameskip": 3}
        self.cpu.set_param(ids[name], value)

    # -- comparisons
    def output_mismatches(self, names=OUTPUTS, atol=0.0) -> list[str]:
        g = gpu_outputs(self.gpu)
        report = []
        for name in names:
            a, b = g[name], self.cpu.get(name)
            a = a.reshape(b.shape)
            if atol == 0.0:
                bad = np.nonzero((a != b).reshape(-1))[0] if a.dtype != np.float32 else \
                    np.nonzero((a.view(np.uint32) != b.view(np.uint32)).reshape(-1))[0]
            else:
                bad = np.nonzero((np.abs(a.astype(np.float64) - b.astype(np.float64)) > atol).reshape(-1))[0]
            if len(bad):
                i = bad[0]
                report.append(f"{name}: {len(bad)}/{a.size} differ, first flat index {i} "
                              f"(engine {a.reshape(-1)[i]!r}, oracle {b.reshape(-1)[i]!r})")
        return report

    def fresh_output_mismatches(self) -> list[str]:
        """output_mismatches after sync_oracle_from_engine: the transition
        observation rows are written only for the simulations that finish in
        a step (the others keep older rows, which the oracle never wrote), so
        that buffer is compared on this step's finished rows."""
        report = self.output_mismatches([n for n in OUTPUTS if n != "transition_obs"])
        done = gpu_outputs(self.gpu)["dones"].reshape(-1).astype(bool)
        a = torch.from_dlpack(self.gpu.get_transition_obs()).cpu().numpy().reshape(self.n_sim, -1)[done]
        b = self.cpu.get("transition_obs").reshape(self.n_sim, -1)[done]
        bad = np.nonzero((a.view(np.uint32) != b.view(np.uint32)).any(axis=1))[0]
        if len(bad):
            report.append(f"transition_obs: {len(bad)}/{int(done.sum())} finished rows differ, "
                          f"first simulation {np.nonzero(done)[0][bad[0]]}")
        return report

    def state_mismatches(self) -> list[str]:
        gc, gs, gt = gpu_state(self.gpu)
        oc, os_, ot = self.cpu.export_state()
        rep = []
        if gt != ot:
            rep.append(f"tick counter engine {gt} oracle {ot}")
        rep += describe_mismatch(CAR_NAMES, gc, oc)
        rep += describe_mismatch(SIM_NAMES, gs, os_)
        return rep

    def import_state(self, car: np.ndarray, sim: np.ndarray, tick: int):
        """Load one persistent state (include/carl_amd.h layout) into both sides."""
        car = np.ascontiguousarray(car, dtype=np.uint32)
        sim = np.ascontiguousarray(sim, dtype=np.uint32)
        self.gpu.import_state(car.tobytes(), sim.tobytes(), int(tick))
        self.cpu.import_state(car, sim, int(tick))

    def sync_oracle_from_engine(self):
        """Copy the engine's persistent state into the oracle."""
        car, sim, tick = gpu_state(self.gpu)
        self.cpu.import_state(car, sim, tick)


def dense_geometry_reset_state(rng: np.random.Generator, n_rows: int, n_cars: int) -> dict[str, np.ndarray]:
    """Reset inputs that put cars and balls where the arena mesh is densest:
    corner ramps, goal mouths and posts, side walls (car on the wall) and the
    ceiling, with velocities pointing into the geometry."""
    spots = np.array([[3900.0, 4950.0, 60.0], [-3900.0, -4950.0, 60.0], [890.0, 5100.0, 100.0],
                      [-890.0, -5100.0, 300.0], [0.0, 5300.0, 200.0], [4050.0, 0.0, 300.0],
                      [-4050.0, 1000.0, 600.0], [2000.0, -3000.0, 1980.0], [3500.0, -4600.0, 200.0]])
    pick = rng.integers(0, len(spots), (n_rows, n_cars))
    car_pos = spots[pick] + rng.uniform(-60, 60, (n_rows, n_cars, 3))
    axis = rng.normal(size=(n_rows, n_cars, 3))
    axis /= np.linalg.norm(axis, axis=-1, keepdims=True)
    ang = rng.uniform(-np.pi, np.pi, (n_rows, n_cars, 1))
    rot = np.concatenate([axis * np.sin(ang / 2), np.cos(ang / 2)], axis=-1)
    toward = -car_pos / np.maximum(np.linalg.norm(car_pos, axis=-1, keepdims=True), 1.0)
    car_vel = -toward * rng.uniform(0, 1500, (n_rows, n_cars, 1))     # into the wall
    bpick = rng.integers(0, len(spots), n_rows)
    ball_pos = spots[bpick] + rng.uniform(-80, 80, (n_rows, 3))
    ball_pos[:, 2] = np.maximum(ball_pos[:, 2], 95.0)
    ball_vel = rng.normal(size=(n_rows, 3)) * 800.0
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    return {
        "ball_position": f32(ball_pos), "ball_velocity": f32(ball_vel),
        "ball_angular_velocity": f32(rng.normal(size=(n_rows, 3))),
        "car_position": f32(car_pos), "car_rotation": f32(rot), "car_velocity": f32(car_vel),
        "car_angular_velocity": f32(rng.normal(size=(n_rows, n_cars, 3))),
        "car_demoed": np.zeros((n_rows, n_cars), dtype=np.bool_),
        "car_boost": f32(rng.uniform(0, 100, (n_rows, n_cars))),
    }


# boost pad centres (x, y, z), big pads first: the standard soccar layout
PAD_XYZ = np.array([
    (-3584, 0, 73), (3584, 0, 73), (-3072, 4096, 73), (3072, 4096, 73), (-3072, -4096, 73), (3072, -4096, 73),
    (0, -4240, 70), (-1792, -4184, 70), (1792, -4184, 70), (-940, -3308, 70), (940, -3308, 70), (0, -2816, 70),
    (-3584, -2484, 70), (3584, -2484, 70), (-1788, -2300, 70), (1788, -2300, 70), (-2048, -1036, 70),
    (0, -1024, 70), (2048, -1036, 70), (-1024, 0, 70), (1024, 0, 70), (-2048, 1036, 70), (0, 1024, 70),
    (2048, 1036, 70), (-1788, 2300, 70), (1788, 2300, 70), (-3584, 2484, 70), (3584, 2484, 70), (0, 2816, 70),
    (-940, 3308, 70), (940, 3308, 70), (-1792, 4184, 70), (1792, 4184, 70), (0, 4240, 70)], dtype=np.float64)


def pad_reset_state(rng: np.random.Generator, n_rows: int, n_cars: int) -> dict[str, np.ndarray]:
    """Reset inputs with every car parked on a boost pad (about a third of the
    cars share the first car's pad, so the last car in order takes it), with
    empty, partial or full boost and a few cars demoed: pickups, pad
    cooldowns and the pad split across threads on every tick."""
    pads = rng.integers(0, len(PAD_XYZ), (n_rows, n_cars))
    share = rng.uniform(size=(n_rows, n_cars)) < 0.35
    pads[:, 1:] = np.where(share[:, 1:], pads[:, :1], pads[:, 1:])
    car_pos = PAD_XYZ[pads].copy()
    car_pos[..., :2] += rng.uniform(-90, 90, (n_rows, n_cars, 2))
    car_pos[..., 2] = 17.0
    yaw = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
    rot = np.stack([np.zeros_like(yaw), np.zeros_like(yaw), np.sin(yaw / 2), np.cos(yaw / 2)], axis=-1)
    car_vel = np.concatenate([rng.uniform(-300, 300, (n_rows, n_cars, 2)), np.zeros((n_rows, n_cars, 1))], axis=-1)
    boost = rng.choice(np.array([0.0, 12.0, 50.0, 99.5, 100.0]), size=(n_rows, n_cars))
    ball_pos = np.stack([rng.uniform(-3000, 3000, n_rows), rng.uniform(-4000, 4000, n_rows),
                         rng.uniform(100, 1500, n_rows)], axis=1)
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    return {
        "ball_position": f32(ball_pos), "ball_velocity": f32(rng.normal(size=(n_rows, 3)) * 500.0),
        "ball_angular_velocity": f32(rng.normal(size=(n_rows, 3))),
        "car_position": f32(car_pos), "car_rotation": f32(rot), "car_velocity": f32(car_vel),
        "car_angular_velocity": f32(np.zeros((n_rows, n_cars, 3))),
        "car_demoed": rng.uniform(size=(n_rows, n_cars)) < 0.05,
        "car_boost": f32(boost),
    }
