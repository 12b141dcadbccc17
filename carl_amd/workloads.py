"""Seeded synthetic workloads for the benchmark and the parity tests.

Distributions (the headline benchmark workload):
  * cars: even simulations keep their kickoff spawn; odd simulations get
    (x, y) ~ U[-3300, 3300] x U[-4300, 4300] (inside the field, clear of the
    side-wall ramps and corners) at z = 17, yaw ~ U[-pi, pi), planar velocity
    with uniform direction and |v| ~ U[0, 2300], boost ~ U[0, 100];
  * ball: x ~ U[-3000, 3000], y ~ U[-4000, 4000], z ~ U[100, 1500],
    |v| ~ U[0, 3000] in a uniform direction, |w| ~ U[0, 6];
  * continuous actions: steer/yaw, pitch, throttle, air roll ~ U[-1, 1];
    powerslide, boost, jump ~ Bernoulli(0.5);
  * direct controls (5 floats + 3 ints): throttle, steer, pitch, yaw, roll
    ~ U[-1, 1]; jump, boost, handbrake ~ Bernoulli(0.5).
"""
from __future__ import annotations

import numpy as np


def _unit_vectors(rng: np.random.Generator, n: int) -> np.ndarray:
    v = rng.normal(size=(n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def random_reset_state(rng: np.random.Generator, n_rows: int, n_cars: int,
                       cluster_radius: float | None = None) -> dict[str, np.ndarray]:
    """apply_reset_state inputs for n_rows simulations (physics units).

    With cluster_radius, cars are placed within that distance of the ball
    (horizontally) to force car-car and car-ball contacts.
    """
    ball_pos = np.stack([rng.uniform(-3000, 3000, n_rows), rng.uniform(-4000, 4000, n_rows),
                         rng.uniform(100, 1500, n_rows)], axis=1)
    ball_vel = _unit_vectors(rng, n_rows) * rng.uniform(0, 3000, (n_rows, 1))
    ball_ang = _unit_vectors(rng, n_rows) * rng.uniform(0, 6, (n_rows, 1))
    if cluster_radius is None:
        cx = rng.uniform(-3300, 3300, (n_rows, n_cars))
        cy = rng.uniform(-4300, 4300, (n_rows, n_cars))
    else:
        r = cluster_radius * np.sqrt(rng.uniform(0, 1, (n_rows, n_cars)))
        a = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
        cx = np.clip(ball_pos[:, :1] + r * np.cos(a), -3300, 3300)
        cy = np.clip(ball_pos[:, 1:2] + r * np.sin(a), -4300, 4300)
    car_pos = np.stack([cx, cy, np.full((n_rows, n_cars), 17.0)], axis=-1)
    yaw = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
    rot = np.zeros((n_rows, n_cars, 4))
    rot[..., 2] = np.sin(yaw / 2)
    rot[..., 3] = np.cos(yaw / 2)
    heading = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
    speed = rng.uniform(0, 2300, (n_rows, n_cars))
    car_vel = np.stack([speed * np.cos(heading), speed * np.sin(heading), np.zeros_like(speed)], axis=-1)
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    return {
        "ball_position": f32(ball_pos),
        "ball_velocity": f32(ball_vel),
        "ball_angular_velocity": f32(ball_ang),
        "car_position": f32(car_pos),
        "car_rotation": f32(rot),
        "car_velocity": f32(car_vel),
        "car_angular_velocity": f32(np.zeros((n_rows, n_cars, 3))),
        "car_demoed": np.zeros((n_rows, n_cars), dtype=np.bool_),
        "car_boost": f32(rng.uniform(0, 100, (n_rows, n_cars))),
    }


def random_continuous_actions(rng: np.random.Generator, n_sim: int, n_cars: int) -> np.ndarray:
    a = rng.uniform(-1, 1, (n_sim, n_cars, 7))
    for f in (3, 4, 6):
        a[..., f] = (rng.uniform(0, 1, (n_sim, n_cars)) < 0.5).astype(np.float64)
    return np.ascontiguousarray(a, dtype=np.float32)


def random_discrete_actions(rng: np.random.Generator, n_sim: int, n_cars: int) -> np.ndarray:
    nvec = np.array([3, 3, 3, 2, 2, 3, 2])
    return np.ascontiguousarray(rng.integers(0, nvec, size=(n_sim, n_cars, 7)), dtype=np.int32)


CONTROLS_DTYPE = np.dtype([("throttle", "<f4"), ("steer", "<f4"), ("yaw", "<f4"), ("pitch", "<f4"),
                           ("roll", "<f4"), ("jump", "<i4"), ("boost", "<i4"), ("slide", "<i4")])


def random_direct_controls(rng: np.random.Generator, n: int) -> np.ndarray:
    c = np.zeros(n, dtype=CONTROLS_DTYPE)
    for f in ("throttle", "steer", "yaw", "pitch", "roll"):
        c[f] = rng.uniform(-1, 1, n)
    for f in ("jump", "boost", "slide"):
        c[f] = rng.uniform(0, 1, n) < 0.5
    return c
