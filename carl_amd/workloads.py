"""Seeded synthetic workloads for the benchmark and the parity tests.

Distributions (the headline benchmark workload; clustered_reset_state and
masked per-step resets for the 3v3 and 2v2 workloads):
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


def _quat_from_axes(fwd: np.ndarray, up: np.ndarray) -> np.ndarray:
    """(x, y, z, w) quaternions of the rotations taking the car's local x (nose)
    to fwd and local z (roof) to up; fwd and up unit and orthogonal."""
    left = np.cross(up, fwd)
    m = np.stack([fwd, left, up], axis=-1)             # columns: images of x, y, z
    tr = m[..., 0, 0] + m[..., 1, 1] + m[..., 2, 2]
    q = np.zeros(fwd.shape[:-1] + (4,))
    # Shepperd: the largest of w, x, y, z first
    cand = np.stack([tr, m[..., 0, 0], m[..., 1, 1], m[..., 2, 2]], axis=-1)
    k = np.argmax(cand, axis=-1)
    for i in range(4):
        sel = k == i
        mm = m[sel]
        if i == 0:
            r = np.sqrt(1.0 + tr[sel]) * 2.0
            q[sel] = np.stack([(mm[:, 2, 1] - mm[:, 1, 2]) / r, (mm[:, 0, 2] - mm[:, 2, 0]) / r,
                               (mm[:, 1, 0] - mm[:, 0, 1]) / r, 0.25 * r], axis=-1)
        else:
            a, b, c = (i - 1), i % 3, (i + 1) % 3
            r = np.sqrt(1.0 + mm[:, a, a] - mm[:, b, b] - mm[:, c, c]) * 2.0
            v = np.zeros((len(mm), 4))
            v[:, a] = 0.25 * r
            v[:, b] = (mm[:, b, a] + mm[:, a, b]) / r
            v[:, c] = (mm[:, c, a] + mm[:, a, c]) / r
            v[:, 3] = (mm[:, c, b] - mm[:, b, c]) / r
            q[sel] = v
    return q / np.linalg.norm(q, axis=-1, keepdims=True)


def _surface_spots(rng: np.random.Generator, n: int):
    """Per simulation a surface kind (floor, side wall, back wall, ceiling),
    a spot on it and its unit normal into the field.  Each spot keeps a disk
    of 321 uu (the farthest a car standing on the surface can be from the spot
    and still lie within 500 uu of the ball) on the flat part of its surface:
    side walls between the floor and ceiling ramps, back walls beside the
    goal, the ceiling inside its curved edges."""
    kind = rng.choice(4, size=n, p=[0.4, 0.2, 0.2, 0.2])   # floor, side wall, back wall, ceiling
    spot = np.zeros((n, 3))
    normal = np.zeros((n, 3))
    side = rng.choice(np.array([-1.0, 1.0]), size=n)
    fl, sw, bw, ce = kind == 0, kind == 1, kind == 2, kind == 3
    spot[fl] = np.stack([rng.uniform(-3000, 3000, fl.sum()), rng.uniform(-4000, 4000, fl.sum()),
                         np.zeros(fl.sum())], axis=1)
    normal[fl] = (0.0, 0.0, 1.0)
    spot[sw] = np.stack([side[sw] * 4096.0, rng.uniform(-2600, 2600, sw.sum()),
                         rng.uniform(700, 1300, sw.sum())], axis=1)
    normal[sw] = np.stack([-side[sw], np.zeros(sw.sum()), np.zeros(sw.sum())], axis=1)
    spot[bw] = np.stack([rng.choice(np.array([-1.0, 1.0]), size=bw.sum()) * rng.uniform(1400, 2400, bw.sum()),
                         side[bw] * 5120.0, rng.uniform(700, 1300, bw.sum())], axis=1)
    normal[bw] = np.stack([np.zeros(bw.sum()), -side[bw], np.zeros(bw.sum())], axis=1)
    spot[ce] = np.stack([rng.uniform(-2800, 2800, ce.sum()), rng.uniform(-3700, 3700, ce.sum()),
                         np.full(ce.sum(), 2044.0)], axis=1)
    normal[ce] = (0.0, 0.0, -1.0)
    return kind, spot, normal


def _tangent_basis(normal: np.ndarray):
    ref = np.where(np.abs(normal[..., 2:3]) > 0.9, np.array([1.0, 0.0, 0.0]), np.array([0.0, 0.0, 1.0]))
    t1 = np.cross(normal, ref)
    t1 /= np.linalg.norm(t1, axis=-1, keepdims=True)
    return t1, np.cross(normal, t1)


def clustered_reset_state(rng: np.random.Generator, n_rows: int, n_cars: int,
                          radius: float = 500.0) -> dict[str, np.ndarray]:
    """apply_reset_state inputs for clustered scenes at the arena's surfaces:
    each simulation's ball sits 93-400 uu off one flat surface (the floor 40%
    of the time, a side wall, a back wall beside the goal or the ceiling 20%
    each) and every car lies within `radius` uu of the ball: half of them
    standing on that surface (wheels on it, resting 17 uu off it, random
    heading along it), the others in the air on the ball's side of the
    surface with random orientations.  Velocities point toward the ball on
    average (surface cars along the surface).  Dense car-car and car-ball
    contacts and wheel hits on walls and the ceiling on every tick."""
    kind, spot, normal = _surface_spots(rng, n_rows)
    t1, t2 = _tangent_basis(normal)
    height = rng.uniform(93.0, 400.0, n_rows)
    ball_pos = spot + normal * height[:, None]
    # cars on the surface: a disk around the spot narrow enough for the car to
    # stay within `radius` of the ball
    reach = np.sqrt(np.maximum(radius ** 2 - (height - 17.0) ** 2, 0.0)) - 1.0
    r = reach[:, None] * np.sqrt(rng.uniform(0, 1, (n_rows, n_cars)))
    a = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
    on_surface = spot[:, None, :] + normal[:, None, :] * 17.0 +         (r * np.cos(a))[..., None] * t1[:, None, :] + (r * np.sin(a))[..., None] * t2[:, None, :]
    # cars in the air: the half ball of `radius` around the ball away from the surface
    d = rng.normal(size=(n_rows, n_cars, 3))
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    away = np.einsum("rkc,rc->rk", d, normal)
    d = d - 2.0 * np.minimum(away, 0.0)[..., None] * normal[:, None, :]
    in_air = ball_pos[:, None, :] + d * (radius * np.cbrt(rng.uniform(0.1, 1.0, (n_rows, n_cars))) - 1.0)[..., None]
    standing = rng.uniform(0, 1, (n_rows, n_cars)) < 0.5
    car_pos = np.where(standing[..., None], on_surface, in_air)
    # orientations: roof along the surface normal with a random heading, or random
    h = rng.uniform(-np.pi, np.pi, (n_rows, n_cars))
    fwd = np.cos(h)[..., None] * t1[:, None, :] + np.sin(h)[..., None] * t2[:, None, :]
    up = np.broadcast_to(normal[:, None, :], fwd.shape)
    rot_surface = _quat_from_axes(fwd, up)
    rot_air = rng.normal(size=(n_rows, n_cars, 4))
    rot_air /= np.linalg.norm(rot_air, axis=-1, keepdims=True)
    rot = np.where(standing[..., None], rot_surface, rot_air)
    to_ball = ball_pos[:, None, :] - car_pos
    to_ball /= np.maximum(np.linalg.norm(to_ball, axis=-1, keepdims=True), 1.0)
    car_vel = to_ball * rng.uniform(0, 1400, (n_rows, n_cars, 1)) + rng.normal(size=(n_rows, n_cars, 3)) * 300.0
    along = car_vel - np.einsum("rkc,rc->rk", car_vel, normal)[..., None] * normal[:, None, :]
    car_vel = np.where(standing[..., None], along, car_vel)
    ball_vel = _unit_vectors(rng, n_rows) * rng.uniform(0, 1500, (n_rows, 1))
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    return {
        "ball_position": f32(ball_pos),
        "ball_velocity": f32(ball_vel),
        "ball_angular_velocity": f32(_unit_vectors(rng, n_rows) * rng.uniform(0, 6, (n_rows, 1))),
        "car_position": f32(car_pos),
        "car_rotation": f32(rot),
        "car_velocity": f32(car_vel),
        "car_angular_velocity": f32(rng.normal(size=(n_rows, n_cars, 3)) * 0.5),
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
