"""The contact search's screening stage changes no result.

The screen drops (car, cell triangle) pairs whose float ray and SAT tests are
proven to reject them (bounds from the rounding analysis of those tests).
These tests run two engines on identical inputs, one with the screen and one
without (CARL_PARAM_CONTACT_SCREEN = 0 runs every test on every pair), and
require every field of the persistent state to agree bit for bit, at sizes the
oracle cannot reach, on poses chosen to sit at the edges of the bounds: rays
grazing walls, floor and ceiling, wheel hubs on wall planes, cars on their
sides and upside down, with axis-exact and slightly perturbed rotations.
"""
import numpy as np
import pytest

import carl_amd
from carl_amd import workloads
from gpu_harness import dense_geometry_reset_state, describe_mismatch, dev, gpu_state
from abi import CAR_NAMES, SIM_NAMES

pytestmark = pytest.mark.gpu


def _quat(axis, angle):
    axis = np.asarray(axis, dtype=np.float64)
    axis = axis / np.linalg.norm(axis)
    return np.concatenate([axis * np.sin(angle / 2), [np.cos(angle / 2)]])


def _qmul(a, b):
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return np.array([aw * bx + ax * bw + ay * bz - az * by, aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw, aw * bw - ax * bx - ay * by - az * bz])


def edge_on_reset_state(rng: np.random.Generator, n_rows: int, n_cars: int) -> dict[str, np.ndarray]:
    """Cars whose suspension rays run along a surface or whose wheel hubs sit
    on (or within a hair of) a wall plane."""
    orient = [_quat([0, 0, 1], k * np.pi / 2) for k in range(4)]                      # upright, axis-exact yaw
    orient += [_qmul(_quat([0, 0, 1], k * np.pi / 2), _quat([1, 0, 0], s * np.pi / 2))  # on its side
               for k in range(4) for s in (-1, 1)]
    orient += [_qmul(_quat([0, 0, 1], k * np.pi / 2), _quat([0, 1, 0], s * np.pi / 2))  # nose up / down
               for k in range(4) for s in (-1, 1)]
    orient += [_quat([1, 0, 0], np.pi)]                                                 # upside down
    orient = np.array(orient)
    offsets = np.array([0.0, 1e-3, 0.05, 1.0, 17.0, 25.9, 29.5, 43.3, 60.2, 100.0])
    pos = np.empty((n_rows, n_cars, 3))
    rot = np.empty((n_rows, n_cars, 4))
    for r in range(n_rows):
        for c in range(n_cars):
            off = offsets[rng.integers(len(offsets))] + (rng.uniform(-1e-3, 1e-3) if rng.uniform() < 0.5 else 0.0)
            surf = rng.integers(5)
            p = np.array([rng.uniform(-3800, 3800), rng.uniform(-4800, 4800), rng.uniform(40, 1900)])
            if surf == 0:
                p[0] = np.sign(rng.uniform(-1, 1)) * (4096.0 - off)       # side wall
            elif surf == 1:
                p[1] = np.sign(rng.uniform(-1, 1)) * (5120.0 - off)       # back wall
                p[0] = rng.uniform(-3000, 3000)
            elif surf == 2:
                p[2] = 2044.0 - off                                       # ceiling
            elif surf == 3:
                p[2] = off                                                # floor
            else:
                p = np.array([rng.uniform(-4000, 4000), rng.uniform(-5000, 5000), rng.uniform(0, 2000)])
            q = orient[rng.integers(len(orient))].copy()
            if rng.uniform() < 0.5:
                q += rng.normal(size=4) * 10.0 ** rng.uniform(-7, -3)
                q /= np.linalg.norm(q)
            pos[r, c], rot[r, c] = p, q
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    return {
        "ball_position": f32(np.stack([rng.uniform(-3000, 3000, n_rows), rng.uniform(-4000, 4000, n_rows),
                                       rng.uniform(100, 1800, n_rows)], 1)),
        "ball_velocity": f32(rng.normal(size=(n_rows, 3)) * 600.0),
        "ball_angular_velocity": f32(rng.normal(size=(n_rows, 3))),
        "car_position": f32(pos), "car_rotation": f32(rot),
        "car_velocity": f32(rng.normal(size=(n_rows, n_cars, 3)) * 400.0),
        "car_angular_velocity": f32(rng.normal(size=(n_rows, n_cars, 3)) * 0.5),
        "car_demoed": np.zeros((n_rows, n_cars), dtype=np.bool_),
        "car_boost": f32(rng.uniform(0, 100, (n_rows, n_cars))),
    }


def _run_both(n, n_blue, frameskip, steps, make_state, seed):
    rng = np.random.default_rng(seed)
    nc = 2 * n_blue
    screened = carl_amd.Env(n, n_blue, n_blue, 5, frameskip, True, False, False)
    full = carl_amd.Env(n, n_blue, n_blue, 5, frameskip, True, False, False)
    assert screened.contact_screen == 1
    full.contact_screen = 0
    assert full.contact_screen == 0
    state = {k: dev(v) for k, v in make_state(rng, n, nc).items()}
    for env in (screened, full):
        env.apply_reset_state(**state)
    for step in range(steps):
        actions = dev(workloads.random_continuous_actions(rng, n, nc))
        screened.step_continuous(actions)
        full.step_continuous(actions)
        a, b = gpu_state(screened), gpu_state(full)
        report = describe_mismatch(CAR_NAMES, a[0], b[0]) + describe_mismatch(SIM_NAMES, a[1], b[1])
        if report:
            pytest.fail(f"screened vs unscreened after step {step}:\n  " + "\n  ".join(report))


def test_screen_random_states_1v1(gpu):
    _run_both(8192, 1, 8, 40, workloads.random_reset_state, seed=31)


def test_screen_dense_geometry_1v1_and_3v3(gpu):
    _run_both(4096, 1, 4, 30, dense_geometry_reset_state, seed=32)
    _run_both(1024, 3, 4, 20, dense_geometry_reset_state, seed=33)


def test_screen_edge_on_poses(gpu):
    _run_both(4096, 1, 1, 40, edge_on_reset_state, seed=34)
