"""Autoroll from the chassis manifold on the engine, against the oracle.

A car with no wheel on the ground but with the arena manifold of the tick
before (a car lying on its side or roof) takes its autoroll direction from
that manifold's normal, and past a quarter roll its roll factor saturates
(the oracle's pin: tests/test_oracle_control_pins.py,
test_autoroll_from_the_chassis_manifold_saturates_past_a_quarter_roll).
Random play reaches this branch only now and then; here 192 cars, rolled and
pitched over the whole circle and carrying that manifold, tick with random
throttle (and without), and the engine's state must equal the oracle's bit
for bit.
"""
import math

import numpy as np
import pytest

from abi import CAR_NAMES
from carl_amd import workloads
from gpu_harness import Pair

pytestmark = pytest.mark.gpu

CAR = {n: i for i, n in enumerate(CAR_NAMES)}
DIRECT = 2


def _quat(axis, angle):
    axis = np.asarray(axis, float) / np.linalg.norm(axis)
    s = math.sin(angle / 2)
    return np.array([axis[0] * s, axis[1] * s, axis[2] * s, math.cos(angle / 2)])


def _mul(a, b):
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return np.array([aw * bx + ax * bw + ay * bz - az * by, aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw, aw * bw - ax * bx - ay * by - az * bz])


@pytest.mark.parametrize("throttle_held", [True, False])
def test_chassis_manifold_autoroll_matches_the_oracle(gpu, throttle_held):
    n = 192
    rng = np.random.default_rng(71 if throttle_held else 72)
    p = Pair(n, 1, 0, seed=5, frameskip=1)
    roll = np.linspace(-math.pi, math.pi, n, endpoint=False) + 0.01
    pitch = rng.uniform(-0.6, 0.6, n)
    yaw = rng.uniform(-math.pi, math.pi, n)
    rot = np.stack([_mul(_quat((0, 0, 1), yaw[i]), _mul(_quat((0, 1, 0), pitch[i]), _quat((1, 0, 0), roll[i])))
                    for i in range(n)]).astype(np.float32)
    pos = np.stack([rng.uniform(-2500, 2500, n), rng.uniform(-3500, 3500, n), rng.uniform(400, 1200, n)], axis=1)
    p.cpu.set_car(pos.astype(np.float32).reshape(n, 1, 3), rot.reshape(n, 1, 4),
                  np.zeros((n, 1, 3), np.float32), np.zeros((n, 1, 3), np.float32), np.zeros((n, 1), np.bool_))
    car, sim, tick = p.cpu.export_state()
    # the manifold a car lying on the floor (or, for some, on a wall) leaves
    normals = np.zeros((n, 3), np.float32)
    normals[:, 2] = 1.0
    wall = rng.uniform(0, 1, n) < 0.25
    normals[wall] = np.array([1.0, 0.0, 0.0], np.float32)
    car[CAR["CARL_CAR_MANIFOLD_COUNT"]] = rng.integers(1, 5, n).astype(np.uint32)
    for k in range(3):
        car[CAR[f"CARL_CAR_MANIFOLD_NORMAL_{k}"]] = normals[:, k].view(np.uint32)
    p.import_state(car, sim, tick)
    for t in range(4):
        c = np.zeros(n, dtype=workloads.CONTROLS_DTYPE)
        if throttle_held:
            c["throttle"] = rng.uniform(-1, 1, n)
        c["steer"] = rng.uniform(-1, 1, n)
        p.tick(c, DIRECT, 1)
        report = p.state_mismatches()
        assert not report, f"tick {t}:\n  " + "\n  ".join(report)
    p.close()
