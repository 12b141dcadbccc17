"""Wheel rays at bodies near the end of their reach, engine against oracle.

The engine does not cast a car's wheel rays at another car or at the ball
whose centre lies beyond the rays' reach plus that body's bounding radius
(car_phase.h: kCarRayReach, 189.7 uu, and kBallRayReach, 200.9 uu), since
every such ray would miss; the oracle casts every ray.  Here each simulation
puts the other car, or the ball, where one wheel ray just reaches it, a
little before the ray's end: a corner of the other car's box, turned so that
the box lies beyond it as seen from the car's centre (the farthest a hit
car can be: about 150 uu between the centres), or the ball straight below
the ray's end.  A reach bound that cut off a hitting ray would show here as
a state that differs from the oracle's.  The engine's state after one tick
must equal the oracle's bit for bit, and most of these rays must hit.
"""
import math

import numpy as np
import pytest

from abi import CAR_NAMES
from carl_amd import workloads
from gpu_harness import Pair, dev

pytestmark = pytest.mark.gpu

CAR = {n: i for i, n in enumerate(CAR_NAMES)}
DIRECT = 2
SRC_CAR, SRC_BALL = 2, 3

# car geometry (constants.h): hitbox half extents and offset, wheel anchors
# relative to the hitbox centre, ray lengths (rest + travel + radius - 2.5)
HALF = np.array([60.186455, 43.282655, 19.262505])
OFFSET = np.array([13.87566, 0.0, 20.755])
ANCHORS = [np.array([37.3743, 25.9, 0.0]), np.array([37.3743, -25.9, 0.0]),
           np.array([-47.6257, 29.5, 0.0]), np.array([-47.6257, -29.5, 0.0])]
RAYS = [26.755 + 12.0 + 12.5 - 2.5] * 2 + [25.055 + 12.0 + 15.0 - 2.5] * 2
BALL_R = 91.25


def _rot(q):
    x, y, z, w = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _random_quat(rng, tilt):
    """A random heading with a random tilt of up to `tilt` radians."""
    yaw = rng.uniform(-math.pi, math.pi)
    ax = rng.normal(size=3)
    ax[2] = 0.0
    ax /= np.linalg.norm(ax)
    a = rng.uniform(0, tilt)
    qy = np.array([0.0, 0.0, math.sin(yaw / 2), math.cos(yaw / 2)])
    qt = np.array([*(ax * math.sin(a / 2)), math.cos(a / 2)])
    x1, y1, z1, w1 = qt
    x2, y2, z2, w2 = qy
    return np.array([w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2, w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2,
                     w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2, w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2])


def _align(a, b, spin):
    """A rotation taking unit vector a to unit vector b, then turning by
    `spin` about b."""
    v = np.cross(a, b)
    c = float(np.dot(a, b))
    vx = np.array([[0, -v[2], v[1]], [v[2], 0, -v[0]], [-v[1], v[0], 0]])
    r = np.eye(3) + vx + vx @ vx / (1.0 + c)
    bx = np.array([[0, -b[2], b[1]], [b[2], 0, -b[0]], [-b[1], b[0], 0]])
    spin_r = np.eye(3) + math.sin(spin) * bx + (1 - math.cos(spin)) * bx @ bx
    return spin_r @ r


def _quat_of(m):
    """(x, y, z, w) of a rotation matrix."""
    w = math.sqrt(max(0.0, 1.0 + m[0, 0] + m[1, 1] + m[2, 2])) / 2
    x = math.copysign(math.sqrt(max(0.0, 1.0 + m[0, 0] - m[1, 1] - m[2, 2])) / 2, m[2, 1] - m[1, 2])
    y = math.copysign(math.sqrt(max(0.0, 1.0 - m[0, 0] + m[1, 1] - m[2, 2])) / 2, m[0, 2] - m[2, 0])
    z = math.copysign(math.sqrt(max(0.0, 1.0 - m[0, 0] - m[1, 1] + m[2, 2])) / 2, m[1, 0] - m[0, 1])
    q = np.array([x, y, z, w])
    return q / np.linalg.norm(q)


@pytest.mark.parametrize("body", ["car", "ball"])
def test_bodies_at_the_end_of_the_wheel_rays(gpu, body):
    n = 256
    rng = np.random.default_rng(11 if body == "car" else 12)
    p = Pair(n, 1, 1, seed=4, frameskip=1)
    pos = np.zeros((n, 2, 3))
    rot = np.zeros((n, 2, 4))
    ball = np.zeros((n, 3))
    reach = np.zeros(n)
    for i in range(n):
        qa = _random_quat(rng, 0.6)
        ra = _rot(qa)
        cen_a = np.array([rng.uniform(-2000, 2000), rng.uniform(-3000, 3000), rng.uniform(700, 1300)])
        k = rng.integers(0, 4)
        start = cen_a + ra @ ANCHORS[k]
        down = -ra[:, 2]
        t = RAYS[k] * rng.uniform(0.95, 0.995)
        hit = start + down * t
        away = cen_a + np.array([-math.copysign(1500.0, cen_a[0]), 0.0, 0.0])
        if body == "car":
            # the box's corner nearest the car at the hit point, the box beyond it
            u = (hit - cen_a) / np.linalg.norm(hit - cen_a)
            corner = HALF * rng.choice([-1.0, 1.0], size=3)
            rb = _align(corner / np.linalg.norm(corner), -u, rng.uniform(-math.pi, math.pi))
            qb = _quat_of(rb)
            cen_b = hit - rb @ (corner * 0.999)
            ball[i] = away
        else:
            qb = np.array([0.0, 0.0, 0.0, 1.0])
            cen_b = away
            ball[i] = hit + down * (BALL_R * 0.999)
        reach[i] = np.linalg.norm((cen_b if body == "car" else ball[i]) - cen_a)
        pos[i, 0] = cen_a - ra @ OFFSET
        rot[i, 0] = qa
        pos[i, 1] = cen_b - _rot(qb) @ OFFSET
        rot[i, 1] = qb
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    zero = np.zeros((n, 2, 3), np.float32)
    demoed = np.zeros((n, 2), np.bool_)
    p.gpu.set_car(dev(f32(pos)), dev(f32(rot)), dev(zero), dev(zero), dev(demoed))
    p.cpu.set_car(f32(pos), f32(rot), zero, zero, demoed)
    zb = np.zeros((n, 3), np.float32)
    p.gpu.set_ball(dev(f32(ball)), dev(zb), dev(zb))
    p.cpu.set_ball(f32(ball), zb, zb)
    p.tick(np.zeros(2 * n, dtype=workloads.CONTROLS_DTYPE), DIRECT, 1)
    report = p.state_mismatches()
    assert not report, "\n  ".join(report)
    car, _, _ = p.cpu.export_state()
    src = np.stack([car[CAR[f"CARL_CAR_WHEEL_SOURCE_{k}"], 0::2].view(np.int32) for k in range(4)])
    hits = (src == (SRC_CAR if body == "car" else SRC_BALL)).any(axis=0)
    assert hits.mean() > 0.5, f"only {hits.mean():.0%} of the placed {body}s were hit"
    assert reach[hits].max() > 145.0, reach[hits].max()
    p.close()
