"""The CPU oracle against what mathematics and the mesh fix, independent of
its own formulas: closed forms of free flight and boost use, equilibria,
restitution, sign of the drive, arena indexing by brute force, and the
accuracy of its own sin/cos/atan2 against double-precision libm.  Each check
is chosen so that a plausible slip (a dropped gravity or drag term, a wrong
sign, a transposed index) fails it."""
import ctypes as C
import math

import numpy as np
import pytest

from abi import CAR_NAMES, SIM_NAMES
from oracle_py import OracleEnv, cell_of, lib

CAR = {n: i for i, n in enumerate(CAR_NAMES)}
SIM = {n: i for i, n in enumerate(SIM_NAMES)}
DT = 1.0 / 120.0
F = C.c_float


def f32(u):
    return np.asarray(u, np.uint32).view(np.float32).astype(np.float64)


def car_vec(car, name, c):
    i = CAR[name + "_0"]
    return f32(car[i:i + 3, c])


def sim_vec(sim, name, s):
    i = SIM[name + "_0"]
    return f32(sim[i:i + 3, s])


# continuous action slots per car (python/carl.cu layout): steer/yaw, pitch,
# throttle, powerslide, boost, air roll, jump
THROTTLE, BOOST = 2, 4


# ---------------------------------------------------------------- ball free flight

def test_ball_free_flight_matches_closed_form():
    """No contacts: v_n = d^n v0 + a (1 - d^n)/(1 - d), p_n = p0 + dt sum v_k,
    with per-tick drag d = 0.97^(1/120) and a = g dt (g = -650 uu/s^2)."""
    env = OracleEnv(1, 1, 1, 0)
    p0 = np.array([100.0, -200.0, 1200.0])
    v0 = np.array([300.0, 150.0, 400.0])
    env.set_ball(p0[None].astype(np.float32), v0[None].astype(np.float32), np.zeros((1, 3), np.float32))
    n = 60
    env.tick(np.zeros((1, 2, 7), np.float32), 1, n)
    _, sim, _ = env.export_state()
    d = 0.97 ** (1.0 / 120.0)
    a = np.array([0.0, 0.0, -650.0 * DT])
    geo = (1 - d ** n) / (1 - d)                     # sum_{k=0}^{n-1} d^k
    v_n = d ** n * v0 + a * geo
    sum_v = v0 * d * geo + a * (n - d * geo) / (1 - d)  # sum_{k=1}^{n} v_k
    p_n = p0 + DT * sum_v
    np.testing.assert_allclose(sim_vec(sim, "CARL_SIM_BALL_VEL", 0), v_n, rtol=2e-5, atol=2e-3)
    np.testing.assert_allclose(sim_vec(sim, "CARL_SIM_BALL_POS", 0), p_n, rtol=2e-5, atol=2e-3)
    env.close()


def test_ball_floor_bounce_restitution():
    """A ball dropped on the floor leaves with about 0.6 of its impact speed."""
    env = OracleEnv(1, 1, 1, 0)
    env.set_ball(np.array([[0.0, 0.0, 400.0]], np.float32), np.array([[0.0, 0.0, -1.0]], np.float32),
                 np.zeros((1, 3), np.float32))
    vz = []
    for _ in range(200):
        env.tick(np.zeros((1, 2, 7), np.float32), 1, 1)
        _, sim, _ = env.export_state()
        vz.append(sim_vec(sim, "CARL_SIM_BALL_VEL", 0)[2])
    vz = np.array(vz)
    k = int(np.argmax(vz > 0))          # first tick moving up
    assert k > 0
    ratio = vz[k] / -vz[k - 1]
    assert 0.5 < ratio < 0.7, ratio
    env.close()


# ---------------------------------------------------------------- car dynamics

def test_car_at_rest_stays_at_rest():
    """Suspension balances gravity: a kickoff car with no input keeps z and speed."""
    env = OracleEnv(4, 1, 1, 0)
    env.tick(np.zeros((4, 2, 7), np.float32), 1, 240)
    car, _, _ = env.export_state()
    for c in range(8):
        assert abs(car_vec(car, "CARL_CAR_POS", c)[2] - 17.0) < 1.0
        assert np.linalg.norm(car_vec(car, "CARL_CAR_VEL", c)) < 1.0
    env.close()


@pytest.mark.parametrize("throttle", [1.0, -1.0])
def test_throttle_drives_along_the_car_axis(throttle):
    env = OracleEnv(1, 1, 0, 0)
    car, _, _ = env.export_state()
    q = f32(car[CAR["CARL_CAR_ROT_0"]:CAR["CARL_CAR_ROT_0"] + 4, 0])
    x, y, z, w = q
    fwd = np.array([1 - 2 * (y * y + z * z), 2 * (x * y + w * z), 2 * (x * z - w * y)])
    a = np.zeros((1, 1, 7), np.float32)
    a[..., THROTTLE] = throttle
    speeds = []
    for _ in range(3):
        env.tick(a, 1, 20)
        car, _, _ = env.export_state()
        speeds.append(float(car_vec(car, "CARL_CAR_VEL", 0) @ fwd))
    assert all(np.sign(s) == np.sign(throttle) for s in speeds)
    assert abs(speeds[0]) < abs(speeds[1]) < abs(speeds[2])
    env.close()


def test_boost_drains_at_a_third_per_second():
    """Boost held for 0.5 s drains 100/3 per second (1/120 s per tick); the car
    starts clear of every pad so none refills it."""
    env = OracleEnv(1, 1, 0, 0)
    env.set_car(np.array([[[500.0, 500.0, 17.0]]], np.float32), np.array([[[0.0, 0.0, 0.0, 1.0]]], np.float32),
                np.zeros((1, 1, 3), np.float32), np.zeros((1, 1, 3), np.float32), np.zeros((1, 1), np.bool_),
                boost=np.array([[50.0]], np.float32))
    a = np.zeros((1, 1, 7), np.float32)
    a[..., BOOST] = 1.0
    car, _, _ = env.export_state()
    b0 = float(f32(car[CAR["CARL_CAR_BOOST"], 0]))
    assert b0 == 50.0
    env.tick(a, 1, 60)
    car, _, _ = env.export_state()
    b1 = float(f32(car[CAR["CARL_CAR_BOOST"], 0]))
    assert abs((b0 - b1) - 60 * (100.0 / 3.0) * DT) < 1e-3
    env.close()


# ---------------------------------------------------------------- arena mesh

@pytest.fixture(scope="module")
def arena():
    env = OracleEnv(1, 1, 1, 0)
    out = env.arena()
    env.close()
    return out


def test_arena_grid_registration_by_brute_force(arena):
    """Every triangle is listed, once and in ascending order, in exactly the
    cells [cell(min) - 1, cell(max)] per axis (clamped at 0)."""
    verts, tris, _, prefix, cell_tris = arena
    tv = verts[tris]
    lo, hi = tv.min(1), tv.max(1)
    expect = {}
    for t in range(len(tris)):
        a = cell_of(*lo[t])
        b = cell_of(*hi[t])
        a = [max(v - 1, 0) for v in a]
        for z in range(a[2], b[2] + 1):
            for y in range(a[1], b[1] + 1):
                for x in range(a[0], b[0] + 1):
                    expect.setdefault(x + 48 * y + 48 * 48 * z, []).append(t)
    for c in range(len(prefix) - 1):
        got = list(cell_tris[prefix[c]:prefix[c + 1]])
        assert got == expect.get(c, []), c


def test_arena_mesh_is_welded_and_closed_where_shared(arena):
    verts, tris, angles, _, _ = arena
    assert len(np.unique(verts, axis=0)) == len(verts)
    e = np.sort(np.stack([tris[:, [0, 1]], tris[:, [1, 2]], tris[:, [2, 0]]], 1).reshape(-1, 2), 1)
    _, counts = np.unique(e, axis=0, return_counts=True)
    assert counts.max() <= 2
    boundary = angles.reshape(-1) == np.float32(2 * math.pi)
    assert boundary.sum() == (counts == 1).sum()
    assert np.all(np.abs(angles.reshape(-1)[~boundary]) <= math.pi)


# ---------------------------------------------------------------- own math

def test_sincos_accuracy():
    s, c = F(), F()
    xs = np.concatenate([np.linspace(-100, 100, 20001), [0.0, -0.0, 1e-8, math.pi, -math.pi, 3 * math.pi / 2]])
    for x in xs.astype(np.float32):
        lib().oracle_sincos(float(x), C.byref(s), C.byref(c))
        assert abs(s.value - math.sin(float(x))) <= 3e-7
        assert abs(c.value - math.cos(float(x))) <= 3e-7


def test_atan2_accuracy_and_quadrants():
    lib().oracle_atan2.restype = F
    rng = np.random.default_rng(0)
    pts = rng.normal(size=(20000, 2)).astype(np.float32)
    pts = np.concatenate([pts, [[0, 1], [0, -1], [1, 0], [-1, 0], [1e-30, -1], [-1e-30, -1]]]).astype(np.float32)
    for y, x in pts:
        got = lib().oracle_atan2(float(y), float(x))
        assert abs(got - math.atan2(float(y), float(x))) <= 4e-7, (y, x)


def test_quaternion_integration_keeps_unit_norm():
    out = (F * 4)()
    rng = np.random.default_rng(1)
    for _ in range(200):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        w = rng.normal(size=3) * 5
        lib().oracle_integrate_quat((F * 4)(*q), (F * 3)(*w), out)
        r = np.array(list(out))
        assert abs(np.linalg.norm(r) - 1.0) < 1e-6
        # small rotation: the result is close to q rotated by |w| dt
        assert abs(abs(float(r @ q)) - math.cos(np.linalg.norm(w) * DT / 2)) < 1e-5
