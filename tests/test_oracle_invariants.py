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


# ---------------------------------------------------------------- SAT by linear programming

HALF = np.array([60.186455, 43.282655, 19.262505])


def _lp_margin(A_ub, b_ub, A_eq=None, b_eq=None, n_free=0, n_pos=0):
    """max s subject to A_ub [x, s] <= b_ub (x: n_free free then n_pos >= 0)."""
    from scipy.optimize import linprog

    n = n_free + n_pos + 1
    c = np.zeros(n)
    c[-1] = -1.0
    bounds = [(None, None)] * n_free + [(0, None)] * n_pos + [(None, None)]
    r = linprog(c, A_ub=A_ub, b_ub=b_ub, A_eq=A_eq, b_eq=b_eq, bounds=bounds, method="highs")
    assert r.status == 0
    return -r.fun


def box_tri_margin(tri):
    """Largest s with a point of the triangle inside the box shrunk by s (s < 0: disjoint)."""
    A, b = [], []
    for k in range(3):
        for sgn in (1.0, -1.0):
            A.append([sgn * tri[i][k] for i in range(3)] + [1.0])
            b.append(HALF[k])
    return _lp_margin(np.array(A), np.array(b), A_eq=np.array([[1.0, 1.0, 1.0, 0.0]]), b_eq=[1.0], n_pos=3)


def _rot(q):
    x, y, z, w = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def box_box_margin(ca, qa, cb, qb):
    A, b = [], []
    for c, q in ((ca, qa), (cb, qb)):
        R = _rot(q)
        for k in range(3):
            for sgn in (1.0, -1.0):
                A.append(list(sgn * R[:, k]) + [1.0])
                b.append(HALF[k] + sgn * R[:, k] @ c)
    return _lp_margin(np.array(A), np.array(b), n_free=3)


def test_box_triangle_sat_agrees_with_linear_programming():
    """The 13-axis SAT verdict equals the LP feasibility of a common point, and
    moving the triangle by the reported depth along the reported axis (one of
    its two senses) separates the pair."""
    rng = np.random.default_rng(5)
    ov, ax, dp = C.c_int(), C.c_int(), F()
    axis = (F * 3)()
    checked = hits = 0
    for _ in range(600):
        centre = rng.normal(size=3) * np.array([70.0, 50.0, 30.0])
        tri = (centre + rng.normal(size=(3, 3)) * rng.uniform(5, 120)).astype(np.float32)
        margin = box_tri_margin(tri.astype(np.float64))
        if abs(margin) < 0.05:
            continue                      # too close to touching to call in float32
        lib().oracle_probe_box_tri_sat((F * 9)(*tri.reshape(-1)), C.byref(ov), C.byref(ax), C.byref(dp), axis)
        checked += 1
        assert bool(ov.value) == (margin > 0), (tri, margin)
        if ov.value:
            hits += 1
            a = np.array(list(axis), np.float64)
            assert 0 <= ax.value < 13 and dp.value >= 0 and abs(np.linalg.norm(a) - 1) < 1e-5
            moved = [box_tri_margin(tri + s * (dp.value + 0.05) * a) for s in (1.0, -1.0)]
            assert min(moved) < 0, (tri, dp.value, a, moved)
    assert checked > 400 and hits > 50


def test_box_box_sat_agrees_with_linear_programming():
    rng = np.random.default_rng(6)
    ov, ax, dp = C.c_int(), C.c_int(), F()
    checked = hits = 0
    for _ in range(400):
        qa, qb = rng.normal(size=4), rng.normal(size=4)
        qa /= np.linalg.norm(qa)
        qb /= np.linalg.norm(qb)
        ca = rng.uniform(-1000, 1000, 3)
        cb = ca + rng.normal(size=3) * 80.0
        qa32, qb32 = qa.astype(np.float32), qb.astype(np.float32)
        ca32, cb32 = ca.astype(np.float32), cb.astype(np.float32)
        margin = box_box_margin(ca32.astype(np.float64), qa32.astype(np.float64) / np.linalg.norm(qa32),
                                cb32.astype(np.float64), qb32.astype(np.float64) / np.linalg.norm(qb32))
        if abs(margin) < 0.05:
            continue
        lib().oracle_probe_box_box_sat((F * 3)(*ca32), (F * 4)(*qa32), (F * 3)(*cb32), (F * 4)(*qb32), C.byref(ov),
                                       C.byref(ax), C.byref(dp))
        checked += 1
        assert bool(ov.value) == (margin > 0), (ca, qa, cb, qb, margin)
        hits += ov.value
        if ov.value:
            assert 0 <= ax.value < 15 and dp.value >= 0
    assert checked > 300 and hits > 50


# ---------------------------------------------------------------- suspension rays by brute force

ANCHORS = np.array([[37.3743, 25.9, 0.0], [37.3743, -25.9, 0.0], [-47.6257, 29.5, 0.0], [-47.6257, -29.5, 0.0]])
RAY_LEN = np.array([26.755 + 12 + 12.5 - 2.5] * 2 + [25.055 + 12 + 15 - 2.5] * 2)
HITBOX_OFFSET = np.array([13.87566, 0.0, 20.755])


def _nearest_hit(start, d, tv):
    """Nearest ray-triangle hit over the whole mesh in float64 (ray-plane
    intersection, then an inside test by barycentric signs)."""
    a, b, c = tv[:, 0], tv[:, 1], tv[:, 2]
    n = np.cross(b - a, c - a)
    den = n @ d
    ok = np.abs(den) > 1e-9
    t = np.where(ok, ((a - start) * n).sum(1) / np.where(ok, den, 1.0), np.inf)
    p = start + t[:, None] * d
    inside = ((np.cross(b - a, p - a) * n).sum(1) >= 0) & ((np.cross(c - b, p - b) * n).sum(1) >= 0) & \
             ((np.cross(a - c, p - c) * n).sum(1) >= 0)
    t = np.where(ok & inside & (t > 0), t, np.inf)
    i = int(np.argmin(t))
    return t[i], n[i] / np.linalg.norm(n[i])


def test_suspension_rays_match_brute_force_over_the_mesh(arena):
    """Each wheel's hit distance and normal equal the nearest hit over all
    triangles (the cell run holds every triangle a ray can reach), for cars
    over the floor, ramps and walls."""
    verts, tris, _, _, _ = arena
    tv = verts[tris].astype(np.float64)
    rng = np.random.default_rng(9)
    n = 128
    env = OracleEnv(n, 1, 0, 0)
    pos = np.stack([rng.uniform(-4000, 4000, n), rng.uniform(-5000, 5000, n), rng.uniform(5, 45, n)], 1)
    tilt = rng.normal(size=(n, 3)) * 0.3
    ang = np.linalg.norm(tilt, axis=1, keepdims=True)
    q = np.concatenate([tilt / ang * np.sin(ang / 2), np.cos(ang / 2)], 1)
    env.set_car(pos[:, None].astype(np.float32), q[:, None].astype(np.float32), np.zeros((n, 1, 3), np.float32),
                np.zeros((n, 1, 3), np.float32), np.zeros((n, 1), np.bool_))
    car, _, _ = env.export_state()
    dist, normal, source = env.raycast()
    hits = 0
    for i in range(n):
        cen = f32(car[CAR["CARL_CAR_CEN_0"]:CAR["CARL_CAR_CEN_0"] + 3, i])
        qq = f32(car[CAR["CARL_CAR_ROT_0"]:CAR["CARL_CAR_ROT_0"] + 4, i])
        R = _rot(qq / np.linalg.norm(qq))
        d = -R[:, 2]
        for k in range(4):
            t, nrm = _nearest_hit(cen + R @ ANCHORS[k], d, tv)
            if t <= RAY_LEN[k] + 1.0 - 1e-3:
                hits += 1
                assert source[i, k] == 1, (i, k, t)
                assert abs(dist[i, k] - t) < 2e-3, (i, k, dist[i, k], t)
                nrm = -nrm if nrm @ d > 0 else nrm
                assert np.abs(normal[i, k] - nrm).max() < 1e-5
            elif t > RAY_LEN[k] + 1.0 + 1e-3:
                assert source[i, k] == 0, (i, k, t)
    assert hits > 150
    env.close()


def test_one_ulp_grows_past_the_long_run_tolerance():
    """The trajectories are chaotic: 32 1v1 simulations from random states,
    run twice for 1,000 ticks on the same actions, the second time with one
    car's starting x velocity moved by one ulp, end more than 1 uu apart -
    past a tolerance of 1e-3 uu over 1,000 ticks by three orders of
    magnitude.  A comparison of the engine with the oracle at that tolerance
    could only pass bit for bit, which is the bar the GPU parity tests hold."""
    from carl_amd import workloads

    rng = np.random.default_rng(10)
    n = 32
    reset = workloads.random_reset_state(rng, n, 2)
    actions = [workloads.random_continuous_actions(rng, n, 2) for _ in range(125)]

    def run(perturb):
        env = OracleEnv(n, 1, 1, 17, 8)
        state = {k: v.copy() for k, v in reset.items()}
        if perturb:
            v = state["car_velocity"]
            v[:, 0, 0] = np.nextafter(v[:, 0, 0], np.float32(np.inf))
        env.apply_reset_state(**state)
        for a in actions:
            env.step(a)
        pos = env.export_state()[0][CAR_NAMES.index("CARL_CAR_POS_0"):][:3].view(np.float32).copy()
        env.close()
        return pos

    drift = np.abs(run(False).astype(np.float64) - run(True)).max()
    assert drift > 1.0, drift

