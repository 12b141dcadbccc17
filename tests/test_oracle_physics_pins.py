"""The CPU oracle's contact responses and forces against what physics and the
published curves fix, each isolated from the rest of the tick:

  car-car solve   linear and angular momentum of an airborne pair are
                  conserved; a symmetric side impact separates at the
                  car-car restitution (CARCAR_COLLISION_RESTITUTION = 0.1,
                  include/RLConstants.cuh:201-202)
  bump            the victim's velocity with the bump minus without it (the
                  bumper's cooldown switches it off) equals the published
                  ground / air / upward curves at the closing speed
                  (include/Physics/CarCar/Response.cuh:8-57)
  demolition      supersonic (>= 2200 uu/s) opposite-team hits with >= 5 uu
                  of overlap demolish, slower or shallower ones do not
  extra impulse   the ball's velocity with the extra impulse minus without
                  it (a hit on the previous tick switches it off) equals the
                  published impulse (include/Physics/CarBall/ExtraImpulse.cuh)
  car-ball solve  car and ball momentum is conserved by the contact
  car-arena solve a car sliding on its roof decelerates at mu*g (Coulomb,
                  CAR_WORLD_FRICTION = 0.3); a single-corner impact on the
                  floor (analytic plane) or the back wall (mesh) obeys the
                  rigid-body impulse law, rebounds at CAR_WORLD_RESTITUTION
                  = 0.3 and keeps friction in the cone; a corner inside the
                  mesh is pushed out by position alone
  suspension      a car left on its wheels settles at the height and pitch
                  where the four springs (include/RLConstants.cuh:79-143)
                  balance gravity plus the sticky force; one tick from a
                  known pose adds the spring and damper forces
  air controls    boost and throttle accelerate along the car's nose at
                  BOOST_ACCEL_AIR and THROTTLE_AIR_ACCEL
  ball on floor   a sliding ball rolls at 5/7 of its speed (solid sphere,
                  angular momentum about the contact point), then keeps
                  v = w r while drag takes 0.03 per second of the linear
                  share (5/7) of that momentum; its spin is capped at
                  6 rad/s (BALL_MAX_ANG_SPEED)
  ball edges      the field floor is two coplanar triangles: a ball landing
                  fast across their shared edge, where it also touches the
                  neighbouring triangle at the edge, bounces straight up
                  (the internal-edge adjustment, BallArena/Contact.cuh:454-476,
                  turns that contact's normal back to the face's)
  ball contacts   the contacts gathered for a ball (cell walk, sphere-
                  triangle test, four-point reduction) are those of a
                  brute-force search over all triangles reduced by Bullet's
                  persistent-manifold rule (keep the deepest, replace the
                  point whose removal leaves the largest quad)

A plausible slip (a sign of one body's impulse, a lever arm of the wrong
body, a swapped curve, a dropped clamp or constant) fails one of them."""
import math

import numpy as np
import pytest

from abi import CAR_NAMES, SIM_NAMES
from ball_geometry import bullet_replacement as _bullet_replacement
from ball_geometry import closest_on_triangles as _closest_on_triangles
from oracle_py import OracleEnv

CAR = {n: i for i, n in enumerate(CAR_NAMES)}
SIM = {n: i for i, n in enumerate(SIM_NAMES)}
DT = 1.0 / 120.0
G = 650.0
CAR_MASS = 180.0
# diagonal body inertia of the car (CAR_INV_INERTIA, include/RLConstants.cuh:122)
CAR_INERTIA = np.array([134665.94, 239607.22, 329747.90])


# ------------------------------------------------------------------ helpers

def f32(u):
    return np.asarray(u, np.uint32).view(np.float32).astype(np.float64)


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def quat_axis_angle(axis, angle):
    axis = np.asarray(axis, float) / np.linalg.norm(axis)
    s = math.sin(angle / 2)
    return np.array([axis[0] * s, axis[1] * s, axis[2] * s, math.cos(angle / 2)])


def rot_matrix(q):
    x, y, z, w = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


class Scene:
    """One simulation of the oracle set up field by field."""

    def __init__(self, n_blue, n_orange, seed=3):
        self.env = OracleEnv(1, n_blue, n_orange, seed)
        self.n = n_blue + n_orange

    def close(self):
        self.env.close()

    def place(self, pos, rot, vel, ang, ball_pos=(0.0, 4000.0, 93.15), ball_vel=(0.0, 0.0, 0.0),
              ball_ang=(0.0, 0.0, 0.0)):
        n = self.n
        self.env.set_car(np.asarray(pos, np.float32).reshape(1, n, 3), np.asarray(rot, np.float32).reshape(1, n, 4),
                         np.asarray(vel, np.float32).reshape(1, n, 3), np.asarray(ang, np.float32).reshape(1, n, 3),
                         np.zeros((1, n), np.bool_))
        self.env.set_ball(np.asarray(ball_pos, np.float32).reshape(1, 3),
                          np.asarray(ball_vel, np.float32).reshape(1, 3),
                          np.asarray(ball_ang, np.float32).reshape(1, 3))

    def set_fields(self, car_fields=None, sim_fields=None):
        car, sim, tick = self.env.export_state()
        for (name, c), v in (car_fields or {}).items():
            car[CAR[name], c] = bits(v) if isinstance(v, float) else np.uint32(np.int32(v).view(np.uint32))
        for name, v in (sim_fields or {}).items():
            sim[SIM[name], 0] = bits(v) if isinstance(v, float) else np.uint32(np.int32(v).view(np.uint32))
        self.env.import_state(car, sim, tick)

    def tick(self, n=1, actions=None):
        a = np.zeros((1, self.n, 7), np.float32) if actions is None else actions
        self.env.tick(a, 1, n)

    def state(self):
        car, sim, tick = self.env.export_state()
        return car, sim, tick

    def car_vec(self, name, c, n=3):
        car, _, _ = self.env.export_state()
        i = CAR[name + "_0"]
        return f32(car[i:i + n, c])

    def car_int(self, name, c):
        car, _, _ = self.env.export_state()
        return int(car[CAR[name], c].astype(np.uint32).view(np.int32))

    def car_float(self, name, c):
        car, _, _ = self.env.export_state()
        return float(f32(car[CAR[name], c]))

    def ball_vec(self, name):
        _, sim, _ = self.env.export_state()
        i = SIM[name + "_0"]
        return f32(sim[i:i + 3, 0])


IDENT = [0.0, 0.0, 0.0, 1.0]
# continuous action slots (python/carl.cu layout): steer/yaw, pitch, throttle,
# powerslide, boost, air roll, jump
THROTTLE_SLOT, BOOST_SLOT = 2, 4


def no_bump_fields(n):
    """Every car's last bump target is every other car, cooldown running: the
    bump response is skipped (Response.cuh), the contact solve is not."""
    out = {}
    for c in range(n):
        out[("CARL_CAR_CONTACT_IDX", c)] = (c + 1) % n
        out[("CARL_CAR_CONTACT_COOLDOWN", c)] = 0.2
    return out


# ------------------------------------------------------------------ car-car solve

def _car_pair_run(pos, rot, vel, ang):
    s = Scene(2, 0)
    s.place(pos, rot, vel, ang)
    s.set_fields(no_bump_fields(2))
    s.tick()
    out = [(s.car_vec("CARL_CAR_VEL", c), s.car_vec("CARL_CAR_ANG", c)) for c in range(2)]
    s.close()
    return out


def test_car_car_solve_conserves_momentum():
    """Airborne pair, same team (no demolition), bumps off: the contact solve
    exchanges equal and opposite impulses, so it keeps the pair's linear
    momentum and its angular momentum about the midpoint, up to the friction
    moment over the contact gap (depth x |P_t|).  The collision's share of
    each car's change is the run minus the same run with the cars 1000 uu
    apart (gravity and the air-control damping of the spin act in both).
    The cars are only yawed, so a face axis separates them: an edge-edge
    axis makes a contact of two support points that are not on one line
    along the normal (CarCar/Clip.cuh), whose normal impulse has a moment of
    its own."""
    rng = np.random.default_rng(5)
    for trial in range(8):
        yaw = rng.uniform(-0.1, 0.1, 2)
        q = [quat_axis_angle([0, 0, 1], y) for y in yaw]
        pa = np.array([0.0, 0.0, 1000.0])
        pb = np.array([rng.uniform(-20, 20), rng.uniform(80.0, 86.0), 1000.0 + rng.uniform(-5, 5)])
        # the contact gap is at most the boxes' overlap along y: each yawed box
        # reaches half_y cos + half_x |sin| from its centre, and the centres
        # sit at the hitbox offset rotated by the yaw
        reach = (43.282655 * np.cos(yaw) + 60.186455 * np.abs(np.sin(yaw))).sum()
        cen_dy = pb[1] + 13.87566 * (np.sin(yaw[1]) - np.sin(yaw[0]))
        gap = reach - abs(cen_dy) + 1.0
        v = [np.array([rng.uniform(-200, 200), rng.uniform(200, 400), rng.uniform(-50, 50)]),
             np.array([rng.uniform(-200, 200), rng.uniform(-400, -200), rng.uniform(-50, 50)])]
        w = [rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.5, 0.5, 3)]
        hit = _car_pair_run([pa, pb], q, v, w)
        apart = _car_pair_run([pa, pb + [0.0, 1000.0, 0.0]], q, v, w)
        dv = [hit[c][0] - apart[c][0] for c in range(2)]
        dw = [hit[c][1] - apart[c][1] for c in range(2)]
        impulse = CAR_MASS * np.linalg.norm(dv[0])
        assert impulse > CAR_MASS * 50.0, trial          # the pair did collide
        np.testing.assert_allclose(CAR_MASS * (dv[0] + dv[1]), 0.0, atol=CAR_MASS * 0.02)
        p0, mid = [pa, pb], (pa + pb) / 2
        dl = np.zeros(3)
        for c in range(2):
            r = rot_matrix(q[c])
            dl += CAR_MASS * np.cross(p0[c] - mid, dv[c]) + r @ (CAR_INERTIA * (r.T @ dw[c]))
        # a lever arm of the wrong body would be off by ~50 uu x impulse
        assert np.linalg.norm(dl) < gap * 0.09 * impulse, (trial, dl, gap, impulse)


def test_car_car_side_impact_restitution():
    """Parallel cars closing sideways at 300 uu/s each: the contact normal is
    y and there is no tangential motion, so they separate at 0.1 of the
    closing speed, symmetrically (to within the convergence of ten
    sequential-impulse sweeps over four coupled contact points)."""
    s = Scene(2, 0)
    s.place([[0, 0, 1000], [0, 85, 1000]], [IDENT, IDENT], [[0, 300, 0], [0, -300, 0]], [[0, 0, 0]] * 2)
    s.set_fields(no_bump_fields(2))
    s.tick()
    va, vb = s.car_vec("CARL_CAR_VEL", 0), s.car_vec("CARL_CAR_VEL", 1)
    assert abs(va[1] - (-30.0)) < 2.0 and abs(vb[1] - 30.0) < 2.0, (va, vb)
    assert abs(va[1] + vb[1]) < 1e-3
    assert abs(va[0]) < 1e-3 and abs(vb[0]) < 1e-3
    assert abs(va[2] + G * DT) < 1e-3 and abs(vb[2] + G * DT) < 1e-3
    s.close()


# ------------------------------------------------------------------ bump, demolition

CAR_LEN = 2 * 60.186455


def _published_curve(speed, points):
    """Piecewise-linear curve through the published (speed, value) points,
    flat outside them."""
    xs, ys = zip(*points)
    return float(np.interp(speed, xs, ys))


BUMP_GROUND = [(0.0, 5.0 / 6.0), (1400.0, 1100.0), (2200.0, 1530.0)]
BUMP_AIR = [(0.0, 5.0 / 6.0), (1400.0, 1390.0), (2200.0, 1945.0)]
BUMP_UP = [(0.0, 2.0 / 6.0), (1400.0, 278.0), (2200.0, 417.0)]


def _rear_end(n_blue, n_orange, speed, z, overlap, bump, alone=False):
    """Car 0 drives at `speed` along +x into the back of car 1 (both at rest
    height z, identity rotation, boxes overlapping by `overlap` uu); returns
    both cars' velocity after one tick and car 1's demolition flag."""
    s = Scene(n_blue, n_orange)
    pb = np.array([0.0, 0.0, z])
    pa = pb - [CAR_LEN - overlap, 0.0, 0.0]
    if alone:
        pb = pb + [0.0, 3000.0, 0.0]
    s.place([pa, pb], [IDENT, IDENT], [[speed, 0.0, 0.0], [0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]] * 2)
    if not bump:
        s.set_fields({("CARL_CAR_CONTACT_IDX", 0): 1, ("CARL_CAR_CONTACT_COOLDOWN", 0): 0.2})
    grounded = s.car_int("CARL_CAR_ON_GROUND", 1)
    s.tick()
    out = [s.car_vec("CARL_CAR_VEL", c) for c in range(2)], s.car_int("CARL_CAR_DEMOED", 1), grounded
    s.close()
    return out


@pytest.mark.parametrize("speed", [300.0, 1000.0, 1400.0, 1800.0, 2150.0, 2290.0])
@pytest.mark.parametrize("where", ["ground", "air"])
def test_bump_impulse_follows_published_curves(speed, where):
    """Same team, so no demolition.  The run without the bump isolates the
    impulse given to the victim: along the bumper's pre-solve velocity, the
    ground or air curve of the closing speed, plus the upward curve along the
    victim's up axis (world up in the air), added after the contact solve and
    capped with the velocity at the 2300 uu/s car speed limit."""
    z = 17.0 if where == "ground" else 600.0
    (with_bump, _, grounded) = _rear_end(2, 0, speed, z, 1.0, True)
    (without, _, _) = _rear_end(2, 0, speed, z, 1.0, False)
    (alone, _, _) = _rear_end(2, 0, speed, z, 1.0, True, alone=True)
    assert grounded == (1 if where == "ground" else 0)
    pre = alone[0]                       # the bumper's velocity entering the car-car stage
    closing = float(pre @ [1.0, 0.0, 0.0])   # delta is +x up to the split correction
    fwd = _published_curve(closing, BUMP_GROUND if where == "ground" else BUMP_AIR)
    up = _published_curve(closing, BUMP_UP)
    impulse = pre / np.linalg.norm(pre) * fwd + np.array([0.0, 0.0, up])
    # the impulse is added after the solve, then the car speed is capped at 2300
    expect = without[1] + impulse
    expect *= min(1.0, 2300.0 / np.linalg.norm(expect))
    np.testing.assert_allclose(with_bump[1], expect, rtol=0, atol=0.01 * np.linalg.norm(impulse) + 0.5)
    # the bumper itself gets nothing from the bump
    np.testing.assert_allclose(with_bump[0], without[0], atol=1e-3)


@pytest.mark.parametrize("speed,overlap,demo", [
    (2290.0, 6.0, 1),    # supersonic, deep enough
    (2150.0, 6.0, 0),    # below supersonic: a bump
    (2290.0, 3.0, 0),    # supersonic but under 5 uu of overlap: a bump
])
def test_demolition_needs_supersonic_speed_and_depth(speed, overlap, demo):
    (vel, demoed, _) = _rear_end(1, 1, speed, 17.0, overlap, True)
    assert demoed == demo
    (vel_same_team, demoed_same, _) = _rear_end(2, 0, speed, 17.0, overlap, True)
    assert demoed_same == 0


# ------------------------------------------------------------------ car-ball extra impulse

# hitbox centre offset and half extents (CAR_OFFSETS, CAR_HALF_EX, include/RLConstants.cuh:33-34)
HITBOX_OFFSET = np.array([13.87566, 0.0, 20.755])
HALF = np.array([60.186455, 43.282655, 19.262505])
BALL_R = 91.25
EXTRA_CURVE = [(0.0, 0.65), (500.0, 0.65), (2300.0, 0.55), (4600.0, 0.30)]


def _ball_hit(car_vel, ball_pos, ball_vel, extra=True, car=True, ball=True):
    """One airborne car (identity rotation, pos at the origin + 500 z) and the
    ball; returns (ball velocity, car velocity) after one tick."""
    s = Scene(1, 0)
    pc = np.array([0.0, 0.0, 500.0]) + ([0.0, 0.0, 0.0] if car else [0.0, -3000.0, 0.0])
    pb = np.asarray(ball_pos, float) + ([0.0, 0.0, 0.0] if ball else [0.0, 3000.0, 0.0])
    s.place([pc], [IDENT], [car_vel], [[0.0, 0.0, 0.0]], ball_pos=pb, ball_vel=ball_vel,
            ball_ang=(0.0, 0.0, 1e-3))
    if not extra:
        s.set_fields({("CARL_CAR_BALL_HIT_TICK", 0): 0})    # hit on the previous tick
    s.tick()
    out = s.ball_vec("CARL_SIM_BALL_VEL"), s.car_vec("CARL_CAR_VEL", 0)
    s.close()
    return out


def _published_extra(ball_pos, car_pos, pre_ball_vel, pre_car_vel):
    rel = pre_ball_vel - pre_car_vel
    speed = min(np.linalg.norm(rel), 4600.0)
    d = np.asarray(ball_pos) - car_pos
    hit = np.array([d[0], d[1], d[2] * 0.35])
    hit /= np.linalg.norm(hit)
    fwd = np.array([1.0, 0.0, 0.0])
    hit = hit - fwd * (hit @ fwd) * (1.0 - 0.65)
    hit /= np.linalg.norm(hit)
    return hit * speed * _published_curve(speed, EXTRA_CURVE)


_cen_z = 500.0 + HITBOX_OFFSET[2]
_front = HITBOX_OFFSET[0] + HALF[0]
EXTRA_CASES = [
    # (car velocity, ball position, ball velocity)
    ([500.0, 0.0, 0.0], [_front + BALL_R - 1.0, 0.0, _cen_z], [0.0, 0.0, 0.0]),
    ([1500.0, 0.0, 0.0], [_front + BALL_R - 1.0, 0.0, _cen_z], [0.0, 0.0, 0.0]),
    ([2200.0, 0.0, 0.0], [_front + BALL_R - 1.0, 0.0, _cen_z], [-900.0, 0.0, 0.0]),      # over 2300 relative
    ([2200.0, 0.0, 0.0], [_front + BALL_R - 1.0, 0.0, _cen_z], [-3000.0, 0.0, 0.0]),     # capped at 4600
    ([1200.0, 300.0, 0.0], [_front + 60.0, 40.0, _cen_z + HALF[2] + 60.0], [0.0, 0.0, 0.0]),  # over the bonnet
    ([1000.0, 0.0, 0.0], [_front + 50.0, HALF[1] + 70.0, _cen_z], [0.0, -400.0, 0.0]),  # front corner, side
]


@pytest.mark.parametrize("car_vel,ball_pos,ball_vel", EXTRA_CASES)
def test_extra_impulse_follows_published_formula(car_vel, ball_pos, ball_vel):
    """The ball's velocity with the extra impulse minus without it is the
    published impulse: the car-to-ball direction with z scaled by 0.35, its
    forward part scaled by 0.65, times the relative speed (capped at 4600)
    times the published factor curve, from the velocities entering the
    car-ball stage (the car's after gravity, the ball's after drag and
    gravity)."""
    with_extra, _ = _ball_hit(car_vel, ball_pos, ball_vel, extra=True)
    without, _ = _ball_hit(car_vel, ball_pos, ball_vel, extra=False)
    _, pre_car = _ball_hit(car_vel, ball_pos, ball_vel, ball=False)
    pre_ball, _ = _ball_hit(car_vel, ball_pos, ball_vel, car=False)
    assert np.linalg.norm(without - pre_ball) > 100.0          # the car did hit the ball
    expect = _published_extra(ball_pos, np.array([0.0, 0.0, 500.0]), pre_ball, pre_car)
    np.testing.assert_allclose(with_extra - without, expect, rtol=0, atol=1e-3 * np.linalg.norm(expect) + 0.05)


# ------------------------------------------------------------------ suspension

# wheel geometry and spring constants (include/RLConstants.cuh:76-92, 135-143;
# include/Physics/SuspensionUtils.cuh): anchors relative to the hitbox centre,
# rays down the car's -z axis
ANCHORS = [np.array([37.3743, 25.9, 0.0]), np.array([37.3743, -25.9, 0.0]),
           np.array([-47.6257, 29.5, 0.0]), np.array([-47.6257, -29.5, 0.0])]
WHEEL_R = [12.5, 12.5, 15.0, 15.0]
REST = [26.755, 26.755, 25.055, 25.055]
SCALE = [35.75, 35.75, 54.265, 54.265]
STIFFNESS, TRAVEL = 500.0, 12.0
STICKY = 0.5          # fraction of gravity added along the wheel normals when not driving


def _rot_y(t):
    return np.array([[math.cos(t), 0.0, math.sin(t)], [0.0, 1.0, 0.0], [-math.sin(t), 0.0, math.cos(t)]])


def _spring_terms(z, th):
    """Per wheel: spring push (rest - length) * stiffness, its lever arm about
    the centre of mass, and cos(pitch), for a car at height z and pitch theta
    over the flat floor."""
    r = _rot_y(th)
    up = r @ [0.0, 0.0, 1.0]
    cen = np.array([0.0, 0.0, z]) + r @ HITBOX_OFFSET
    out = []
    for k in range(4):
        start = cen + r @ ANCHORS[k]
        dist = start[2] / up[2]                       # along -up to the floor
        length = np.clip(dist - WHEEL_R[k], REST[k] - TRAVEL, REST[k] + TRAVEL)
        out.append(((REST[k] - length) * STIFFNESS, r @ (HITBOX_OFFSET + ANCHORS[k]) - up * dist))
    return out, up[2]


def _spring_balance(x):
    """Net vertical spring force minus weight (gravity + sticky force), and the
    springs' pitching moment about the centre of mass."""
    terms, cos_th = _spring_terms(*x)
    force = moment = 0.0
    for k, (push, lever) in enumerate(terms):
        f = max(push / cos_th * SCALE[k], 0.0)
        force += f
        moment += lever[0] * f
    return [force - CAR_MASS * G * (1.0 + STICKY), moment]


def _equilibrium():
    from scipy.optimize import fsolve
    z, th = fsolve(_spring_balance, [17.0, 0.0], xtol=1e-12)
    return z, th


def test_suspension_settles_at_spring_equilibrium():
    """A car left on its wheels comes to rest where the four springs carry
    gravity plus the sticky force and their moments cancel."""
    z_eq, th_eq = _equilibrium()
    s = Scene(1, 0)
    s.place([[0.0, 0.0, 17.0]], [IDENT], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.tick(240)
    pos, q = s.car_vec("CARL_CAR_POS", 0), s.car_vec("CARL_CAR_ROT", 0, 4)
    pitch = 2.0 * math.atan2(q[1], q[3])
    assert abs(pos[2] - z_eq) < 1e-3, (pos[2], z_eq)
    assert abs(pitch - th_eq) < 1e-5, (pitch, th_eq)
    assert np.linalg.norm(s.car_vec("CARL_CAR_VEL", 0)) < 1e-3
    s.close()


@pytest.mark.parametrize("vz", [-100.0, -30.0, 10.0, 20.0, 100.0])
def test_suspension_damping_one_tick(vz):
    """From the equilibrium pose moving vertically at vz, one tick changes vz
    by the wheel forces, ((rest - length) * 500 - d * vz) * scale / cos(pitch)
    with d = 25 while the wheels close in and 40 while they open, each
    clamped at zero (a wheel only pushes), less gravity and the sticky force.
    At +100 uu/s relaxation damping outweighs every spring: weight alone."""
    z_eq, th_eq = _equilibrium()
    terms, cos_th = _spring_terms(z_eq, th_eq)
    damping = 25.0 if vz < 0 else 40.0
    force = sum(max((push - damping * vz) / cos_th * SCALE[k], 0.0) for k, (push, _) in enumerate(terms))
    expect = vz + (force / CAR_MASS - G * (1.0 + STICKY)) * DT
    s = Scene(1, 0)
    s.place([[0.0, 0.0, z_eq]], [quat_axis_angle([0, 1, 0], th_eq)], [[0.0, 0.0, vz]], [[0.0, 0.0, 0.0]])
    s.tick()
    got = s.car_vec("CARL_CAR_VEL", 0)[2]
    assert abs(got - expect) < 0.02, (got, expect)
    s.close()


@pytest.mark.parametrize("pitch", [0.2, -0.25, 0.35])
def test_suspension_force_one_tick_pitched(pitch):
    """Pitched over the flat floor at rest, the lowest wheel 1.5 uu into its
    travel (short of the 2.5 uu pushback band): one tick adds the springs'
    push, each (rest - length) * 500 * scale / cos(pitch) for a wheel whose
    ray (rest + travel + radius - 2.5 long) reaches the floor, clamped at
    zero, less gravity and the sticky force along the floor normal."""
    r = _rot_y(pitch)
    up = r @ [0.0, 0.0, 1.0]
    reach = [r @ (HITBOX_OFFSET + ANCHORS[k]) for k in range(4)]
    # height putting the deepest wheel at 1.5 uu of compression
    z = max((REST[k] + WHEEL_R[k] - 1.5) * up[2] - reach[k][2] for k in range(4))
    terms, cos_th = _spring_terms(z, pitch)
    force, count = 0.0, 0
    for k, (push, _) in enumerate(terms):
        dist = (z + reach[k][2]) / up[2]
        if dist > REST[k] + TRAVEL + WHEEL_R[k] - 2.5:
            continue                                   # ray misses the floor
        count += 1
        force += max(push / cos_th * SCALE[k], 0.0)
    assert 0 < count < 4
    expect = (force / CAR_MASS - G * (1.0 + STICKY)) * DT
    s = Scene(1, 0)
    s.place([[0.0, 0.0, z]], [quat_axis_angle([0, 1, 0], pitch)], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.tick()
    got = s.car_vec("CARL_CAR_VEL", 0)
    assert abs(got[2] - expect) < 0.02, (got, expect)
    s.close()


# ------------------------------------------------------------------ car-arena solve

UPSIDE_DOWN = [1.0, 0.0, 0.0, 0.0]       # half turn about x
# a flipped car's roof lies on the floor when its hitbox centre is half a
# box height up, i.e. pos z = half z + offset z (the offset points down)
ROOF_Z = HALF[2] + HITBOX_OFFSET[2]


def test_car_sliding_on_roof_decelerates_at_coulomb_rate():
    """Upside down on the flat floor (wheels in the air, no input) the only
    horizontal force is the body's friction: |dv/dt| = mu g = 0.3 * 650.
    The manifold is rebuilt every tick from the deepest point of each
    analytic plane, so the roof rests on one corner at a time and the car
    rocks (its vertical velocity is not zero); the split impulse keeps it on
    the floor."""
    s = Scene(1, 0)
    s.place([[0.0, 0.0, ROOF_Z + 0.5]], [UPSIDE_DOWN], [[800.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.tick(30)
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    s.tick(60)
    v1 = s.car_vec("CARL_CAR_VEL", 0)
    assert abs(v1[1]) < 0.5 and abs(s.car_vec("CARL_CAR_POS", 0)[2] - ROOF_Z) < 1.0
    decel = (v0[0] - v1[0]) / (60 * DT)
    assert abs(decel - 0.3 * G) < 0.02 * 0.3 * G, decel
    s.close()


def _quat_from_matrix(r):
    w = math.sqrt(max(0.0, 1.0 + r[0, 0] + r[1, 1] + r[2, 2])) / 2.0
    if w > 1e-6:
        return np.array([(r[2, 1] - r[1, 2]) / (4 * w), (r[0, 2] - r[2, 0]) / (4 * w), (r[1, 0] - r[0, 1]) / (4 * w), w])
    x = math.sqrt(max(0.0, 1.0 + r[0, 0] - r[1, 1] - r[2, 2])) / 2.0
    return np.array([x, (r[0, 1] + r[1, 0]) / (4 * x), (r[0, 2] + r[2, 0]) / (4 * x), (r[2, 1] - r[1, 2]) / (4 * x)])


# (surface normal, point on the surface, corner offset along the normal):
# the floor is an analytic plane of the car-arena manifold (a contact within
# the break distance counts); the back wall above the goal is arena mesh
# (contacts need the box-triangle SAT to overlap, so the corner is 1 uu in)
SURFACES = {
    "floor": (np.array([0.0, 0.0, 1.0]), np.array([0.0, 0.0, 0.0]), 1.0),
    "back_wall": (np.array([0.0, -1.0, 0.0]), np.array([-597.0, 5120.0, 1109.0]), -1.0),
}


@pytest.mark.parametrize("surface", ["floor", "back_wall"])
@pytest.mark.parametrize("tilt,speed,slide", [
    ((0.25, 0.15), 250.0, (0.0, 0.0)),
    ((-0.3, 0.2), 200.0, (150.0, -80.0)),
    ((0.1, -0.35), 300.0, (-300.0, 200.0)),
])
def test_single_corner_impact(surface, tilt, speed, slide):
    """A tilted car, no spin, wheels clear of everything, moves into a flat
    surface with one box corner leading (touching it): the car-arena
    manifold holds one point, so the body's momentum change less gravity is
    the contact impulse P, and
      its spin change is I_world^-1 (r x P), r the contact from the centre
      of mass: the corner itself on an analytic plane (then capped at
      5.5 rad/s), a point within 1 uu of it on the mesh;
      that point leaves the surface at 0.3 of its approach speed
      (restitution);
      the friction part of P stays inside the cone |P_t| <= 0.3 P_n."""
    normal, on_surface, offset = SURFACES[surface]
    flip = np.diag([1.0, -1.0, -1.0]) if surface == "floor" else np.eye(3)   # roof first onto the floor
    yaw = 0.0 if surface == "floor" else 0.3              # a side, not an edge, facing the wall
    r_yaw = np.array([[math.cos(yaw), -math.sin(yaw), 0.0], [math.sin(yaw), math.cos(yaw), 0.0], [0.0, 0.0, 1.0]])
    r = r_yaw @ _rot_y(tilt[1]) @ np.array([[1.0, 0.0, 0.0], [0.0, math.cos(tilt[0]), -math.sin(tilt[0])],
                                            [0.0, math.sin(tilt[0]), math.cos(tilt[0])]]) @ flip
    q = _quat_from_matrix(r)
    local = np.sign(r.T @ -normal) * HALF                  # box corner deepest along -normal, car frame
    arm = r @ (HITBOX_OFFSET + local)                      # corner from the centre of mass
    # every other corner stays more than 1 uu behind it along the normal
    corners = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)]) * HALF
    lead = np.sort((corners @ r.T) @ -normal)
    assert lead[-1] - lead[-2] > 1.5, lead[-2:]
    corner = on_surface + normal * offset
    pos = corner - arm
    tangent = np.cross(normal, [1.0, 0.0, 0.0] if abs(normal[0]) < 0.9 else [0.0, 1.0, 0.0])
    tangent /= np.linalg.norm(tangent)
    v0 = -normal * speed + tangent * slide[0] + np.cross(normal, tangent) * slide[1]
    s = Scene(1, 0)
    s.place([pos], [q], [v0], [[0.0, 0.0, 0.0]])
    s.tick()
    assert s.car_int("CARL_CAR_MANIFOLD_COUNT", 0) == 1
    v1, w1 = s.car_vec("CARL_CAR_VEL", 0), s.car_vec("CARL_CAR_ANG", 0)
    impulse = CAR_MASS * (v1 - v0 - np.array([0.0, 0.0, -G * DT]))
    inv_inertia = r @ np.diag(1.0 / CAR_INERTIA) @ r.T
    if surface == "floor":
        # an analytic plane's manifold point is the box corner itself
        w_solve = inv_inertia @ np.cross(arm, impulse)
        # the spin is capped at 5.5 rad/s after the solve
        np.testing.assert_allclose(w1, w_solve * min(1.0, 5.5 / np.linalg.norm(w_solve)), rtol=2e-3, atol=1e-4)
        point = arm
    else:
        # a mesh contact is the deepest point of the triangle clipped to the
        # car's witness face (CarArena/Clip.cuh): next to the corner, not on it.
        # Its lever arm follows from P and the spin up to a part along P; that
        # part puts the point at the corner's depth along the normal (the
        # corner is only 1 uu into the wall).
        assert np.linalg.norm(w1) < 5.4
        w_solve = w1
        along = impulse / np.linalg.norm(impulse)
        point = np.cross(impulse, r @ (CAR_INERTIA * (r.T @ w1))) / (impulse @ impulse)
        point = point + along * ((arm - point) @ normal / (along @ normal))
        assert np.linalg.norm(point - arm) < 1.0, (point, arm)
    approach = v0 @ normal                                 # the corner's normal velocity before (no spin)
    leave = (v1 + np.cross(w_solve, point)) @ normal
    slack = 0.0 if surface == "floor" else 2.0             # the 1 uu the mesh point may sit off the corner
    assert abs(leave - 0.3 * -approach) < 0.01 * abs(approach) + slack, (leave, approach)
    p_n = impulse @ normal
    p_t = np.linalg.norm(impulse - normal * p_n)
    assert p_n > 0 and p_t <= 0.3 * p_n * (1 + 1e-4), (p_n, p_t)
    s.close()


@pytest.mark.parametrize("depth", [0.5, 1.0, 3.0])
def test_mesh_penetration_is_pushed_out_by_position_only(depth):
    """A car at rest with one corner `depth` uu into the back wall (mesh):
    the split impulse moves it out of the wall within the tick (by the
    contact ERP, 0.8, of the depth at most) and leaves no velocity along
    the normal (a resting contact has nothing to rebound from)."""
    normal, on_surface, _ = SURFACES["back_wall"]
    yaw, tilt = 0.3, (0.25, 0.15)
    r_yaw = np.array([[math.cos(yaw), -math.sin(yaw), 0.0], [math.sin(yaw), math.cos(yaw), 0.0], [0.0, 0.0, 1.0]])
    r = r_yaw @ _rot_y(tilt[1]) @ np.array([[1.0, 0.0, 0.0], [0.0, math.cos(tilt[0]), -math.sin(tilt[0])],
                                            [0.0, math.sin(tilt[0]), math.cos(tilt[0])]])
    arm = r @ (HITBOX_OFFSET + np.sign(r.T @ -normal) * HALF)
    pos = on_surface - normal * depth - arm
    s = Scene(1, 0)
    s.place([pos], [_quat_from_matrix(r)], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.tick()
    moved = (s.car_vec("CARL_CAR_POS", 0) - pos) @ normal
    assert 0.05 * depth < moved <= 0.8 * depth * 1.01, (moved, depth)
    assert abs(s.car_vec("CARL_CAR_VEL", 0) @ normal) < 1e-3
    s.close()

# ------------------------------------------------------------------ ball on the floor

BALL_REST_Z = 91.25


def _roll(v0, direction, ticks):
    d = np.asarray(direction, float) / np.linalg.norm(direction)
    s = Scene(1, 0)
    s.place([[0.0, -4000.0, 17.0]], [IDENT], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]],
            ball_pos=(-1500.0 * d[0], -1500.0 * d[1], BALL_REST_Z), ball_vel=tuple(v0 * d), ball_ang=(0.0, 0.0, 0.0))
    out = []
    for _ in range(ticks):
        s.tick()
        out.append((s.ball_vec("CARL_SIM_BALL_POS"), s.ball_vec("CARL_SIM_BALL_VEL"), s.ball_vec("CARL_SIM_BALL_ANG")))
    s.close()
    return d, out


def test_ball_slides_into_rolling_at_five_sevenths():
    v0 = 600.0
    d, traj = _roll(v0, (1.0, 0.6, 0.0), 360)
    side = np.array([-d[1], d[0], 0.0])
    for pos, vel, ang in traj:
        assert abs(pos[2] - BALL_REST_Z) < 0.01 and abs(vel[2]) < 0.02     # no kick at any triangle edge
        assert abs(vel @ side) < 0.02
    speed = [float(v @ d) for _, v, _ in traj]
    spin = [float(np.cross([0.0, 0.0, 1.0], d) @ w) for _, _, w in traj]  # rolling axis z x d
    # rolling from about 1 s on: v = w r
    for t in (150, 240, 359):
        assert abs(speed[t] - spin[t] * BALL_REST_Z) < 1e-4 * speed[t], t
    # 5/7 of v0, less the drag of the first 1.25 s on a share between 5/7 and 1
    t = 150
    lo, hi = 5 / 7 * 0.97 ** (t / 120), 5 / 7 * 0.97 ** (5 / 7 * t / 120)
    assert lo < speed[t - 1] / v0 < hi, (speed[t - 1] / v0, lo, hi)
    # rolling decay: drag on the linear 5/7 share of the rolling momentum
    ratio = speed[359] / speed[149]
    assert abs(ratio - 0.97 ** (5 / 7 * 210 / 120)) < 2e-5, ratio


def test_ball_spin_cap():
    """Fast enough that rolling would need more than 6 rad/s: the spin sits at
    the cap while the ball slides, and rolling starts at 6 r."""
    d, traj = _roll(1200.0, (1.0, 0.0, 0.0), 420)
    spin = np.array([np.linalg.norm(w) for _, _, w in traj])
    speed = np.array([float(v @ d) for _, v, _ in traj])
    assert spin.max() <= 6.0 * (1 + 1e-6)
    capped = np.nonzero(spin >= 6.0 * (1 - 1e-6))[0]
    assert len(capped) > 60
    rolling = np.nonzero(np.abs(speed - spin * BALL_REST_Z) < 1e-4 * speed)[0]
    assert len(rolling) > 0 and speed[rolling[0]] <= 6.0 * BALL_REST_Z * (1 + 1e-4)


def _floor_diagonal():
    env = OracleEnv(1, 1, 0, 0)
    verts, tris, _, _, _ = env.arena()
    env.close()
    tv = verts[tris]
    n = np.cross(tv[:, 1] - tv[:, 0], tv[:, 2] - tv[:, 0])
    n /= np.linalg.norm(n, axis=1)[:, None]
    floor = np.nonzero((np.abs(n[:, 2]) > 0.999) & (tv[:, :, 2].max(1) < 5.0))[0]
    assert len(floor) == 2
    shared = sorted(set(tris[floor[0]]) & set(tris[floor[1]]))
    assert len(shared) == 2
    return verts[shared[0]], verts[shared[1]]


@pytest.mark.parametrize("along", [0.3, 0.5, 0.7])
@pytest.mark.parametrize("off", [-15.0, 10.0, 25.0])
def test_ball_bounces_straight_up_across_the_floor_seam(along, off):
    """Landing at 2500 uu/s, 10-25 uu from the seam: the ball sinks far enough
    into the floor to touch the other triangle at the seam; that contact's
    normal is corrected to the floor normal, so no sideways velocity
    appears (without the correction: hundreds of uu/s)."""
    a, b = _floor_diagonal()
    e = (b - a) / np.linalg.norm(b - a)
    start = a + (b - a) * along + np.array([-e[1], e[0], 0.0]) * off
    s = Scene(1, 0)
    s.place([[0.0, 4500.0 if start[1] < 0 else -4500.0, 17.0]], [IDENT], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]],
            ball_pos=(start[0], start[1], 130.0), ball_vel=(0.0, 0.0, -2500.0))
    bounced = False
    for _ in range(6):
        s.tick()
        v = s.ball_vec("CARL_SIM_BALL_VEL")
        bounced |= v[2] > 0
        assert np.linalg.norm(v[:2]) < 0.1, v
    assert bounced
    s.close()


# ------------------------------------------------------------------ ball contact gather and reduction

BALL_BREAK = 1.905        # contact distance beyond the radius (BallArena/Contact.cuh)


def _brute_force_ball_contacts(tv, center):
    """Every triangle of the mesh (tv: [n, 3, 3] float64) in ascending index
    order: a contact when the closest point lies within radius + break; at
    most four kept, the rest placed by the replacement rule.  Returns the
    kept triangles in slot order and the reason, if any, that a decision sat
    within float32 rounding of its threshold."""
    q = _closest_on_triangles(center, tv[:, 0], tv[:, 1], tv[:, 2])
    dist = np.linalg.norm(center - q, axis=1)
    reach = BALL_R + BALL_BREAK
    if np.any(np.abs(dist - reach) < 2e-3):
        return None, "reach"
    if np.count_nonzero(dist < reach) > 12:
        return None, "long"          # long replacement chains amplify rounding
    kept, slot_tri = [], []
    for t in np.nonzero(dist < reach)[0]:
        cand = (-(center - q[t]) / dist[t] * BALL_R, BALL_R - dist[t])     # reduction offset, depth
        if len(kept) < 4:
            kept.append(cand)
            slot_tri.append(int(t))
            continue
        depths = sorted([k[1] for k in kept] + [cand[1]], reverse=True)
        if depths[0] - depths[1] < 1e-3:
            return None, "depth"
        slot, tie = _bullet_replacement(kept, cand)
        if tie:
            return None, "area"
        kept[slot] = cand
        slot_tri[slot] = int(t)
    return slot_tri, None


def test_ball_contacts_match_brute_force_with_bullet_reduction():
    """Ball centres placed into the mesh at random triangles (up to 6 uu
    deep), weighted to the finely tessellated curved parts: the oracle's
    contacts (cell walk, sphere-triangle test, four-point reduction) are the
    brute-force contacts over all triangles reduced by Bullet's rule."""
    env = OracleEnv(1, 1, 0, 0)
    verts, tris, _, _, _ = env.arena()
    tv = verts[tris].astype(np.float64)
    n = np.cross(tv[:, 1] - tv[:, 0], tv[:, 2] - tv[:, 0])
    area = np.linalg.norm(n, axis=1)
    n /= area[:, None]
    rng = np.random.default_rng(11)
    weights = 1.0 / np.sqrt(np.maximum(area, 1.0))  # favour small triangles: curved, tessellated surfaces
    picks = rng.choice(len(tris), 600, p=weights / weights.sum())
    checked = reduced = 0
    skipped = {}
    for t in picks:
        centroid = tv[t].mean(0)
        center = (centroid + n[t] * (BALL_R - rng.uniform(0.0, 6.0))).astype(np.float32).astype(np.float64)
        expect, ambiguous = _brute_force_ball_contacts(tv, center)
        if ambiguous:
            skipped[ambiguous] = skipped.get(ambiguous, 0) + 1
            continue
        got = env.ball_contacts(center)[0]
        assert list(got) == expect, (t, center, list(got), expect)
        checked += 1
        reduced += len(expect) == 4
    env.close()
    assert checked >= 100 and reduced >= 20, (checked, reduced, skipped)


# ------------------------------------------------------------------ car-ball solve, air controls

@pytest.mark.parametrize("car_vel,ball_pos,ball_vel", EXTRA_CASES)
def test_car_ball_solve_conserves_momentum(car_vel, ball_pos, ball_vel):
    """With the one-sided extra impulse off, the car-ball contact exchanges
    equal and opposite impulses: the car's (180) and the ball's (30) momentum
    change, each against its velocity entering the stage, sums to zero."""
    ball, car = _ball_hit(car_vel, ball_pos, ball_vel, extra=False)
    _, pre_car = _ball_hit(car_vel, ball_pos, ball_vel, ball=False)
    pre_ball, _ = _ball_hit(car_vel, ball_pos, ball_vel, car=False)
    dp_car = CAR_MASS * (car - pre_car)
    dp_ball = (CAR_MASS / 6.0) * (ball - pre_ball)
    assert np.linalg.norm(dp_ball) > 30.0 * 100.0
    np.testing.assert_allclose(dp_car + dp_ball, 0.0, atol=1e-3 * np.linalg.norm(dp_ball))


@pytest.mark.parametrize("axis,angle", [((0, 0, 1), 0.0), ((0, 1, 0), -0.6), ((1, 1, 0), 0.9), ((1, -2, 1), 2.5)])
@pytest.mark.parametrize("boost,throttle,accel", [(1.0, 0.0, 3175.0 / 3.0), (0.0, 1.0, 200.0 / 3.0),
                                                  (0.0, -0.5, -100.0 / 3.0)])
def test_air_boost_and_throttle_accelerate_along_the_nose(axis, angle, boost, throttle, accel):
    """In the air, boost adds 3175/3 uu/s^2 and throttle 200/3 uu/s^2 per
    unit along the car's forward axis, on top of gravity
    (BOOST_ACCEL_AIR, THROTTLE_AIR_ACCEL, include/RLConstants.cuh:173-181)."""
    q = quat_axis_angle(axis, angle)
    s = Scene(1, 0)
    s.place([[0.0, 0.0, 1000.0]], [q], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.set_fields({("CARL_CAR_BOOST", 0): 50.0})
    a = np.zeros((1, 1, 7), np.float32)
    a[..., BOOST_SLOT] = boost
    a[..., THROTTLE_SLOT] = throttle
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    s.tick(3, actions=a)
    dv = s.car_vec("CARL_CAR_VEL", 0) - v0 - np.array([0.0, 0.0, -3 * G * DT])
    np.testing.assert_allclose(dv, rot_matrix(q)[:, 0] * accel * 3 * DT, atol=1e-3)
    s.close()
