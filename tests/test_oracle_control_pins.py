"""The CPU oracle's control model against the game's published numbers, each
isolated in a scene where nothing else acts (free flight, or a differential
run that changes only the control under test):

  jump           a grounded press adds JUMP_IMMEDIATE_FORCE = 875/3 uu/s plus
                 one tick of 0.62 x JUMP_ACCEL along the car's up axis; the
                 jump then accelerates at JUMP_ACCEL = 4375/3 uu/s^2 (x0.62
                 before JUMP_MIN_TIME = 0.025 s) while jump is held, up to
                 JUMP_MAX_TIME = 0.2 s, or only to JUMP_MIN_TIME when it is
                 released (include/RLConstants.cuh:150-155)
  double jump    a press in the air with less than 0.5 of stick adds
                 875/3 uu/s along up at once
  dodges         a forward dodge adds 500 uu/s along the horizontal heading at
                 any speed; a side dodge 500 x (1 + 0.9 s/2300); a backward
                 dodge 500 x 16/15 x (1 + 1.5 s/2300) (FLIP_INITIAL_VEL_SCALE,
                 the side/backward max-speed scales 1.9 and 2.5, include/
                 RLConstants.cuh:157-169)
  flip           the flip spins the car at FLIP_TORQUE_Y = 224 (forward)
                 or FLIP_TORQUE_X = 260 (side) rad/s^2 about the car's own
                 axes, and damps the vertical velocity by 0.35 per tick from
                 0.15 s to 0.21 s into the flip and while falling up to 0.65 s
  air control    full pitch, yaw and roll input accelerate at 130, 95 and 400
                 x 2 pi/65.536 = 12.46, 9.11 and 38.35 rad/s^2 about the car's
                 -right, up and -forward axes; spin decays at 30, 20 and 50 x
                 2 pi/65.536 per second, pitch and yaw damping switched off by
                 full input on that axis, roll damping never
  drive          from rest on the flat floor, throttle accelerates at
                 THROTTLE_GROUND_ACCEL = 1600 uu/s^2 scaled by the drive curve
                 1 - 0.9 v/1400, to the 1410 uu/s top speed (Drive.cuh:28-66,
                 RLConstants.cuh:270-278)
  powerslide     the handbrake value rises at 5/s and falls at 2/s; the front
                 wheels turn by the normal full-lock angle moved toward the
                 powerslide angle by the handbrake value (read from the
                 direction of the front axle's impulse); the wheels keep a
                 lateral friction 1 - 0.8 c scaled by 1 - 0.9 h and a
                 longitudinal 1 + (0.5 + 0.4 c - 1) h for slip curve input c,
                 used in the following tick (CarSuspension.cuh:150-190)

Each expected value is computed here from those constants, in float64, so
a plausible slip in the oracle (a constant swapped between two dodges, the
heading not flattened, a damping term on the wrong axis, a curve breakpoint
moved) fails one of them.
"""
import math

import numpy as np
import pytest

from carl_amd import workloads
from test_oracle_physics_pins import CAR, DT, G, IDENT, Scene, bits, f32, quat_axis_angle, rot_matrix

JUMP_IMMEDIATE = 875.0 / 3.0
JUMP_ACCEL = 4375.0 / 3.0
JUMP_MIN, JUMP_MAX = 0.025, 0.2
TORQUE_SCALE = 2.0 * math.pi / 65536.0 * 1000.0
AIR_TORQUE = np.array([130.0, 95.0, 400.0])     # pitch, yaw, roll
AIR_DAMPING = np.array([30.0, 20.0, 50.0])

DIRECT = 2


def direct(n_cars=1, **fields):
    c = np.zeros(n_cars, workloads.CONTROLS_DTYPE)
    for k, v in fields.items():
        c[k] = v
    return c


def tick_direct(s: Scene, controls, n=1):
    s.env.tick(np.ascontiguousarray(controls), DIRECT, n)


def airborne(rot=IDENT, vel=(0.0, 0.0, 0.0), ang=(0.0, 0.0, 0.0), z=1000.0, **fields):
    """One car in free flight far from every surface, internal fields set."""
    s = Scene(1, 0)
    s.place([[0.0, 0.0, z]], [rot], [vel], [ang])
    s.set_fields({(k, 0): v for k, v in fields.items()})
    return s


def up_axis(q):
    return rot_matrix(q)[:, 2]


# ------------------------------------------------------------------ jump

ALONG_Y = quat_axis_angle((0, 0, 1), math.pi / 2)


def _settled_car(rot=IDENT, pos=(0.0, -1500.0, 17.0)):
    s = Scene(1, 0)
    s.place([pos], [rot], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    tick_direct(s, direct(), 240)
    return s


def _long_straight():
    """A settled car at the blue end facing +y, beside the goal: 9,000 uu of
    flat floor ahead."""
    return _settled_car(ALONG_Y, (-2000.0, -4000.0, 17.0))


def test_grounded_jump_press_adds_the_immediate_impulse_and_first_acceleration():
    """Same settled car, one tick with and one without a jump press: the
    difference is JUMP_IMMEDIATE_FORCE + 0.62 JUMP_ACCEL dt along up."""
    s = _settled_car()
    saved = s.env.export_state()
    up = _rot(s)[:, 2]                             # the settled car rests slightly pitched
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    tick_direct(s, direct())
    v_plain = s.car_vec("CARL_CAR_VEL", 0)
    s.env.import_state(*saved)
    tick_direct(s, direct(jump=1))
    v_jump = s.car_vec("CARL_CAR_VEL", 0)
    assert abs(v_plain[2] - v0[2]) < 1.0           # settled: the plain tick barely moves it
    np.testing.assert_allclose(v_jump - v_plain, up * (JUMP_IMMEDIATE + 0.62 * JUMP_ACCEL * DT), atol=2e-3)
    assert s.car_int("CARL_CAR_IS_JUMPING", 0) == 1 and s.car_int("CARL_CAR_HAS_JUMPED", 0) == 1
    s.close()


def _jump_timeline(held: bool, t0: float) -> list[float]:
    """Per-tick jump acceleration from the published rule, with the jump
    clock kept in float32 as the game keeps it."""
    dt = np.float32(DT)
    t = np.float32(t0)
    jumping, out = True, []
    for _ in range(40):
        if jumping:
            jumping = bool(t < np.float32(JUMP_MIN) or (held and t < np.float32(JUMP_MAX)))
        out.append(JUMP_ACCEL * (0.62 if t < np.float32(JUMP_MIN) else 1.0) if jumping else 0.0)
        t = np.float32(t + dt)
    return out


@pytest.mark.parametrize("held,t0", [(True, 0.0), (False, 0.0), (True, 0.1), (False, 0.1)])
@pytest.mark.parametrize("axis,angle", [((0, 0, 1), 0.0), ((1, 0, 0), 0.7), ((1, 2, 0), -1.1)])
def test_airborne_jump_acceleration_follows_the_timeline(held, t0, axis, angle):
    """An airborne car mid-jump: each tick adds JUMP_ACCEL dt (x0.62 before
    JUMP_MIN_TIME) along its up axis until JUMP_MAX_TIME with jump held, or
    until JUMP_MIN_TIME once released; gravity is the only other change."""
    q = quat_axis_angle(axis, angle)
    s = airborne(q, CARL_CAR_HAS_JUMPED=1, CARL_CAR_IS_JUMPING=1, CARL_CAR_JUMP_TIME=float(t0), CARL_CAR_LAST_JUMP=1)
    want = _jump_timeline(held, t0)
    up = up_axis(q)
    for k, a in enumerate(want):
        v0 = s.car_vec("CARL_CAR_VEL", 0)
        tick_direct(s, direct(jump=int(held)))
        dv = s.car_vec("CARL_CAR_VEL", 0) - v0 - np.array([0.0, 0.0, -G * DT])
        np.testing.assert_allclose(dv, up * a * DT, atol=2e-3, err_msg=f"tick {k}")
    assert s.car_int("CARL_CAR_IS_JUMPING", 0) == 0
    s.close()


@pytest.mark.parametrize("pitch,yaw,roll", [(0.0, 0.0, 0.0), (0.2, 0.2, 0.0), (0.0, 0.0, 0.49)])
def test_double_jump_below_the_dodge_deadzone(pitch, yaw, roll):
    q = quat_axis_angle((0, 1, 1), 0.8)
    s = airborne(q, CARL_CAR_HAS_JUMPED=1, CARL_CAR_AIR_TIME_SINCE_JUMP=0.3)
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    tick_direct(s, direct(jump=1, pitch=pitch, yaw=yaw, roll=roll))
    dv = s.car_vec("CARL_CAR_VEL", 0) - v0 - np.array([0.0, 0.0, -G * DT])
    np.testing.assert_allclose(dv, up_axis(q) * JUMP_IMMEDIATE, atol=2e-3)
    assert s.car_int("CARL_CAR_HAS_DOUBLE_JUMPED", 0) == 1 and s.car_int("CARL_CAR_HAS_FLIPPED", 0) == 0
    s.close()


def test_no_second_jump_after_the_dodge_window():
    """DOUBLEJUMP_MAX_DELAY = 1.25 s after the jump the press does nothing."""
    s = airborne(CARL_CAR_HAS_JUMPED=1, CARL_CAR_AIR_TIME_SINCE_JUMP=1.25)
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    tick_direct(s, direct(jump=1, pitch=-1.0))
    np.testing.assert_allclose(s.car_vec("CARL_CAR_VEL", 0) - v0, [0.0, 0.0, -G * DT], atol=1e-3)
    assert s.car_int("CARL_CAR_HAS_FLIPPED", 0) == 0 and s.car_int("CARL_CAR_HAS_DOUBLE_JUMPED", 0) == 0
    s.close()


# ------------------------------------------------------------------ dodges

def _published_dodge(heading: float, fwd_speed: float, pitch: float, yaw: float, roll: float) -> np.ndarray:
    """World velocity a dodge adds: 500 uu/s scaled per direction by speed."""
    d = np.array([-pitch, yaw + roll])
    d = d / np.linalg.norm(d)
    d[np.abs(d) < 0.1] = 0.0
    speed_frac = min(abs(fwd_speed) / 2300.0, 1.0)
    backward = d[0] < 0.0 if abs(fwd_speed) < 100.0 else (d[0] >= 0.0) != (fwd_speed >= 0.0)
    forward_scale = (1.0 + 1.5 * speed_frac) * 16.0 / 15.0 if backward else 1.0
    local = 500.0 * np.array([d[0] * forward_scale, d[1] * (1.0 + 0.9 * speed_frac)])
    ahead = np.array([math.cos(heading), math.sin(heading), 0.0])
    side = np.array([-math.sin(heading), math.cos(heading), 0.0])
    return ahead * local[0] + side * local[1]


@pytest.mark.parametrize("pitch,yaw,roll", [(-1.0, 0.0, 0.0), (1.0, 0.0, 0.0), (0.0, 1.0, 0.0), (0.0, 0.0, -1.0),
                                            (-0.7, 0.7, 0.0), (-1.0, 0.05, 0.0), (0.6, -0.3, -0.3)])
@pytest.mark.parametrize("speed", [0.0, 50.0, -50.0, 1000.0, -800.0, 2300.0])
@pytest.mark.parametrize("heading,nose_up", [(0.0, 0.0), (1.1, 0.4)])
def test_dodge_impulse_at_published_scales(pitch, yaw, roll, speed, heading, nose_up):
    """Dodges from free flight with the car moving along its nose: the added
    velocity (with gravity, same tick) is the published dodge impulse in
    the car's horizontal frame, whatever the car's pitch, and the result is
    capped at CAR_MAX_SPEED = 2300 uu/s."""
    q = quat_axis_angle((0, 0, 1), heading)
    q = _compose(q, quat_axis_angle((0, 1, 0), -nose_up))
    nose = rot_matrix(q)[:, 0]
    s = airborne(q, vel=tuple(nose * speed), CARL_CAR_HAS_JUMPED=1, CARL_CAR_AIR_TIME_SINCE_JUMP=0.1)
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    tick_direct(s, direct(jump=1, pitch=pitch, yaw=yaw, roll=roll))
    want = v0 + _published_dodge(heading, speed, pitch, yaw, roll) + np.array([0.0, 0.0, -G * DT])
    if np.linalg.norm(want) > 2300.0:
        want *= 2300.0 / np.linalg.norm(want)
    np.testing.assert_allclose(s.car_vec("CARL_CAR_VEL", 0), want, atol=5e-3)
    assert s.car_int("CARL_CAR_HAS_FLIPPED", 0) == 1 and s.car_int("CARL_CAR_IS_FLIPPING", 0) == 1
    s.close()


def _compose(a, b):
    """Quaternion product a*b (xyzw)."""
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return np.array([aw * bx + ax * bw + ay * bz - az * by, aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw, aw * bw - ax * bx - ay * by - az * bz])


def _rot(s: Scene) -> np.ndarray:
    """The car's rotation matrix now (the controls of the next tick use it)."""
    i = CAR["CARL_CAR_ROT_0"]
    return rot_matrix(f32(s.env.export_state()[0][i:i + 4, 0]))


@pytest.mark.parametrize("pitch,yaw,local_accel", [(-1.0, 0.0, (0.0, 224.0, 0.0)), (1.0, 0.0, (0.0, -224.0, 0.0)),
                                                   (0.0, 1.0, (-260.0, 0.0, 0.0)), (0.0, -1.0, (260.0, 0.0, 0.0))])
@pytest.mark.parametrize("axis,angle", [((0, 0, 1), 0.0), ((1, 1, 1), 1.2)])
def test_flip_spins_about_the_car_axes(pitch, yaw, local_accel, axis, angle):
    """After a dodge the flip adds FLIP_TORQUE_Y = 224 (forward/backward) or
    FLIP_TORQUE_X = 260 (sideways) rad/s^2 about the car's own axis, the
    stick held in the flip's direction; air control is off meanwhile."""
    q = quat_axis_angle(axis, angle)
    s = airborne(q, CARL_CAR_HAS_JUMPED=1, CARL_CAR_AIR_TIME_SINCE_JUMP=0.1)
    tick_direct(s, direct(jump=1, pitch=pitch, yaw=yaw))            # starts the flip
    for k in range(2):
        frame = _rot(s)
        w0 = s.car_vec("CARL_CAR_ANG", 0)
        tick_direct(s, direct(jump=1, pitch=pitch, yaw=yaw))
        dw = s.car_vec("CARL_CAR_ANG", 0) - w0
        np.testing.assert_allclose(dw, frame @ np.array(local_accel) * DT, atol=2e-4, err_msg=f"tick {k}")
    s.close()


def _damped_ticks(v0z: float) -> list[bool]:
    """Ticks whose vertical velocity the flip damps (float32 flip clock)."""
    dt = np.float32(DT)
    t = np.float32(0.0)
    vz = v0z
    out = []
    for _ in range(90):
        t = np.float32(t + dt)
        damp = t <= np.float32(0.65) and t >= np.float32(0.15) and (vz < 0.0 or t < np.float32(0.21))
        out.append(bool(damp))
        vz = vz * (0.65 if damp else 1.0) - G * DT
    return out


@pytest.mark.parametrize("vz", [400.0, 900.0, -100.0])
def test_flip_damps_vertical_velocity_on_the_published_window(vz):
    """From 0.15 s into the flip vz is multiplied by 1 - 0.35 each tick up to
    0.21 s, and afterwards while it is negative, until FLIP_TORQUE_TIME."""
    s = airborne(vel=(0.0, 0.0, vz), z=1500.0, CARL_CAR_HAS_JUMPED=1, CARL_CAR_AIR_TIME_SINCE_JUMP=0.1)
    v0 = s.car_vec("CARL_CAR_VEL", 0)
    tick_direct(s, direct(jump=1, pitch=-1.0))                      # starts the flip (this tick counts)
    vz_now = s.car_vec("CARL_CAR_VEL", 0)[2]
    np.testing.assert_allclose(vz_now, v0[2] - G * DT, atol=1e-3)
    plan = _damped_ticks(vz_now)
    for k, damp in enumerate(plan[1:60]):
        before = s.car_vec("CARL_CAR_VEL", 0)[2]
        tick_direct(s, direct(pitch=-1.0))
        after = s.car_vec("CARL_CAR_VEL", 0)[2]
        want = before * (0.65 if damp else 1.0) - G * DT
        assert abs(after - want) < 2e-3 * max(1.0, abs(want)), (k, before, after, damp)
    assert any(plan) and not all(plan)
    s.close()


# ------------------------------------------------------------------ air control

PUBLISHED_AIR_ACCEL = {"pitch": 12.46, "yaw": 9.11, "roll": 38.35}   # rad/s^2 at full input


@pytest.mark.parametrize("axis_name,sign", [("pitch", 1.0), ("pitch", -1.0), ("yaw", 1.0), ("roll", -1.0)])
@pytest.mark.parametrize("axis,angle", [((0, 0, 1), 0.0), ((0.3, -1, 2), 2.2)])
def test_air_control_angular_acceleration(axis_name, sign, axis, angle):
    """Full stick from no spin: angular acceleration equals the published
    air-control values about -right (pitch), up (yaw) and -forward (roll)."""
    q = quat_axis_angle(axis, angle)
    s = airborne(q)
    r = _rot(s)
    w0 = s.car_vec("CARL_CAR_ANG", 0)
    tick_direct(s, direct(**{axis_name: sign}))
    dw = s.car_vec("CARL_CAR_ANG", 0) - w0
    direction = {"pitch": -r[:, 1], "yaw": r[:, 2], "roll": -r[:, 0]}[axis_name]
    accel = AIR_TORQUE[["pitch", "yaw", "roll"].index(axis_name)] * TORQUE_SCALE
    assert abs(accel - PUBLISHED_AIR_ACCEL[axis_name]) < 0.01
    np.testing.assert_allclose(dw / DT, direction * sign * accel, atol=1e-3)
    s.close()


@pytest.mark.parametrize("spin_axis", [0, 1, 2])
@pytest.mark.parametrize("hold", [None, "pitch", "yaw", "roll"])
def test_air_control_damping_rates(spin_axis, hold):
    """Spin about one car axis with no stick decays at 30/20/50 x the torque
    scale (pitch/yaw/roll); full stick on the spinning axis removes pitch
    and yaw damping but not roll damping."""
    s = airborne()
    dirs = np.array([[0.0, -1.0, 0.0], [0.0, 0.0, 1.0], [-1.0, 0.0, 0.0]])   # pitch, yaw, roll axes (identity)
    w = dirs[spin_axis] * 2.0
    s.set_fields({("CARL_CAR_ANG_0", 0): float(w[0]), ("CARL_CAR_ANG_1", 0): float(w[1]),
                  ("CARL_CAR_ANG_2", 0): float(w[2])})
    controls = direct(**({hold: 1.0} if hold else {}))
    w0 = s.car_vec("CARL_CAR_ANG", 0)
    tick_direct(s, controls)
    dw = s.car_vec("CARL_CAR_ANG", 0) - w0
    axis_names = ["pitch", "yaw", "roll"]
    damping_on = hold != axis_names[spin_axis] or spin_axis == 2
    want = -dirs[spin_axis] * (dirs[spin_axis] @ w0) * AIR_DAMPING[spin_axis] * TORQUE_SCALE * DT * damping_on
    if hold:
        want = want + {"pitch": dirs[0], "yaw": dirs[1], "roll": dirs[2]}[hold] * AIR_TORQUE[
            axis_names.index(hold)] * TORQUE_SCALE * DT
    np.testing.assert_allclose(dw, want, atol=1e-5)
    s.close()


# ------------------------------------------------------------------ ground drive

def _drive_curve(v: float) -> float:
    if v <= 0.0:
        return 1.0
    if v >= 1410.0:
        return 0.0
    if v <= 1400.0:
        return 1.0 - 0.9 * v / 1400.0
    return 0.1 * (1.0 - (v - 1400.0) / 10.0)


def test_throttle_from_rest_follows_the_drive_curve_to_top_speed():
    """Full throttle (no boost) on the flat floor: the forward acceleration
    is 1600 uu/s^2 x (1 - 0.9 v / 1400) and the speed tops out at 1410."""
    s = _long_straight()
    speeds = []
    for _ in range(480):
        tick_direct(s, direct(throttle=1.0))
        speeds.append(s.car_vec("CARL_CAR_VEL", 0)[1])
    v = np.array(speeds)
    # drive is staged one tick behind; compare the acceleration over ticks 4..120
    accel = np.diff(v)[3:120] / DT
    want = np.array([1600.0 * _drive_curve(x) for x in v[2:119]])
    np.testing.assert_allclose(accel, want, rtol=0.02, atol=8.0)
    assert 1405.0 < v[-1] <= 1411.0        # one tick of staged drive may overshoot 1410 slightly
    assert abs(s.car_vec("CARL_CAR_VEL", 0)[0]) < 1.0
    s.close()


@pytest.mark.parametrize("throttle_after,decel", [(0.0, 525.0), (-1.0, 3500.0)])
def test_coasting_and_braking_deceleration(throttle_after, decel):
    """Rolling at speed, releasing the throttle coasts at 0.15 of the full
    brake and opposing throttle brakes fully: CAR_MASS x (14.25 + 1/3) of
    brake torque per wheel, four wheels sharing the car's mass three ways,
    gives 525 and 3500 uu/s^2 (Drive.cuh:14-26, CarSuspension.cuh:207-215)."""
    s = _long_straight()
    tick_direct(s, direct(throttle=1.0), 90)
    speeds = [s.car_vec("CARL_CAR_VEL", 0)[1]]
    assert speeds[0] > 800.0
    for _ in range(12):
        tick_direct(s, direct(throttle=throttle_after))
        speeds.append(s.car_vec("CARL_CAR_VEL", 0)[1])
    # the brake is staged one tick behind the input
    got = -np.diff(speeds)[2:] / DT
    np.testing.assert_allclose(got, decel, rtol=0.01)
    s.close()


def test_reverse_throttle_follows_the_drive_curve():
    s = _settled_car()
    speeds = []
    for _ in range(60):
        tick_direct(s, direct(throttle=-1.0))
        speeds.append(-s.car_vec("CARL_CAR_VEL", 0)[0])
    v = np.array(speeds)
    accel = np.diff(v)[3:] / DT
    np.testing.assert_allclose(accel, [1600.0 * _drive_curve(x) for x in v[2:-2]], rtol=0.02, atol=8.0)
    s.close()


# ------------------------------------------------------------------ steering

WHEELBASE = 37.3743 + 47.6257      # front and rear suspension x (include/RLConstants.cuh:84-87)
_STEER_CURVE = ((0.0, 0.53356), (500.0, 0.31930), (1000.0, 0.18203), (1500.0, 0.10570), (1750.0, 0.08507),
                (3000.0, 0.03454))


def _steer_angle(speed: float) -> float:
    """Published front-wheel steer angle at full lock (RLConstants.cuh:252-262)."""
    pts = _STEER_CURVE
    if speed <= 0.0:
        return pts[0][1]
    for (a, fa), (b, fb) in zip(pts, pts[1:]):
        if speed <= b:
            return fa + (fb - fa) * (speed - a) / (b - a)
    return pts[-1][1]


@pytest.mark.parametrize("target", [250.0, 300.0, 400.0])
@pytest.mark.parametrize("steer", [1.0, -1.0])
def test_full_lock_turning_radius_at_low_speed(target, steer):
    """Held at a steady low speed with full lock, the car turns on the
    circle of the kinematic bicycle model: yaw rate / speed = tan(delta) / L
    with delta the published steer angle at that speed and L the distance
    between the axles (lateral slip is negligible this slowly)."""
    s = _settled_car(ALONG_Y, (0.0, -2000.0, 17.0))
    kappa = []
    for t in range(720):
        v = s.car_vec("CARL_CAR_VEL", 0)
        speed = float(np.hypot(v[0], v[1]))
        throttle = float(np.clip((target - speed) / 100.0, -1.0, 1.0))
        tick_direct(s, direct(throttle=throttle, steer=steer if t >= 60 else 0.0))
        if t >= 600:
            w = s.car_vec("CARL_CAR_ANG", 0)
            kappa.append((w[2] / speed, speed))
    got, speed = np.mean([k for k, _ in kappa]), np.mean([v for _, v in kappa])
    assert abs(speed - target) < 0.05 * target
    want = math.copysign(math.tan(_steer_angle(speed)) / WHEELBASE, steer)
    assert abs(got / want - 1.0) < 0.02, (got, want, speed)
    s.close()


# ------------------------------------------------------------------ autoroll

AUTOROLL_FORCE, AUTOROLL_TORQUE = 100.0, 80.0     # CAR_AUTOROLL_FORCE / _TORQUE (RLConstants.cuh:145-146)


def _autoroll_difference(q, z):
    """One tick from the same pose with a small throttle and with none; the
    throttle's only same-tick effects are the autoroll and (off the ground)
    the air throttle (drive and brake act a tick later)."""
    s = Scene(1, 0)
    s.place([[0.0, -1500.0, z]], [q], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    saved = s.env.export_state()
    out = []
    for throttle in (0.0, 0.01):
        s.env.import_state(*saved)
        tick_direct(s, direct(throttle=throttle))
        out.append((s.car_vec("CARL_CAR_VEL", 0), s.car_vec("CARL_CAR_ANG", 0)))
        car, _, _ = s.env.export_state()
        contacts = car[CAR["CARL_CAR_WHEEL_CONTACT_0"]:CAR["CARL_CAR_WHEEL_CONTACT_0"] + 4, 0].tolist()
        chassis = int(car[CAR["CARL_CAR_MANIFOLD_COUNT"], 0])
    s.close()
    return out[1][0] - out[0][0], out[1][1] - out[0][1], contacts, chassis


@pytest.mark.parametrize("phi,z,wheels", [(0.3, 28.0, [0, 1, 0, 1]), (0.6, 32.0, [0, 1, 0, 1]),
                                          (-0.5, 28.0, [1, 0, 1, 0])])
def test_autoroll_on_two_side_wheels_rolls_the_car_upright(phi, z, wheels):
    """A car rolled by phi, on the two wheels of one side on the flat floor,
    with throttle: autoroll pushes it down at CAR_AUTOROLL_FORCE and turns
    it back about its nose: the contact-aligned right axis (floor normal x
    nose) makes an angle phi with the car's right axis, so the torque is
    CAR_AUTOROLL_TORQUE x (1 - cos phi), against the roll."""
    q = quat_axis_angle((1, 0, 0), phi)
    dv, dw, contacts, chassis = _autoroll_difference(q, z)
    assert contacts == wheels and chassis == 0
    nose = rot_matrix(q)[:, 0]
    np.testing.assert_allclose(dv, [0.0, 0.0, -AUTOROLL_FORCE * DT] + nose * 0.01 * 200.0 / 3.0 * DT, atol=2e-5)
    want = -math.copysign(1.0, phi) * np.array([1.0, 0.0, 0.0]) * (1.0 - math.cos(phi)) * AUTOROLL_TORQUE * DT
    np.testing.assert_allclose(dw, want, atol=2e-6)


@pytest.mark.parametrize("theta,z,wheels", [(0.25, 28.0, [1, 1, 0, 0]), (0.4, 36.0, [1, 1, 0, 0]),
                                            (-0.35, 28.0, [0, 0, 1, 1])])
def test_autoroll_on_two_end_wheels_pitches_the_car_level(theta, z, wheels):
    """Pitched by theta onto its front (or rear) wheels: the pitch torque is
    CAR_AUTOROLL_TORQUE x sin^2 theta about the car's right axis, against
    the pitch (the nose projected on the floor-aligned frame keeps
    cos^2 theta of it), plus (1 - cos theta) about the nose."""
    q = quat_axis_angle((0, 1, 0), theta)
    dv, dw, contacts, chassis = _autoroll_difference(q, z)
    assert contacts == wheels and chassis == 0
    r = rot_matrix(q)
    nose, right = r[:, 0], r[:, 1]
    np.testing.assert_allclose(dv, [0.0, 0.0, -AUTOROLL_FORCE * DT] + nose * 0.01 * 200.0 / 3.0 * DT, atol=2e-5)
    pitch_back = -math.copysign(1.0, theta) * right * math.sin(theta) ** 2
    want = (pitch_back - nose * (1.0 - math.cos(theta))) * AUTOROLL_TORQUE * DT
    np.testing.assert_allclose(dw, want, atol=2e-6)


def _chassis_autoroll_difference(q):
    """_autoroll_difference for a car high in the air whose arena manifold of
    the tick before holds one contact of normal +z, as a car lying on the
    floor leaves it: no wheel touches, so autoroll takes its up direction
    from that normal."""
    s = Scene(1, 0)
    s.place([[0.0, -1500.0, 600.0]], [q], [[0.0, 0.0, 0.0]], [[0.0, 0.0, 0.0]])
    s.set_fields({("CARL_CAR_MANIFOLD_COUNT", 0): 1, ("CARL_CAR_MANIFOLD_NORMAL_0", 0): 0.0,
                  ("CARL_CAR_MANIFOLD_NORMAL_1", 0): 0.0, ("CARL_CAR_MANIFOLD_NORMAL_2", 0): 1.0})
    saved = s.env.export_state()
    out = []
    for throttle in (0.0, 0.01):
        s.env.import_state(*saved)
        tick_direct(s, direct(throttle=throttle))
        out.append((s.car_vec("CARL_CAR_VEL", 0), s.car_vec("CARL_CAR_ANG", 0)))
    s.close()
    return out[1][0] - out[0][0], out[1][1] - out[0][1]


@pytest.mark.parametrize("phi", [0.5, -1.2, 2.0, -2.4, 2.9, -3.1])
def test_autoroll_from_the_chassis_manifold_saturates_past_a_quarter_roll(phi):
    """A car rolled by phi about its level nose, touching the floor with its
    body only: autoroll pushes it down at CAR_AUTOROLL_FORCE and turns it
    about the nose against the roll, at CAR_AUTOROLL_TORQUE x (1 - cos phi)
    up to a quarter roll and at the full CAR_AUTOROLL_TORQUE beyond it (on
    its side or its roof the contact-aligned right axis points against the
    car's, and the factor stays at 1); the level nose gets no pitch torque."""
    q = quat_axis_angle((1, 0, 0), phi)
    dv, dw = _chassis_autoroll_difference(q)
    nose = rot_matrix(q)[:, 0]
    np.testing.assert_allclose(dv, [0.0, 0.0, -AUTOROLL_FORCE * DT] + nose * 0.01 * 200.0 / 3.0 * DT, atol=2e-5)
    factor = 1.0 - max(math.cos(phi), 0.0)
    want = -math.copysign(1.0, math.sin(phi)) * np.array([1.0, 0.0, 0.0]) * factor * AUTOROLL_TORQUE * DT
    np.testing.assert_allclose(dw, want, atol=2e-6)


def test_no_autoroll_on_four_wheels():
    s = _settled_car()
    saved = s.env.export_state()
    out = []
    for throttle in (0.0, 0.01):
        s.env.import_state(*saved)
        tick_direct(s, direct(throttle=throttle))
        out.append((s.car_vec("CARL_CAR_VEL", 0), s.car_vec("CARL_CAR_ANG", 0)))
    np.testing.assert_allclose(out[1][0], out[0][0], atol=1e-6)
    np.testing.assert_allclose(out[1][1], out[0][1], atol=1e-7)
    s.close()


# ------------------------------------------------------------------ powerslide

POWERSLIDE_RISE, POWERSLIDE_FALL = 5.0, 2.0      # POWERSLIDE_RISE_RATE / _FALL_RATE (RLConstants.cuh:185-186)
_SLIDE_CURVE = ((0.0, 0.39235), (2500.0, 0.12610))


def _slide_angle(speed: float) -> float:
    """Published front-wheel steer angle at full lock under full handbrake
    (RLConstants.cuh:263-268)."""
    (a, fa), (b, fb) = _SLIDE_CURVE
    if speed <= a:
        return fa
    return fa + (fb - fa) * min(speed, b) / b


def test_handbrake_rises_and_falls_at_the_published_rates():
    """Powerslide held, the handbrake value climbs at 5 per second to 1;
    released, it falls at 2 per second to 0 (Drive.cuh:123-146)."""
    s = _settled_car()
    h = 0.0
    for t in range(40):
        tick_direct(s, direct(slide=1))
        h = min(1.0, h + POWERSLIDE_RISE * DT)
        assert abs(s.car_float("CARL_CAR_HANDBRAKE", 0) - h) < 1e-5, t
    for t in range(70):
        tick_direct(s, direct())
        h = max(0.0, h - POWERSLIDE_FALL * DT)
        assert abs(s.car_float("CARL_CAR_HANDBRAKE", 0) - h) < 1e-5, t
    s.close()


def _coasting_start(speed: float, handbrake: float, slip: float = 0.0, lat_used: float = 1.0):
    """A car settled on the flat floor, set moving at `speed` at `slip`
    radians from its nose, without spin, the handbrake value set, the
    previous tick's brake, drive and steer cleared and every wheel's
    friction of the previous tick set to lat_used: no wheel acts along the
    floor before the first tick's lateral impulses."""
    s = _settled_car()
    car, _, _ = s.state()
    r = rot_matrix(f32(car[s_idx("CARL_CAR_ROT_0"):s_idx("CARL_CAR_ROT_0") + 4, 0]))
    v = speed * (math.cos(slip) * r[:, 0] + math.sin(slip) * r[:, 1])
    fields = {("CARL_CAR_VEL_%d" % i, 0): float(v[i]) for i in range(3)}
    fields.update({("CARL_CAR_ANG_%d" % i, 0): 0.0 for i in range(3)})
    fields.update({("CARL_CAR_HANDBRAKE", 0): handbrake, ("CARL_CAR_BRAKE_STAGE", 0): 0.0,
                   ("CARL_CAR_DRIVE_STAGE", 0): 0.0, ("CARL_CAR_STEER_STAGE", 0): 0.0})
    fields.update({("CARL_CAR_LAT_FRICTION_%d" % w, 0): lat_used for w in range(4)})
    fields.update({("CARL_CAR_LON_FRICTION_%d" % w, 0): lat_used for w in range(4)})
    s.set_fields(fields)
    return s, r


def s_idx(name):
    from test_oracle_physics_pins import CAR
    return CAR[name]


@pytest.mark.parametrize("speed", [300.0, 1200.0, 2200.0])
@pytest.mark.parametrize("handbrake", [0.5, 1.0])
@pytest.mark.parametrize("steer", [1.0, -1.0])
def test_powerslide_blends_the_steer_angle(speed, handbrake, steer):
    """Under the handbrake the front wheels turn by the normal full-lock
    angle moved toward the powerslide angle in proportion to the handbrake
    value: delta = steer x (a(v) + (p(v) - a(v)) h) with a and p the
    published curves.  Measured from the wheels themselves: a car rolling
    straight with powerslide held and no throttle gets no brake, drive or
    rolling friction, so the only impulses along the floor in the tick
    after the steer is staged are the front wheels' lateral ones, along
    their axle; the direction of that velocity change is the axle's, turned
    by delta from the car's right axis."""
    h0 = handbrake - POWERSLIDE_RISE * DT if handbrake < 1.0 else 1.0
    s, r0 = _coasting_start(speed, h0)
    fwd_speed = abs(float(s.car_vec("CARL_CAR_VEL", 0) @ r0[:, 0]))
    tick_direct(s, direct(slide=1, steer=steer))           # stages the steer angle
    assert abs(s.car_float("CARL_CAR_HANDBRAKE", 0) - handbrake) < 1e-6
    car, _, _ = s.state()
    r = rot_matrix(f32(car[s_idx("CARL_CAR_ROT_0"):s_idx("CARL_CAR_ROT_0") + 4, 0]))
    v0 = s.car_vec("CARL_CAR_VEL", 0).astype(np.float64)
    tick_direct(s, direct(slide=1, steer=steer))
    dv = s.car_vec("CARL_CAR_VEL", 0).astype(np.float64) - v0
    s.close()
    dv[2] = 0.0
    delta = steer * (_steer_angle(fwd_speed) + (_slide_angle(fwd_speed) - _steer_angle(fwd_speed)) * handbrake)
    right, up = r[:, 1], r[:, 2]
    axle = right * math.cos(delta) + np.cross(up, right) * math.sin(delta)
    axle[2] = 0.0
    axle /= np.linalg.norm(axle)
    assert np.linalg.norm(dv) > 0.5, dv
    sin_err = np.linalg.norm(np.cross(dv / np.linalg.norm(dv), axle))
    assert sin_err < 2e-3, (sin_err, delta, dv)


@pytest.mark.parametrize("slip", [0.0, 0.3, 0.8, math.pi / 2])
@pytest.mark.parametrize("handbrake", [0.0, 0.4, 1.0])
def test_wheel_friction_under_slip_and_handbrake(slip, handbrake):
    """The friction each wheel keeps for the next tick (CarSuspension.cuh:
    150-190): with curve input c = |v.axle| / (|v.(axle x n)| + |v.axle|)
    for a wheel sliding at slip angle b (c = sin b / (cos b + sin b)), zero
    below 5 uu/s of side speed, the lateral friction is (1 - 0.8 c) scaled
    by 1 - 0.9 h under handbrake h, the longitudinal 1 + (0.5 + 0.4 c - 1) h,
    both x the non-sticky factor (1 on the flat floor).  A car coasting at
    800 uu/s with the powerslide on (h rises by 5/120 in the tick) or off
    (falls by 2/120); every wheel's figure is compared."""
    held = handbrake > 0.0
    h0 = max(0.0, handbrake - POWERSLIDE_RISE * DT) if held else 0.0
    s, _ = _coasting_start(800.0, h0, slip)
    tick_direct(s, direct(slide=1 if held else 0))
    h = s.car_float("CARL_CAR_HANDBRAKE", 0)
    assert abs(h - handbrake) < 1e-6
    side, along = 800.0 * math.sin(slip), 800.0 * math.cos(slip)
    c = side / (along + side) if side > 5.0 else 0.0
    lat = (1.0 - 0.8 * c) * (1.0 - 0.9 * h)
    lon = 1.0 + (0.5 + 0.4 * c - 1.0) * h
    for w in range(4):
        got_lat = s.car_float("CARL_CAR_LAT_FRICTION_%d" % w, 0)
        got_lon = s.car_float("CARL_CAR_LON_FRICTION_%d" % w, 0)
        assert abs(got_lat - lat) < 3e-3 and abs(got_lon - lon) < 3e-3, (w, got_lat, lat, got_lon, lon)
    s.close()


@pytest.mark.parametrize("slip", [0.5, math.pi / 2])
def test_lateral_friction_acts_one_tick_later(slip):
    """The lateral impulse of a tick uses the friction the previous tick
    kept: two runs differing only in the handbrake value (1 and 0.4 after
    the first tick) take the same first tick, and in the second the
    sideways velocity change of the one is (1 - 0.9) / (1 - 0.36) times the
    other's."""
    out = []
    for h in (1.0, 0.4):
        s, r = _coasting_start(800.0, h - POWERSLIDE_RISE * DT if h < 1.0 else 1.0, slip, lat_used=0.5)
        v0 = s.car_vec("CARL_CAR_VEL", 0).astype(np.float64)
        tick_direct(s, direct(slide=1))
        v1 = s.car_vec("CARL_CAR_VEL", 0).astype(np.float64)
        tick_direct(s, direct(slide=1))
        v2 = s.car_vec("CARL_CAR_VEL", 0).astype(np.float64)
        out.append(((v1 - v0) @ r[:, 1], (v2 - v1) @ r[:, 1]))
        s.close()
    (a1, a2), (b1, b2) = out
    assert a1 == b1 and abs(a1) > 1.0
    assert abs(a2 / b2 - 0.1 / 0.64) < 2e-3 * 0.1 / 0.64, (a2, b2)
