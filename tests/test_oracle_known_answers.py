"""The CPU oracle against the reference's own known-answer tests and tables.

Pins the oracle before it is trusted as the checker of the HIP engine:
  * tests/physics_regressions.cu  - ball-hit window, split floor correction,
    dodge classification, goal recording, ball reset, steer staging,
    reset-after-done scope;
  * tests/turtle_recovery.cu      - 27 auto-flip cases;
  * src/RLConstants.cu, include/RLConstants.cuh, include/Physics/BoostPads.cuh
    tables (tests/golden/reference_tables.json) - kickoff spawn order and
    positions.
"""
import ctypes as C
import json
import math
from pathlib import Path

import numpy as np
import pytest

from abi import CAR_NAMES, SIM_NAMES
from oracle_py import OracleEnv, lib

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_tables.json").read_text())
CAR = {n: i for i, n in enumerate(CAR_NAMES)}
SIM = {n: i for i, n in enumerate(SIM_NAMES)}
F = C.c_float
SRC_NONE, SRC_BALL = 0, 3


def _f32(u):
    return np.asarray(u, np.uint32).view(np.float32)


def _i32(u):
    return int(np.asarray(u, np.uint32).view(np.int32))


# ---------------------------------------------------------------- physics_regressions.cu

@pytest.mark.parametrize("hit_tick,tick,expected", [(-1, 0, False), (99, 100, True), (98, 100, False),
                                                     (100, 100, False)])
def test_ball_hit_on_previous_tick(hit_tick, tick, expected):
    """physics_regressions.cu:20-23: a past kickoff hit must not disable floor depenetration."""
    assert bool(lib().oracle_ball_hit_prev_tick(hit_tick, tick)) is expected


@pytest.mark.parametrize("hit_age", [1, 2])
def test_floor_split_correction_only_without_recent_hit(hit_age):
    """physics_regressions.cu:25-36: depth 30 floor contact, vz = -5."""
    was_hit = lib().oracle_ball_hit_prev_tick(100 - hit_age, 100)
    push_z = lib().oracle_probe_ball_floor_split(30.0, -5.0, was_hit)
    if hit_age == 1:
        assert push_z == 0.0
    else:
        assert push_z > 0.0


DODGE_INPUTS = [(0.0, 1.0, -1.0), (0.0, -1.0, 1.0), (0.3, 0.3, 0.0), (-0.3, -0.3, 0.0), (0.0, 0.25, -0.25),
                (0.0, 0.24, -0.24), (0.0, 0.0, 0.0), (1.0, 0.0, 0.0)]
DODGE_FLIPS = [True, True, True, True, True, False, False, True]


@pytest.mark.parametrize("case", range(8))
def test_dodge_classification(case):
    """physics_regressions.cu:38-75: dodge vs double jump from (pitch, yaw, roll)."""
    pitch, yaw, roll = DODGE_INPUTS[case]
    flipped, double = C.c_int(), C.c_int()
    vel = (F * 3)()
    lib().oracle_probe_dodge(pitch, yaw, roll, C.byref(flipped), C.byref(double), vel)
    assert bool(flipped.value) is DODGE_FLIPS[case]
    assert bool(double.value) is (not DODGE_FLIPS[case])
    assert all(math.isfinite(v) for v in vel)
    if case < 2:  # yaw/roll cancel: a dodge with no impulse
        assert sum(v * v for v in vel) == 0.0


def test_steer_stage_lags_one_tick():
    """physics_regressions.cu:104-112: staged steer 0.25 moves to prev, zero input stages 0."""
    prev, cur = F(), F()
    lib().oracle_probe_steer_stage(0.25, C.byref(prev), C.byref(cur))
    assert prev.value == 0.25 and cur.value == 0.0


@pytest.mark.parametrize("sign", [-1, 1])
def test_goal_recorded_once_without_replacing_ball(sign):
    """physics_regressions.cu:77-98 at environment level: a ball inside the goal
    scores once for the attacking side; the ball state is not reset."""
    env = OracleEnv(1, 1, 1, 42)
    env.set_ball(np.array([[0.0, sign * 5500.0, 200.0]], np.float32),
                 np.array([[10.0, sign * 1000.0, -50.0]], np.float32), np.zeros((1, 3), np.float32))
    zero = np.zeros((1, 2, 7), np.float32)
    env.tick(zero, 1, 1)
    _, sim, tick = env.export_state()
    first_tick = _i32(sim[SIM["CARL_SIM_GOAL_TICK"], 0])
    for _ in range(3):
        env.tick(zero, 1, 1)
    _, sim, _ = env.export_state()
    assert _i32(sim[SIM["CARL_SIM_BLUE_SCORE"], 0]) + _i32(sim[SIM["CARL_SIM_ORANGE_SCORE"], 0]) == 1
    assert _i32(sim[SIM["CARL_SIM_LAST_SCORER"], 0]) == sign
    assert _i32(sim[SIM["CARL_SIM_GOAL_TICK"], 0]) == first_tick == tick
    ball_y = float(_f32(sim[SIM["CARL_SIM_BALL_POS_1"], 0]))
    assert sign * ball_y > 5215.5  # still past the goal line: not re-centred
    env.close()


def test_reset_clears_ball_integration_state():
    """physics_regressions.cu:100-102: resetBall clears integrationValid."""
    env = OracleEnv(2, 1, 1, 42)
    env.tick(np.zeros((2, 2, 7), np.float32), 1, 3)
    env.set_ball(np.array([[0.0, 0.0, 500.0]] * 2, np.float32), np.array([[0.0, 300.0, 0.0]] * 2, np.float32),
                 np.zeros((2, 3), np.float32))
    env.tick(np.zeros((2, 2, 7), np.float32), 1, 2)
    _, sim, _ = env.export_state()
    assert (sim[SIM["CARL_SIM_BALL_INT_VALID"]] == 1).all()
    env.reset()
    _, sim, _ = env.export_state()
    assert (sim[SIM["CARL_SIM_BALL_INT_VALID"]] == 0).all()
    env.close()


def test_reset_after_done_touches_only_the_finished_simulation():
    """physics_regressions.cu:114-150: state at tick 77, sim 0 scored."""
    env = OracleEnv(2, 1, 1, 42)
    car, sim, _ = env.export_state()
    car, sim = car.copy(), sim.copy()
    for s in range(2):
        for f in ("CARL_SIM_BLUE_SCORE", "CARL_SIM_ORANGE_SCORE", "CARL_SIM_LAST_SCORER", "CARL_SIM_GOAL_TICK",
                  "CARL_SIM_OVERTIME"):
            sim[SIM[f], s] = 0
        sim[SIM["CARL_SIM_EPISODE_TICKS"], s] = 10
        sim[SIM["CARL_SIM_LAST_TOUCH_TICK"], s] = 77
        sim[SIM["CARL_SIM_BALL_ARENA_CONTACT_TICK"], s] = 77
    for c in range(4):
        car[CAR["CARL_CAR_ARENA_CONTACT_TICK"], c] = 77
        for w in range(4):
            car[CAR[f"CARL_CAR_WHEEL_SOURCE_{w}"], c] = SRC_BALL
    sim[SIM["CARL_SIM_LAST_SCORER"], 0] = 1
    env.import_state(car, sim, 77)
    env.reset_dones()
    car, sim, _ = env.export_state()
    as_int = _i32
    assert as_int(sim[SIM["CARL_SIM_LAST_SCORER"], 0]) == 0
    assert as_int(sim[SIM["CARL_SIM_EPISODE_TICKS"], 0]) == 0
    assert as_int(sim[SIM["CARL_SIM_EPISODE_TICKS"], 1]) == 10
    assert as_int(sim[SIM["CARL_SIM_BALL_ARENA_CONTACT_TICK"], 0]) == -1
    assert as_int(sim[SIM["CARL_SIM_BALL_ARENA_CONTACT_TICK"], 1]) == 77
    for c in range(4):
        assert as_int(car[CAR["CARL_CAR_ARENA_CONTACT_TICK"], c]) == (-1 if c < 2 else 77)
        for w in range(4):
            assert as_int(car[CAR[f"CARL_CAR_WHEEL_SOURCE_{w}"], c]) == (SRC_NONE if c < 2 else SRC_BALL)
    env.close()


# ---------------------------------------------------------------- turtle_recovery.cu

def _quat_mul(a, b):
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return (aw * bx + ax * bw + ay * bz - az * by, aw * by - ax * bz + ay * bw + az * bx,
            aw * bz + ax * by - ay * bx + az * bw, aw * bw - ax * bx - ay * by - az * bz)


def _rotate(q, v):
    x, y, z, w = q
    u = np.array([x, y, z])
    v = np.asarray(v, dtype=np.float64)
    t = 2.0 * np.cross(u, v)
    return v + w * t + np.cross(u, t)


TURTLE = [(yaw, roll, roll_abs == 3.0) for yaw in (0.0, 0.7, math.pi / 2, math.pi, -math.pi / 2, -0.7)
          for roll, roll_abs in ((-3.0, 3.0), (3.0, 3.0), (-2.7, 2.7), (2.7, 2.7))]
TURTLE += [(0.0, 3.0, False, False, 1, (0.0, 0.0, 1.0)),   # no jump
           (0.0, 3.0, False, True, 0, (0.0, 0.0, 1.0)),    # no contact
           (0.0, 3.0, False, True, 1, (1.0, 0.0, 0.0))]    # wall contact


@pytest.mark.parametrize("case", TURTLE)
def test_turtle_recovery(case):
    """turtle_recovery.cu:31-93: upside-down cars recover only past |roll| 2.8 with
    jump held and one floor contact; the recovery torque opposes the roll."""
    yaw, roll, expected = case[:3]
    jump, contacts, normal = (case[3], case[4], case[5]) if len(case) > 3 else (True, 1, (0.0, 0.0, 1.0))
    tilt = (math.sin(roll / 2), 0.0, 0.0, math.cos(roll / 2))
    spin = (0.0, 0.0, math.sin(yaw / 2), math.cos(yaw / 2))
    q = _quat_mul(spin, tilt)
    quat = (F * 4)(*q)
    flipping, timer, ang = C.c_int(), F(), (F * 3)()
    lib().oracle_probe_autoflip(quat, int(jump), contacts, (F * 3)(*normal), C.byref(flipping), C.byref(timer), ang)
    ang = np.array(list(ang), np.float64)
    torque = float(ang @ _rotate(q, (1.0, 0.0, 0.0)))
    if expected:
        assert flipping.value and torque * roll < 0.0 and timer.value > 0.0
    else:
        assert not flipping.value and float(ang @ ang) == 0.0


# ---------------------------------------------------------------- reference tables

def test_kickoff_permutation_closed_form_matches_table():
    """The spawn-order table (src/RLConstants.cu) is generated, not stored: index p
    excludes spawn p/24 and takes the (p%24)-th lexicographic order of the rest."""
    table = GOLDEN["kickoff_permutations"]
    for p in range(120):
        assert [lib().oracle_kickoff_perm(p, s) for s in range(4)] == table[p], p


@pytest.mark.parametrize("n_blue,n_orange", [(1, 1), (2, 2), (3, 3), (4, 4), (1, 0)])
def test_kickoff_positions_follow_a_table_row(n_blue, n_orange):
    """Reset places blue car i at kickoff_locations[row[i]] for one row of the
    permutation table, orange cars at the point mirror, yaw + pi."""
    locs = GOLDEN["kickoff_locations"]
    rows = {tuple(r[:n_blue]) for r in GOLDEN["kickoff_permutations"]}
    env = OracleEnv(64, n_blue, n_orange, 3)
    car, _, _ = env.export_state()
    pos = _f32(car[CAR["CARL_CAR_POS_0"]:CAR["CARL_CAR_POS_2"] + 1]).T.reshape(64, n_blue + n_orange, 3)
    for s in range(64):
        spawn = []
        for i in range(n_blue):
            x, y = float(pos[s, i, 0]), float(pos[s, i, 1])
            match = [k for k, (lx, ly, _) in enumerate(locs) if lx == x and ly == y]
            assert len(match) == 1, (s, i, x, y)
            spawn.append(match[0])
        assert tuple(spawn) in rows
        for i in range(n_orange):
            ox, oy = float(pos[s, n_blue + i, 0]), float(pos[s, n_blue + i, 1])
            assert any(-lx == ox and -ly == oy for lx, ly, _ in locs)
        assert (pos[s, :, 2] == 17.0).all()
    env.close()


def test_boost_pad_table_matches_module_constants():
    import carl_amd

    pads = GOLDEN["boost_pads"]
    assert [list(p) for p in carl_amd.BOOST_PAD_POSITIONS] == [p[:3] for p in pads]
    assert [p[3] for p in pads] == [1] * 6 + [0] * 28  # big pads first


# ---------------------------------------------------------------- tests/test_resets.py behaviours

def reset_values(n, n_cars):
    """The reset inputs of tests/test_resets.py:28-72 (ball at z 800 moving +x,
    cars in a row at y -1000, last car demoed, boost 61, held-jump internals)."""
    ball_pos = np.zeros((n, 3), np.float32)
    ball_pos[:, 2] = 800
    ball_vel = np.zeros((n, 3), np.float32)
    ball_vel[:, 0] = 170
    car_pos = np.zeros((n, n_cars, 3), np.float32)
    car_pos[..., 0] = np.arange(n_cars) * 250 - 500
    car_pos[..., 1] = -1000
    car_pos[..., 2] = 17
    rot = np.zeros((n, n_cars, 4), np.float32)
    rot[..., 3] = 1
    demoed = np.zeros((n, n_cars), np.bool_)
    demoed[:, -1] = True
    internal = np.zeros((n, n_cars, 19), np.float32)
    internal[..., 3] = 1
    internal[..., 5] = 1
    return dict(ball_position=ball_pos, ball_velocity=ball_vel, ball_angular_velocity=np.zeros((n, 3), np.float32),
                car_position=car_pos, car_rotation=rot, car_velocity=np.zeros((n, n_cars, 3), np.float32),
                car_angular_velocity=np.zeros((n, n_cars, 3), np.float32), car_demoed=demoed,
                car_boost=np.full((n, n_cars), 61, np.float32), car_internal_state=internal,
                blue_score=np.full(n, 2, np.int32), orange_score=np.full(n, 1, np.int32),
                episode_ticks=np.full(n, 23, np.int32))


def test_restored_match_clock_enters_overtime_or_truncates():
    """tests/test_resets.py:351-381: max_ticks 4, overtime 2; a tied restored
    match enters overtime, the other truncates; overtime then expires."""
    env = OracleEnv(2, 1, 1, 7)
    env.set_param(0, 4)   # max_ticks
    env.set_param(1, 2)   # overtime_timeout_ticks
    v = reset_values(2, 2)
    v["orange_score"][0] = 2
    v["episode_ticks"][:] = 3
    env.apply_reset_state(**v)
    zero = np.zeros((2, 2, 7), np.float32)
    env.step(zero)
    assert env.get("dones").tolist() == [False, True]
    assert env.get("overtime").tolist() == [True, False]
    assert env.get("transition_episode_ticks").tolist() == [4, 4]
    for _ in range(2):
        env.step(zero)
    assert env.get("dones").tolist() == [True, False]
    assert bool(env.get("transition_overtime")[0])
    assert not env.get("overtime").any()
    env.close()


@pytest.mark.parametrize("masked", [False, True])
def test_restored_contacts_use_the_complete_scene(masked):
    """tests/test_resets.py:289-323: the top car's wheels rest on the bottom
    car (z 257 over z 200, both above the floor's reach): grounded only on top;
    a demoed restored car is never grounded."""
    env = OracleEnv(1, 1, 1, 7, previous_controls=True)
    v = reset_values(1, 2)
    v["car_position"][0] = [[0, 0, 257], [0, 0, 200]]
    v["car_demoed"][:] = False
    mask = np.ones(1, np.bool_) if masked else None
    env.apply_reset_state(**v, reset_mask=mask)
    state = env.get("state")
    cars = state[:, 9:9 + 2 * 22].reshape(1, 2, 22)
    np.testing.assert_array_equal(cars[..., :3], v["car_position"])
    np.testing.assert_array_equal(cars[..., 3:6], v["car_velocity"])
    assert cars[0, 0, 16] == 1.0 and cars[0, 1, 16] == 0.0   # OBS_ON_GROUND
    assert not cars[..., 21].any()                           # STATE_BALL_TOUCH
    v["car_demoed"][:, 0] = True
    env.apply_reset_state(**v, reset_mask=mask)
    assert env.get("obs")[0, 0, 9 + 16] == 0.0
    env.close()


def test_observation_layout_closed_form():
    """include/Physics/Observations.cuh:97-238 layout for a set state: ball
    block, ego car first, others after, orange cars seeing the field point
    mirrored (x, y negated), boost pads, all at the offsets of DLPack.h."""
    env = OracleEnv(1, 1, 1, 7)
    ball_p, ball_v, ball_w = [100.0, -200.0, 300.0], [10.0, 20.0, -30.0], [0.5, -0.25, 1.0]
    env.set_ball(np.array([ball_p], np.float32), np.array([ball_v], np.float32), np.array([ball_w], np.float32))
    cp = np.array([[[-500.0, 1000.0, 17.0], [700.0, -1500.0, 17.0]]], np.float32)
    cv = np.array([[[100.0, 0.0, 0.0], [0.0, -200.0, 0.0]]], np.float32)
    rot = np.zeros((1, 2, 4), np.float32)
    rot[..., 3] = 1
    env.set_car(cp, rot, cv, np.zeros((1, 2, 3), np.float32), np.zeros((1, 2), np.bool_),
                boost=np.array([[40.0, 70.0]], np.float32))
    obs = env.get("obs")[0]
    blue, orange = obs[0], obs[1]
    np.testing.assert_array_equal(blue[0:3], ball_p)
    np.testing.assert_array_equal(blue[3:6], ball_v)
    np.testing.assert_array_equal(blue[6:9], ball_w)
    np.testing.assert_array_equal(blue[9:12], cp[0, 0])           # ego = own car
    np.testing.assert_array_equal(blue[9 + 21:9 + 24], cp[0, 1])   # then the other car
    assert blue[9 + 15] == 40.0 and blue[9 + 21 + 15] == 70.0     # OBS_BOOST
    mirror = np.array([-1.0, -1.0, 1.0], np.float32)
    np.testing.assert_array_equal(orange[0:3], np.array(ball_p, np.float32) * mirror)
    np.testing.assert_array_equal(orange[3:6], np.array(ball_v, np.float32) * mirror)
    np.testing.assert_array_equal(orange[9:12], cp[0, 1] * mirror)  # orange ego first, mirrored
    np.testing.assert_array_equal(orange[9 + 21:9 + 24], cp[0, 0] * mirror)
    env.close()
