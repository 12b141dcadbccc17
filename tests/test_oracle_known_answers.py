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
