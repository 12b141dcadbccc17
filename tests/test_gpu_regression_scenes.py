"""The reference's device-side known-answer scenes (tests/physics_regressions.cu:20-150),
set up as engine state through import_state and run through the engine's own
ticks, resets and done handling.  Each scene checks the reference's
expectation on the engine's state and the whole state against the oracle,
bit for bit.

The reference drives single device functions (solveBallArenaContacts,
tryStartDodge, detectGoal, resetBall, updateSteer, resetAfterDone) on a
hand-built GameState; here the same situations are states the whole tick
passes through:
  * floor depenetration and the ball-hit window: a ball 30 uu into the floor
    falling at 5 uu/s, last touched one or two ticks before the tick;
  * dodge versus double jump: a car in the air after its first jump presses
    jump with each of the reference's eight stick inputs;
  * a ball inside either goal scores once and is not moved back;
  * a reset clears the ball's integration state;
  * a staged steer angle is consumed by the next tick, and a zero input
    stages zero;
  * finishing one simulation at tick 77 resets only its own contact state.
"""
import numpy as np
import pytest

from abi import CAR_NAMES, SIM_NAMES
from gpu_harness import Pair, dev, gpu_state

pytestmark = pytest.mark.gpu

CAR = {n: i for i, n in enumerate(CAR_NAMES)}
SIM = {n: i for i, n in enumerate(SIM_NAMES)}
CONTINUOUS, DIRECT = 1, 2
SRC_NONE, SRC_BALL = 0, 3
BALL_RADIUS = 91.25


def f32bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).view(np.uint32)


def as_f32(u) -> np.ndarray:
    return np.asarray(u, np.uint32).view(np.float32)


def as_i32(u) -> np.ndarray:
    return np.asarray(u, np.uint32).view(np.int32)


def agree(pair: Pair, context: str):
    report = pair.state_mismatches()
    if report:
        pytest.fail(f"{context}: engine and oracle differ:\n  " + "\n  ".join(report))


def parked_cars(pair: Pair, n_cars: int):
    """Every car parked at rest far from the field centre, on its wheels."""
    n = pair.n_sim
    pos = np.zeros((n, n_cars, 3), np.float32)
    pos[..., 0] = np.linspace(-3000, 3000, n_cars)[None, :]
    pos[..., 1] = -3500.0
    pos[..., 2] = 17.0
    rot = np.zeros((n, n_cars, 4), np.float32)
    rot[..., 3] = 1.0
    zero = np.zeros((n, n_cars, 3), np.float32)
    demoed = np.zeros((n, n_cars), np.bool_)
    pair.gpu.set_car(dev(pos), dev(rot), dev(zero), dev(zero), dev(demoed))
    pair.cpu.set_car(pos, rot, zero, zero, demoed)


def set_ball(pair: Pair, pos, vel, ang=None):
    n = pair.n_sim
    pos = np.broadcast_to(np.asarray(pos, np.float32), (n, 3)).copy()
    vel = np.broadcast_to(np.asarray(vel, np.float32), (n, 3)).copy()
    ang = np.zeros((n, 3), np.float32) if ang is None else np.broadcast_to(np.asarray(ang, np.float32), (n, 3)).copy()
    pair.gpu.set_ball(dev(pos), dev(vel), dev(ang))
    pair.cpu.set_ball(pos, vel, ang)


def test_floor_depenetration_waits_one_tick_after_a_ball_hit(gpu):
    """physics_regressions.cu:20-36: a ball 30 uu deep in the floor, falling at
    5 uu/s.  Touched by a car on the tick just before, it gets no split
    position correction; touched two ticks before (or never), it is pushed
    out of the floor.  Simulation 0 was hit one tick before, 1 two ticks
    before, 2 never; the cars are parked far away so nothing touches the ball
    during the tick."""
    p = Pair(3, 1, 1, seed=42, frameskip=1)
    parked_cars(p, 2)
    # a spot inside one floor triangle: the ball's single contact, as in the
    # reference scene (with several contacts the correction never waits)
    set_ball(p, (-2000.0, -2000.0, BALL_RADIUS - 30.0), (0.0, 0.0, -5.0))
    car, sim, tick = gpu_state(p.gpu)
    car, sim = car.copy(), sim.copy()
    tick = 99                                      # the next tick is tick 100
    car[CAR["CARL_CAR_BALL_HIT_TICK"]] = np.uint32(0xFFFFFFFF)             # -1: never hit
    car[CAR["CARL_CAR_BALL_HIT_TICK"], 0] = np.uint32(99)    # simulation 0, car 0: the tick before
    car[CAR["CARL_CAR_BALL_HIT_TICK"], 3] = np.uint32(98)    # simulation 1, car 1: two ticks before
    p.import_state(car, sim, tick)
    agree(p, "imported state")
    p.tick(np.zeros((3, 2, 7), np.float32), CONTINUOUS, 1)
    agree(p, "after the tick")
    _, sim, tick = gpu_state(p.gpu)
    assert tick == 100
    z = as_f32(sim[SIM["CARL_SIM_BALL_POS_2"]]).astype(np.float64)
    # the same contact solve in all three; only the split push differs: the
    # ball hit on the tick before stays where it was (the contact stops its
    # fall), the others are pushed out of the floor
    assert z[0] == np.float32(BALL_RADIUS - 30.0), z
    assert z[1] > z[0] and z[2] > z[0], z
    assert z[1] == z[2], z
    p.close()


# physics_regressions.cu:38-75: (pitch, yaw, roll) and whether a dodge starts
DODGE_INPUTS = [(0.0, 1.0, -1.0), (0.0, -1.0, 1.0), (0.3, 0.3, 0.0), (-0.3, -0.3, 0.0), (0.0, 0.25, -0.25),
                (0.0, 0.24, -0.24), (0.0, 0.0, 0.0), (1.0, 0.0, 0.0)]
DODGE_FLIPS = [True, True, True, True, True, False, False, True]


def test_second_jump_is_a_dodge_or_a_double_jump_by_stick_input(gpu):
    """physics_regressions.cu:38-75: one car per simulation, in the air at
    rest 0.2 s after its first jump (jump released since), presses jump with
    each of the eight stick inputs: past the deadzone the press is a dodge
    (has flipped), inside it a double jump; yaw and roll that cancel with no
    pitch give a dodge without an impulse, so the car keeps no horizontal
    velocity, while the other dodges push it along the floor plane."""
    n = len(DODGE_INPUTS)
    p = Pair(n, 1, 0, seed=42, frameskip=1)
    pos = np.zeros((n, 1, 3), np.float32)
    pos[:, 0, 0] = np.linspace(-2000, 2000, n)
    pos[:, 0, 2] = 600.0
    rot = np.zeros((n, 1, 4), np.float32)
    rot[..., 3] = 1.0
    zero = np.zeros((n, 1, 3), np.float32)
    demoed = np.zeros((n, 1), np.bool_)
    p.gpu.set_car(dev(pos), dev(rot), dev(zero), dev(zero), dev(demoed))
    p.cpu.set_car(pos, rot, zero, zero, demoed)
    set_ball(p, (0.0, 3000.0, 93.0), (0.0, 0.0, 0.0))
    car, sim, tick = gpu_state(p.gpu)
    car, sim = car.copy(), sim.copy()
    for name, value in (("CARL_CAR_ON_GROUND", 0), ("CARL_CAR_HAS_JUMPED", 1), ("CARL_CAR_IS_JUMPING", 0),
                        ("CARL_CAR_LAST_JUMP", 0), ("CARL_CAR_HAS_DOUBLE_JUMPED", 0), ("CARL_CAR_HAS_FLIPPED", 0),
                        ("CARL_CAR_IS_FLIPPING", 0)):
        car[CAR[name]] = np.uint32(value)
    for name, value in (("CARL_CAR_AIR_TIME", 0.25), ("CARL_CAR_AIR_TIME_SINCE_JUMP", 0.2),
                        ("CARL_CAR_JUMP_TIME", 0.2)):
        car[CAR[name]] = f32bits(value)
    p.import_state(car, sim, tick)
    c = np.zeros(n, dtype=[("throttle", "<f4"), ("steer", "<f4"), ("yaw", "<f4"), ("pitch", "<f4"),
                           ("roll", "<f4"), ("jump", "<i4"), ("boost", "<i4"), ("slide", "<i4")])
    for i, (pitch, yaw, roll) in enumerate(DODGE_INPUTS):
        c[i] = (0.0, 0.0, yaw, pitch, roll, 1, 0, 0)
    p.tick(c, DIRECT, 1)
    agree(p, "after the press")
    car, _, _ = gpu_state(p.gpu)
    flipped = as_i32(car[CAR["CARL_CAR_HAS_FLIPPED"]]) != 0
    double = as_i32(car[CAR["CARL_CAR_HAS_DOUBLE_JUMPED"]]) != 0
    np.testing.assert_array_equal(flipped, DODGE_FLIPS)
    np.testing.assert_array_equal(double, ~np.array(DODGE_FLIPS))
    vel = as_f32(car[CAR["CARL_CAR_VEL_0"]:CAR["CARL_CAR_VEL_0"] + 3]).T.astype(np.float64)
    assert np.isfinite(vel).all()
    # yaw + roll = 0 and no pitch: a dodge with no impulse (inputs 0, 1, 4)
    assert (vel[[0, 1, 4], :2] == 0.0).all(), vel
    assert (np.abs(vel[[2, 3, 7], :2]).sum(axis=1) > 0.0).all(), vel
    p.close()


@pytest.mark.parametrize("sign", [-1, 1])
def test_goal_scores_once_and_leaves_the_ball(gpu, sign):
    """physics_regressions.cu:77-98: a ball inside the goal scores once for the
    attacking side; later ticks keep the score and the goal tick, and the
    ball is not moved back into play."""
    p = Pair(1, 1, 1, seed=42, frameskip=1)
    set_ball(p, (0.0, sign * 5500.0, 200.0), (10.0, sign * 1000.0, -50.0))
    zero = np.zeros((1, 2, 7), np.float32)
    p.tick(zero, CONTINUOUS, 1)
    _, sim, tick = gpu_state(p.gpu)
    goal_tick = int(as_i32(sim[SIM["CARL_SIM_GOAL_TICK"], 0]))
    assert goal_tick == tick
    p.tick(zero, CONTINUOUS, 3)
    agree(p, "after the goal")
    _, sim, _ = gpu_state(p.gpu)
    score = int(as_i32(sim[SIM["CARL_SIM_BLUE_SCORE"], 0])) + int(as_i32(sim[SIM["CARL_SIM_ORANGE_SCORE"], 0]))
    assert score == 1
    assert int(as_i32(sim[SIM["CARL_SIM_LAST_SCORER"], 0])) == sign
    assert int(as_i32(sim[SIM["CARL_SIM_GOAL_TICK"], 0])) == goal_tick
    assert sign * float(as_f32(sim[SIM["CARL_SIM_BALL_POS_1"], 0])) > 5215.5
    p.close()


def test_reset_clears_the_ball_integration_state(gpu):
    """physics_regressions.cu:100-102: after ticks the ball's integration state
    is valid; a reset clears it."""
    p = Pair(2, 1, 1, seed=42, frameskip=1)
    zero = np.zeros((2, 2, 7), np.float32)
    p.tick(zero, CONTINUOUS, 3)
    set_ball(p, (0.0, 0.0, 500.0), (0.0, 300.0, 0.0))
    p.tick(zero, CONTINUOUS, 2)
    _, sim, _ = gpu_state(p.gpu)
    assert (sim[SIM["CARL_SIM_BALL_INT_VALID"]] == 1).all()
    p.gpu.reset()
    p.cpu.reset()
    agree(p, "after the reset")
    _, sim, _ = gpu_state(p.gpu)
    assert (sim[SIM["CARL_SIM_BALL_INT_VALID"]] == 0).all()
    p.close()


def test_staged_steer_is_consumed_by_the_next_tick(gpu):
    """physics_regressions.cu:104-112: a staged steer angle of 0.25 is the one
    the next tick steers with, and that tick stages the new input (zero).
    Simulation 0 has 0.25 staged, simulation 1 nothing; both cars roll
    forward on the floor with no input: after one tick both stage 0, and only
    the first has turned."""
    p = Pair(2, 1, 0, seed=42, frameskip=1)
    pos = np.array([[[-1000.0, 0.0, 17.0]], [[1000.0, 0.0, 17.0]]], np.float32)
    rot = np.zeros((2, 1, 4), np.float32)
    rot[..., 3] = 1.0
    vel = np.array([[[1000.0, 0.0, 0.0]], [[1000.0, 0.0, 0.0]]], np.float32)
    zero = np.zeros((2, 1, 3), np.float32)
    demoed = np.zeros((2, 1), np.bool_)
    p.gpu.set_car(dev(pos), dev(rot), dev(vel), dev(zero), dev(demoed))
    p.cpu.set_car(pos, rot, vel, zero, demoed)
    set_ball(p, (0.0, 3000.0, 93.0), (0.0, 0.0, 0.0))
    # settle onto the wheels first, so the steer acts through wheel contact
    p.tick(np.zeros((2, 1, 7), np.float32), CONTINUOUS, 30)
    car, sim, tick = gpu_state(p.gpu)
    assert (as_i32(car[CAR["CARL_CAR_ON_GROUND"]]) != 0).all()
    car = car.copy()
    car[CAR["CARL_CAR_STEER_STAGE"], 0] = f32bits(0.25)
    car[CAR["CARL_CAR_STEER_STAGE"], 1] = f32bits(0.0)
    p.import_state(car, sim, tick)
    p.tick(np.zeros((2, 1, 7), np.float32), CONTINUOUS, 1)
    agree(p, "after the tick")
    car, _, _ = gpu_state(p.gpu)
    assert (as_f32(car[CAR["CARL_CAR_STEER_STAGE"]]) == 0.0).all()
    yaw_rate = as_f32(car[CAR["CARL_CAR_ANG_2"]])
    assert yaw_rate[0] != yaw_rate[1], yaw_rate
    p.close()


def test_finished_simulation_resets_only_its_own_contact_state(gpu):
    """physics_regressions.cu:114-150: at tick 77 simulation 0 has scored
    (last scorer set), simulation 1 plays on; both have ten episode ticks,
    the ball and every car touched at tick 77 and every wheel on the ball.
    Resetting the finished simulations clears simulation 0's scorer, episode
    clock, ball contact tick, its cars' contact ticks and wheel sources, and
    leaves simulation 1's untouched."""
    p = Pair(2, 1, 1, seed=42, frameskip=1)
    car, sim, _ = gpu_state(p.gpu)
    car, sim = car.copy(), sim.copy()
    for s in range(2):
        for name in ("CARL_SIM_BLUE_SCORE", "CARL_SIM_ORANGE_SCORE", "CARL_SIM_LAST_SCORER", "CARL_SIM_GOAL_TICK",
                     "CARL_SIM_OVERTIME"):
            sim[SIM[name], s] = 0
        sim[SIM["CARL_SIM_EPISODE_TICKS"], s] = 10
        sim[SIM["CARL_SIM_LAST_TOUCH_TICK"], s] = 77
        sim[SIM["CARL_SIM_BALL_ARENA_CONTACT_TICK"], s] = 77
    for c in range(4):
        car[CAR["CARL_CAR_ARENA_CONTACT_TICK"], c] = 77
        for w in range(4):
            car[CAR[f"CARL_CAR_WHEEL_SOURCE_{w}"], c] = SRC_BALL
    sim[SIM["CARL_SIM_LAST_SCORER"], 0] = 1
    p.import_state(car, sim, 77)
    p.gpu.reset_dones()
    p.cpu.reset_dones()
    agree(p, "after the done reset")
    car, sim, _ = gpu_state(p.gpu)
    assert int(as_i32(sim[SIM["CARL_SIM_LAST_SCORER"], 0])) == 0
    assert list(as_i32(sim[SIM["CARL_SIM_EPISODE_TICKS"]])) == [0, 10]
    assert list(as_i32(sim[SIM["CARL_SIM_BALL_ARENA_CONTACT_TICK"]])) == [-1, 77]
    assert list(as_i32(car[CAR["CARL_CAR_ARENA_CONTACT_TICK"]])) == [-1, -1, 77, 77]
    for w in range(4):
        assert list(as_i32(car[CAR[f"CARL_CAR_WHEEL_SOURCE_{w}"]])) == [SRC_NONE, SRC_NONE, SRC_BALL, SRC_BALL]
    p.close()
