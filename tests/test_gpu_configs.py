"""HIP engine vs CPU oracle on the benchmark configurations' own workloads.

* the CPU reference configuration: one 1v1 arena driven by direct controls
  (independent steer and yaw, jump/boost/handbrake Bernoulli 0.5) held for 8
  ticks, for 10,000 ticks (tests/direct_controls.cu:35-76 restated, plus the
  full trajectory against the oracle);
* the one-car turtle-recovery case: a car upside down at z = 40, jump
  pressed again every 16 ticks (auto-flip starts on a press,
  include/Physics/Controls/Drive.cuh:134-178, Context.cuh:77) or held from
  the first tick;
* the creation options the other parity tests leave at their defaults:
  observations without orange inversion, with the previous controls, and
  normalised;
* a few steps of the three GPU configurations at their full sizes: 1v1 at
  65,536 simulations with frameskip 8, clustered 3v3 at 16,384, and 2v2 at
  131,072 with frameskip 1 and a quarter of the simulations reset from random
  states after every step.

Every comparison is bit-exact over every output buffer (actions included)
and every field of the persistent state.
"""
import numpy as np
import pytest

from carl_amd import workloads
from gpu_harness import Pair, gpu_state

pytestmark = pytest.mark.gpu

CONTINUOUS, DIRECT = 1, 2
CTRL_FIELDS = 34        # CARL_CAR_CTRL_THROTTLE .. CARL_CAR_CTRL_SLIDE: 8 planes
POS, ROT, AUTO_FLIPPING = 0, 9, 54


def _assert_clean(report, context):
    if report:
        pytest.fail(f"{context}:\n  " + "\n  ".join(report))


def _up_z(car_state: np.ndarray) -> np.ndarray:
    """z component of each car's up axis from the quaternion planes."""
    x, y = car_state[ROT].view(np.float32), car_state[ROT + 1].view(np.float32)
    return 1.0 - 2.0 * (x.astype(np.float64) ** 2 + y.astype(np.float64) ** 2)


def test_direct_controls_read_back_after_eight_ticks(gpu):
    """tests/direct_controls.cu:35-76: two cars' direct controls, held for 8
    ticks from a reset, are the controls the state holds afterwards (every
    field bit for bit, steer and yaw independent) and the positions stay
    finite; the whole state also matches the oracle."""
    p = Pair(1, 1, 1, seed=42, frameskip=1)
    c = np.zeros(2, workloads.CONTROLS_DTYPE)
    c[0] = (1.0, 0.5, -0.75, 0.25, -0.5, 0, 1, 0)
    c[1] = (-1.0, -0.25, 0.5, -0.5, 0.75, 1, 0, 1)
    p.tick(c, DIRECT, 8)
    car, _, _ = gpu_state(p.gpu)
    words = np.ascontiguousarray(c).view(np.uint32).reshape(2, 8)
    np.testing.assert_array_equal(car[CTRL_FIELDS:CTRL_FIELDS + 8].T, words)
    assert np.isfinite(car[POS:POS + 3].view(np.float32)).all()
    _assert_clean(p.state_mismatches(), "state after 8 direct-control ticks")
    p.close()


def test_direct_controls_10000_ticks_one_arena(gpu):
    """The CPU reference workload on the engine: 1 arena, 1v1, seeded direct
    controls resampled every 8 ticks, 10,000 ticks, compared after every
    8-tick hold."""
    rng = np.random.default_rng(2024)
    p = Pair(1, 1, 1, seed=0, frameskip=1)
    for hold in range(10_000 // 8):
        p.tick(workloads.random_direct_controls(rng, 2), DIRECT, 8)
        report = p.state_mismatches()
        if report:
            pytest.fail(f"state after tick {8 * (hold + 1)}:\n  " + "\n  ".join(report))
    car, _, tick = gpu_state(p.gpu)
    assert tick == 10_000
    assert np.isfinite(car[POS:POS + 3].view(np.float32)).all()
    p.close()


@pytest.mark.parametrize("n_blue,n_orange", [(1, 1), (2, 2), (3, 3)])
def test_direct_controls_many_arenas(gpu, n_blue, n_orange):
    """Direct controls across whole waves of cars, from random states: every
    lane decodes its own controls."""
    rng = np.random.default_rng(40 + n_blue)
    n, nc = 192, n_blue + n_orange
    p = Pair(n, n_blue, n_orange, seed=5, frameskip=1)
    odd = np.arange(1, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(odd), nc), simulation_indices=odd.astype(np.int64))
    for hold in range(30):
        p.tick(workloads.random_direct_controls(rng, n * nc), DIRECT, 8)
        _assert_clean(p.state_mismatches(), f"{n_blue}v{n_orange} state after hold {hold}")
    p.close()


def _turtle_state(yaws: np.ndarray, rolls: np.ndarray) -> dict[str, np.ndarray]:
    """One car per arena, upside down at z = 40: rotation = yaw about z
    composed with the roll about the car's forward axis; ball parked away."""
    n = len(yaws)
    hz, hr = yaws / 2, rolls / 2
    # (0, 0, sin hz, cos hz) * (sin hr, 0, 0, cos hr)
    rot = np.stack([np.cos(hz) * np.sin(hr), np.sin(hz) * np.sin(hr), np.sin(hz) * np.cos(hr),
                    np.cos(hz) * np.cos(hr)], axis=-1)
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    car_pos = np.stack([np.linspace(-3000, 3000, n), np.full(n, -1500.0), np.full(n, 40.0)], axis=-1)
    return {
        "ball_position": f32(np.tile([0.0, 2500.0, 93.15], (n, 1))),
        "ball_velocity": f32(np.zeros((n, 3))), "ball_angular_velocity": f32(np.zeros((n, 3))),
        "car_position": f32(car_pos[:, None, :]), "car_rotation": f32(rot[:, None, :]),
        "car_velocity": f32(np.zeros((n, 1, 3))), "car_angular_velocity": f32(np.zeros((n, 1, 3))),
        "car_demoed": np.zeros((n, 1), dtype=np.bool_),
    }


@pytest.mark.parametrize("jump", ["pressed_every_16_ticks", "held"])
def test_turtle_recovery_one_car(gpu, jump):
    """Config 4's extra case: n_blue = 1, n_orange = 0, the car upside down at
    z = 40 at six yaws and rolls of +-3 and +-2.7 rad, ticked per tick
    against the oracle for 2 s.  With jump pressed again every 16 ticks the
    rolls of +-3 rad recover through the auto-flip (up axis z > 0.9 within
    1 s, as tests/turtle_recovery.cu:68-71 expects the flip to start); held
    from the first tick, the press comes before the roof touches the floor,
    so the car must stay on its roof, at rest and finite."""
    yaws = np.array([0.0, 0.7, np.pi / 2, np.pi, -np.pi / 2, -0.7])
    rolls = np.array([3.0, -3.0, 2.7, -2.7])
    yy, rr = np.meshgrid(yaws, rolls)
    yy, rr = yy.reshape(-1), rr.reshape(-1)
    n = len(yy)
    p = Pair(n, 1, 0, seed=42, frameskip=1)
    p.apply_reset_state(_turtle_state(yy, rr))
    _assert_clean(p.state_mismatches(), "state after the upside-down reset")
    a = np.zeros((n, 1, 7), np.float32)
    recovered_by = np.full(n, -1)
    for t in range(240):
        a[..., 6] = 1.0 if jump == "held" else float((t // 8) % 2)
        p.tick(a, CONTINUOUS, 1)
        _assert_clean(p.state_mismatches(), f"state after tick {t + 1}")
        car, _, _ = gpu_state(p.gpu)
        up = _up_z(car)
        recovered_by[(recovered_by < 0) & (up > 0.9)] = t + 1
    car, _, _ = gpu_state(p.gpu)
    assert np.isfinite(car[:POS + 13].view(np.float32)).all()
    steep = np.abs(rr) == 3.0
    if jump == "held":
        assert (recovered_by[steep] < 0).all(), recovered_by
        assert (_up_z(car)[steep] < -0.9).all()
        assert (car[AUTO_FLIPPING] == 0).all()
    else:
        assert ((recovered_by[steep] > 0) & (recovered_by[steep] <= 120)).all(), recovered_by
    p.close()


@pytest.mark.parametrize("n_blue,n_orange,invert,normalize,previous,discrete", [
    (1, 1, False, False, True, False),
    (2, 2, False, True, True, True),
    (3, 2, True, False, True, True),
    (1, 1, False, True, False, False),
    (2, 1, False, False, False, True),
    (3, 3, True, True, False, False),
    (4, 3, True, True, True, False),
])
def test_creation_options_stepping(gpu, n_blue, n_orange, invert, normalize, previous, discrete):
    """Observations without orange inversion, normalised, with the previous
    controls, over many steps from kickoffs and random states."""
    rng = np.random.default_rng(60 + 7 * n_blue + n_orange)
    n, nc = 80, n_blue + n_orange
    p = Pair(n, n_blue, n_orange, seed=19, frameskip=4, invert_orange=invert, normalize=normalize,
             previous_controls=previous)
    odd = np.arange(1, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(odd), nc), simulation_indices=odd.astype(np.int64))
    p.set_param("max_ticks", 40)
    for step in range(16):
        if discrete:
            p.step_discrete(workloads.random_discrete_actions(rng, n, nc))
        else:
            p.step_continuous(workloads.random_continuous_actions(rng, n, nc))
        ctx = f"{n_blue}v{n_orange} invert={invert} normalize={normalize} previous={previous} step {step}"
        _assert_clean(p.state_mismatches(), ctx + " state")
        _assert_clean(p.output_mismatches(), ctx + " outputs")
    p.close()


@pytest.mark.timeout(600)
def test_full_size_1v1_65536_frameskip_8(gpu):
    """The headline workload at its own size: half kickoffs, half random
    states, random continuous actions, 3 steps of 8 ticks."""
    rng = np.random.default_rng(65536)
    n = 65536
    p = Pair(n, 1, 1, seed=1, frameskip=8)
    odd = np.arange(1, n, 2)
    p.apply_reset_state(workloads.random_reset_state(rng, len(odd), 2), simulation_indices=odd.astype(np.int64))
    for step in range(3):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 2))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


@pytest.mark.timeout(600)
def test_full_size_3v3_16384_clustered(gpu):
    """3v3 at 16,384 simulations, every car within 500 uu of the ball."""
    rng = np.random.default_rng(16384)
    n = 16384
    p = Pair(n, 3, 3, seed=2, frameskip=8)
    p.apply_reset_state(workloads.random_reset_state(rng, n, 6, cluster_radius=500.0))
    for step in range(3):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 6))
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()


@pytest.mark.timeout(600)
def test_full_size_2v2_131072_per_tick_masked_resets(gpu):
    """2v2 at 131,072 simulations, frameskip 1, a seeded quarter of the
    simulations reset from random states through the masked path after
    every step."""
    rng = np.random.default_rng(131072)
    n = 131072
    p = Pair(n, 2, 2, seed=3, frameskip=1)
    for step in range(3):
        p.step_continuous(workloads.random_continuous_actions(rng, n, 4))
        mask = rng.uniform(0, 1, n) < 0.25
        p.apply_reset_state(workloads.random_reset_state(rng, n, 4), reset_mask=mask)
        _assert_clean(p.state_mismatches(), f"state after step {step}")
        _assert_clean(p.output_mismatches(), f"outputs after step {step}")
    p.close()
