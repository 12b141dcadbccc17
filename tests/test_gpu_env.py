"""The drop-in surface on the GPU: carl._carl.Env and CARLTorchVectorEnv.

The behaviours the reference checks in tests/test_gpu.py,
test_gpu_backend.py, test_stream_handoff.py and the ResetTests of
test_resets.py:217-529, checked here with this suite's own structure (a pair
of environments driven in lockstep, reset routes as interchangeable
functions, invalid inputs as named mutations of valid ones, match-clock
expectations as a timeline) and the reference's inputs and expected values:
  * a wrapper step returns typed, finite tensors of the advertised shapes;
  * max_ticks = 16 truncates within 8 steps; the reset observation is not
    overwritten by later steps;
  * a run on a side stream without host synchronisation sees the same
    frames as a synchronised one;
  * apply_reset_state equals the individual setters, leaves other
    simulations and the transition buffers alone, and the two
    environments stay equal for 8 more steps; a masked reset equals the
    indexed reset of the same rows;
  * restored cars get their contacts from the whole restored scene;
  * every malformed input is refused before anything changes;
  * a restored match clock enters overtime or truncates on time;
  * inputs made on other streams, as temporaries or capsules, survive until
    the engine has read them, and destroying the environment waits for them;
  * the wrapper keeps terminal successors and defers episode reports
    without host synchronisation.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import partial
from itertools import product

import pytest
import torch

import carl
from carl.gymnasium.state import CARLObservation
from carl.gymnasium.torch import CARLTorchVectorEnv
import reset_fixtures as fixtures
from reset_fixtures import NoHostSync, typed_reset_state

pytestmark = pytest.mark.gpu

# the buffers a reset may rewrite, and the step's transition buffers it must not touch
LIVE = ("obs", "state", "score_difference", "episode_ticks", "overtime")
STEP = ("transition_obs", "transition_state", "transition_score_difference", "transition_episode_ticks",
        "transition_overtime", "rewards", "dones")


def capture(env, names) -> dict[str, torch.Tensor]:
    """Copies of the named output buffers once the environment's stream has
    produced them."""
    torch.cuda.current_stream().wait_stream(torch.cuda.ExternalStream(env.stream))
    copies = {name: torch.from_dlpack(getattr(env, f"get_{name}")()).clone() for name in names}
    torch.cuda.synchronize()
    return copies


def identical(a, b):
    torch.testing.assert_close(a, b, rtol=0, atol=0)


def expect_typed(t, shape, dtype):
    assert isinstance(t, torch.Tensor), type(t)
    assert t.is_cuda and t.dtype == dtype and tuple(t.shape) == tuple(shape), (t.device, t.dtype, t.shape)
    assert bool(torch.isfinite(t.float()).all())


def zero_actions(n_sim, n_cars):
    return torch.zeros((n_sim, n_cars, 7), device="cuda")


class Lockstep:
    """Two native environments of the same configuration, stepped together."""

    def __init__(self, n_sim, team, seed=7):
        self.a = carl.Env(n_sim, team, team, seed, previous_controls=True)
        self.b = carl.Env(n_sim, team, team, seed, previous_controls=True)
        self.n_sim, self.n_cars = n_sim, 2 * team

    def set_no_touch_timeout(self, ticks):
        self.a.no_touch_timeout_ticks = self.b.no_touch_timeout_ticks = ticks

    def step(self, actions):
        self.a.step_continuous(actions)
        self.b.step_continuous(actions)

    def assert_equal(self, names):
        got, want = capture(self.b, names), capture(self.a, names)
        for name in names:
            identical(got[name], want[name])


# --------------------------------------------------------------- reset routes

def reset_by_setters(env, values, indices):
    """The restore through the separate setters, in the reference order."""
    env.reset_boost_pads(indices)
    env.set_ball(values["ball_position"], values["ball_velocity"], values["ball_angular_velocity"],
                 simulation_indices=indices)
    env.set_car(values["car_position"], values["car_rotation"], values["car_velocity"],
                values["car_angular_velocity"], values["car_demoed"], boost=values.get("car_boost"),
                internal_state=values.get("car_internal_state"), simulation_indices=indices)
    if "blue_score" in values:
        env.set_match_state(values["blue_score"], values["orange_score"], values["episode_ticks"],
                            simulation_indices=indices)


def reset_combined(env, values, indices):
    env.apply_reset_state(**values, simulation_indices=indices)


# ------------------------------------------------------------ tests/test_gpu.py

def test_wrapper_step_returns_typed_outputs(gpu):
    env = CARLTorchVectorEnv(n_sim=1, n_blue=1, n_orange=1, frameskip=1, discrete_actions=True, synchronize=True)
    try:
        first = env.reset()
        shapes = {"obs": env.observation_space.shape, "ball": (env.n_envs, 3), "cars": (env.n_envs, env.n_cars, 3)}
        assert isinstance(first, CARLObservation)
        for t, shape in ((first, shapes["obs"]), (first.ball.position, shapes["ball"]),
                         (first.cars.position, shapes["cars"])):
            expect_typed(t, shape, torch.float32)
        act = torch.zeros((env.n_envs, len(carl.ACTION_NVECS)), dtype=torch.long, device=env.device)
        obs, reward, terminated, truncated, info = env.step(act)
        assert isinstance(obs, CARLObservation) and isinstance(info, dict)
        expect_typed(obs, shapes["obs"], torch.float32)
        expect_typed(reward, (env.n_envs,), torch.float32)
        for flags in (terminated, truncated):
            expect_typed(flags, (env.n_envs,), torch.bool)
    finally:
        env.close()


# ---------------------------------------------------- tests/test_gpu_backend.py

@pytest.mark.parametrize("n_sim,discrete", [(17, False), (17, True), (8192, False)])
def test_short_episodes_truncate_and_keep_the_reset_observation(gpu, n_sim, discrete):
    env = CARLTorchVectorEnv(n_sim=n_sim, n_blue=1, n_orange=1, discrete_actions=discrete, max_ticks=16,
                             overtime_timeout_ticks=8)
    act = torch.zeros(env.action_space.shape, dtype=torch.int64 if discrete else torch.float32, device=env.device)
    start = env.reset()
    kept = start.clone()
    expect_typed(start, env.observation_space.shape, torch.float32)
    assert torch.from_dlpack(env._env.get_obs()).__dlpack_device__() == (10, 0)   # ROCm device 0
    truncations = 0
    for _ in range(8):
        obs, reward, terminated, truncated, _ = env.step(act)
        expect_typed(obs, env.observation_space.shape, torch.float32)
        expect_typed(reward, (env.n_envs,), torch.float32)
        expect_typed(terminated, (env.n_envs,), torch.bool)
        expect_typed(truncated, (env.n_envs,), torch.bool)
        truncations += int(truncated.sum())
    env.close()
    assert truncations > 0
    identical(start, kept)


# --------------------------------------------------- tests/test_stream_handoff.py

def _frames(synchronize):
    """Eight steps with a ball placement and a reset halfway, every frame
    copied (the ball set 800 uu up, then a slow kernel on the caller's
    stream before the engine's buffer is read)."""
    env = CARLTorchVectorEnv(n_sim=4, n_blue=1, n_orange=1, seed=7, synchronize=synchronize)
    act = torch.zeros(env.action_space.shape, device=env.device)
    frames = [env.reset().clone()]
    for step in range(8):
        if step != 4:
            frames.append(env.step(act)[0].clone())
            continue
        zero = torch.zeros((env.n_sim, 3), device=env.device)
        lifted = zero.clone()
        lifted[:, 2] = 800.0
        env.set_ball(lifted, zero, zero)
        torch.cuda._sleep(50_000_000)
        frames.append(torch.from_dlpack(env._env.get_obs()).clone())
        frames.append(env.reset().clone())
    env.close()
    return frames


def test_unsynchronised_side_stream_sees_the_synchronised_frames(gpu):
    want = _frames(synchronize=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = _frames(synchronize=False)
    torch.cuda.synchronize()
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-4)


# ------------------------------------------------------------ tests/test_resets.py

@dataclass(frozen=True)
class Restore:
    team: int                    # cars per team
    rows: tuple | None           # simulation indices (None: every simulation)
    full: bool                   # boost, internal state and match fields supplied

    def inputs(self):
        count = 3 if self.rows is None else len(self.rows)
        v = fixtures.reset_inputs(count, 2 * self.team, match=self.full, internal=self.full, device="cuda")
        if not self.full:
            del v["car_boost"]
            v["car_demoed"] = v["car_demoed"].int()     # int32 demolished flags
        return v

    def indices(self):
        return None if self.rows is None else torch.tensor(self.rows, device="cuda", dtype=torch.int64)


RESTORES = [Restore(t, r, f) for t, r, f in product((1, 2, 3), ((), (2, 0), None), (False, True))]


@pytest.mark.parametrize("case", RESTORES, ids=lambda c: f"team{c.team}-rows{c.rows}-full{c.full}")
def test_combined_reset_equals_the_setters(gpu, case):
    envs = Lockstep(3, case.team)
    values, indices = case.inputs(), case.indices()
    jump = zero_actions(3, 2 * case.team)
    jump[..., 6] = 1.0
    # one step that ends every episode (no touch within a tick), so the
    # transition buffers hold known rows
    envs.set_no_touch_timeout(1)
    envs.step(jump)
    start = capture(envs.b, LIVE + STEP)
    envs.set_no_touch_timeout(0)
    for _ in range(2):
        reset_by_setters(envs.a, values, indices)
        reset_combined(envs.b, values, indices)
        now = capture(envs.b, STEP)
        for name in STEP:
            identical(now[name], start[name])
        envs.assert_equal(("obs", "state"))
    end = capture(envs.b, LIVE)
    chosen = set(range(3)) if case.rows is None else set(case.rows)
    others = [s for s in range(3) if s not in chosen]
    for name in LIVE:
        identical(end[name][others], start[name][others])
    if case.full and chosen:
        where = slice(None) if indices is None else indices
        identical(end["score_difference"][where], values["blue_score"] - values["orange_score"])
        identical(end["episode_ticks"][where], values["episode_ticks"])
        assert not bool(end["overtime"][where].any())
    for _ in range(8):
        envs.step(jump)
        envs.assert_equal(LIVE + STEP)


@pytest.mark.parametrize("team,mask", list(product((1, 2, 3), ((False, False, False), (True, False, True),
                                                             (True, True, True)))))
def test_masked_reset_equals_the_indexed_reset(gpu, team, mask):
    envs = Lockstep(3, team)
    values = fixtures.reset_inputs(3, 2 * team, device="cuda")
    rest = zero_actions(3, 2 * team)
    envs.set_no_touch_timeout(1)
    envs.step(rest)
    start = capture(envs.b, STEP)
    envs.set_no_touch_timeout(0)
    chosen = torch.tensor(mask, device="cuda")
    for round_ in range(3):
        chosen = torch.roll(chosen, 1)
        rows = chosen.nonzero().flatten()
        values["ball_position"][:, 0] = 100.0 * torch.arange(3, device="cuda") + round_
        envs.a.apply_reset_state(**{k: v[rows].contiguous() for k, v in values.items()}, simulation_indices=rows)
        envs.b.apply_reset_state(**values, reset_mask=chosen)
        envs.assert_equal(LIVE)
        now = capture(envs.b, STEP)
        for name in STEP:
            identical(now[name], start[name])
    for _ in range(8):
        envs.step(rest)
        envs.assert_equal(LIVE + STEP)


@pytest.mark.parametrize("masked", [False, True])
def test_restored_stack_gets_contacts_from_the_whole_scene(gpu, masked):
    """One car restored with its wheels on another's roof (z = 257 over
    z = 200), far above the arena: the top car is on the ground, the bottom
    one is not, neither touches the ball, and the restored positions and
    velocities are what the state reports; a demolished top car has no
    grounded contact."""
    env = carl.Env(1, 1, 1, 7, previous_controls=True)
    values = fixtures.reset_inputs(1, 2, device="cuda")
    values["car_position"][0] = torch.tensor([[0.0, 0.0, 257.0], [0.0, 0.0, 200.0]], device="cuda")
    values["car_demoed"].zero_()
    extra = {"reset_mask": torch.ones(1, device="cuda", dtype=torch.bool)} if masked else {}
    env.apply_reset_state(**values, **extra)
    rows = capture(env, ("state",))["state"]
    cars = rows[:, carl.OBS_BALL:carl.OBS_BALL + 2 * carl.STATE_PER_CAR].reshape(1, 2, carl.STATE_PER_CAR)
    identical(cars[..., 0:3], values["car_position"])
    identical(cars[..., 3:6], values["car_velocity"])
    assert [bool(cars[0, k, carl.OBS_ON_GROUND]) for k in range(2)] == [True, False]
    assert not bool(cars[..., carl.STATE_BALL_TOUCH].any())
    values["car_demoed"][:, 0] = True
    env.apply_reset_state(**values, **extra)
    obs = capture(env, ("obs",))["obs"]
    assert not bool(obs[0, 0, carl.OBS_BALL + carl.OBS_ON_GROUND])


def _malformed(values):
    """Named ways to break valid apply_reset_state inputs for two simulations."""
    ones_bool = lambda n: torch.ones(n, device="cuda", dtype=torch.bool)  # noqa: E731
    return {
        "episode_ticks without the other match fields": {"episode_ticks": None},
        "int64 episode ticks": {"episode_ticks": values["episode_ticks"].long()},
        "internal state of the wrong width": {"car_internal_state": torch.zeros((2, 2, 1), device="cuda")},
        "non-contiguous car positions": {"car_position": values["car_position"].transpose(0, 1)},
        "host ball velocity capsule": {"ball_velocity": torch.utils.dlpack.to_dlpack(values["ball_velocity"].cpu())},
        "float mask": {"reset_mask": torch.ones(2, device="cuda")},
        "mask of the wrong length": {"reset_mask": ones_bool(3)},
        "mask together with indices": {"reset_mask": ones_bool(2),
                                       "simulation_indices": torch.arange(2, device="cuda")},
        "mask with too few ball rows": {"reset_mask": ones_bool(2), "ball_position": values["ball_position"][:1]},
    }


def test_malformed_inputs_change_nothing(gpu):
    env = carl.Env(2, 1, 1, 7)
    untouched = capture(env, LIVE)
    good = fixtures.reset_inputs(2, 2, device="cuda")
    for what, change in _malformed(good).items():
        with pytest.raises((ValueError, TypeError)):
            env.apply_reset_state(**{**good, **change})
        after = capture(env, LIVE)
        changed = [name for name in LIVE if not torch.equal(after[name], untouched[name])]
        assert not changed, (what, changed)


# the restored clock: max_ticks 4, overtime limit 2, both simulations at tick
# 3, simulation 0 tied 2-2, simulation 1 leading 2-1; (steps so far, dones,
# overtime, transition episode ticks or None, transition overtime of
# simulation 0 or None)
CLOCK = [
    (1, (False, True), (True, False), (4, 4), None),
    (3, (True, False), (False, False), None, True),
]


def test_restored_match_clock_enters_overtime_or_truncates(gpu):
    env = carl.Env(2, 1, 1, 7)
    env.max_ticks, env.overtime_timeout_ticks = 4, 2
    values = fixtures.reset_inputs(2, 2, device="cuda")
    values["orange_score"][0] = 2
    values["episode_ticks"][:] = 3
    env.apply_reset_state(**values)
    rest, taken = zero_actions(2, 2), 0
    for steps, dones, overtime, ticks, t_over in CLOCK:
        while taken < steps:
            env.step_continuous(rest)
            taken += 1
        out = capture(env, LIVE + STEP)
        identical(out["dones"], torch.tensor(dones, device="cuda"))
        identical(out["overtime"], torch.tensor(overtime, device="cuda"))
        if ticks is not None:
            identical(out["transition_episode_ticks"], torch.tensor(ticks, device="cuda", dtype=torch.int32))
        if t_over is not None:
            assert bool(out["transition_overtime"][0]) is t_over


def _restore_from_side_stream(*, capsules=False, masked=False):
    """Four restores whose inputs are temporaries made on a side stream behind
    a slow kernel, freed (and their memory reused) right after the call."""
    env = carl.Env(3, 1, 1, 7)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        values = fixtures.reset_inputs(3 if masked else 2, 2, device="cuda")
        if masked:
            values["reset_mask"] = torch.tensor([True, False, True], device="cuda")
        else:
            values["simulation_indices"] = torch.tensor([2, 0], device="cuda")
        for k in range(4):
            torch.cuda._sleep(1_000_000)
            values["ball_position"][:, 0] = 100.0 * k
            temp = {name: t.clone() for name, t in values.items()}
            if capsules:
                torch.cuda.ExternalStream(env.stream).wait_stream(side)
                temp = {name: torch.utils.dlpack.to_dlpack(t) for name, t in temp.items()}
            env.apply_reset_state(**temp)
            del temp
            reuse = [torch.full_like(t, -999) for t in values.values()]
            del reuse
    torch.cuda.current_stream().wait_stream(side)
    return capture(env, LIVE)


def test_side_stream_temporaries_survive_until_read(gpu):
    want = _restore_from_side_stream()
    for capsules, masked in product((False, True), repeat=2):
        got = _restore_from_side_stream(capsules=capsules, masked=masked)
        for name in LIVE:
            identical(got[name], want[name])


def test_destroying_the_environment_waits_for_pending_masked_inputs(gpu):
    env = carl.Env(3, 1, 1, 7)
    engine = torch.cuda.ExternalStream(env.stream)
    with torch.cuda.stream(engine):
        torch.cuda._sleep(1_000_000)       # the engine stream is busy when the reset is queued
    done = torch.cuda.Event()
    env.apply_reset_state(**fixtures.reset_inputs(3, 2, device="cuda"),
                          reset_mask=torch.ones(3, device="cuda", dtype=torch.bool))
    done.record(engine)
    del env
    assert done.query()


# ------------------------------------------------------------------ the wrapper

def _wrapper(**extra):
    return CARLTorchVectorEnv(n_sim=2, n_blue=1, n_orange=1, frameskip=1, no_touch_timeout_ticks=1, **extra)


def _provider(mask, *, typed, masked):
    """Reset inputs for the eligible simulations of `mask`: fixed-shape with
    the mask itself, or compacted with their indices."""
    rows = None if masked else mask.nonzero().flatten()
    values = fixtures.reset_inputs(len(mask) if masked else len(rows), 2, device=mask.device)
    if typed:
        return typed_reset_state(values, rows, reset_mask=mask if masked else None)
    return {**values, **({"reset_mask": mask} if masked else {"simulation_indices": rows})}


def _same_step_results(got, want):
    for g, w in zip(got[1:4], want[1:4]):
        identical(g, w)
    assert got[4].keys() == want[4].keys()
    for key, w in want[4].items():
        if isinstance(w, torch.Tensor):
            identical(got[4][key], w)
        else:
            assert got[4][key] == w, key


@pytest.mark.parametrize("typed,goal,masked", list(product((False, True), repeat=3)))
def test_wrapper_keeps_terminal_successors(gpu, typed, goal, masked):
    """With a reset-state provider, an episode that ends (by a goal scored from
    a ball placed in the goal, else by the one-tick no-touch timeout) reports
    the same rewards, flags, final observations and transition rows as
    without it, and the next observation is the provider's scene (ball
    800 uu up)."""
    plain, provided = _wrapper(), _wrapper(masked_resets=masked)
    for env in (plain, provided):
        env.reset()
        if goal:
            spot = torch.tensor([[0.0, 5300.0, 100.0]] * 2, device="cuda")
            env.set_ball(spot, torch.zeros_like(spot), torch.zeros_like(spot))
    source = partial(_provider, typed=typed, masked=masked)
    provided.reset_state_provider = source
    rest = torch.zeros(plain.action_space.shape, device="cuda")
    for episode in range(2):
        want, got = plain.step(rest), provided.step(rest)
        _same_step_results(got, want)
        ended = got[2] if (goal and episode == 0) else got[3]
        assert bool(ended.all())
        rows_got, rows_want = capture(provided._env, STEP), capture(plain._env, STEP)
        for name in STEP:
            identical(rows_got[name], rows_want[name])
        assert bool((got[0].ball.position[:, 2] == 800.0).all())
        provided.reset_state_provider = None          # both back to kickoffs
        provided.reset()
        plain.reset()
        provided.reset_state_provider = source
    provided.close()
    plain.close()


@pytest.mark.parametrize("copy_outputs", [False, True])
def test_deferred_episode_reports_equal_the_immediate_ones(gpu, copy_outputs):
    """Every step ends both simulations' episodes (one-tick no-touch timeout).
    Deferred reporting returns the same step results without any host
    synchronisation, keeps the reports out of info, and hands over all of them
    (five steps of two) on the first drain only; a reset discards pending
    ones."""
    now, later = _wrapper(copy_outputs=copy_outputs), _wrapper(copy_outputs=copy_outputs,
                                                               defer_episode_reporting=True)
    now.reset()
    later.reset()
    rest = torch.zeros(later.action_space.shape, device="cuda")
    reported = {"reward": [], "length": []}
    for _ in range(5):
        want = now.step(rest)
        with NoHostSync():
            got = later.step(rest)
        for g, w in zip(got[:4], want[:4]):
            identical(g, w)
        identical(got[4]["final_obs"], want[4]["final_obs"])
        assert "reward" not in got[4]
        for key in reported:
            reported[key] += list(want[4][key])
    assert len(reported["reward"]) == 5 * later.n_envs
    assert later.drain_episode_reports() == reported
    assert later.drain_episode_reports() == {"reward": [], "length": []}
    later.step(rest)
    later.reset()
    assert later.drain_episode_reports() == {"reward": [], "length": []}
    later.close()
    now.close()
